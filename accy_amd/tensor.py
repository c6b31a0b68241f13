"""Recording tensor programs with named axes, and writing them as ACTP v1 wire bytes.

This is the host-side mirror of the reference tracer: ``define`` (src/tensor/trace/define.zig:8-19),
``Builder`` (src/tensor/trace/builder.zig:62-1047) and ``Value`` (src/tensor/trace/value.zig:13-193),
with the shape algebra of src/tensor/type/algebra.zig and the dims checks of
src/tensor/type/dim.zig. Every operation derives and checks its result type while recording, so
shape errors such as ``AxisExtentMismatch`` fire here, before anything runs (algebra.zig:14).

``Program.encode`` writes the version-1 wire layout of src/tensor/wire/format.zig and encode.zig;
the HIP target decodes those bytes and derives every type again.
"""
from __future__ import annotations

import math
import struct
from dataclasses import dataclass, field
from typing import Callable, Dict, List, Optional, Sequence, Tuple, Union

import numpy as np

# Wire codes: position in these lists (src/tensor/wire/format.zig:79-113).
DTYPES = ["i1", "i8", "i16", "i32", "i64", "u8", "u16", "u32", "u64", "f16", "bf16", "f32", "f64", "key"]
KINDS = ["parameter", "constant", "unary", "binary", "iota", "broadcast", "broadcast_in_dim", "reshape",
         "transpose", "reduce", "gather", "scatter_add", "sparse_cross_entropy", "dot_general", "compare",
         "select", "custom_call", "scan", "projection"]
UNARY = ["neg", "abs", "exp", "log", "sqrt", "tanh", "sin", "cos", "tan"]
BINARY = ["add", "sub", "mul", "div", "max", "min", "pow"]
REDUCERS = ["sum", "max", "min"]
COMPARE = ["lt", "le", "gt", "ge", "eq", "ne"]

MAGIC = struct.unpack("<I", b"ACTP")[0]
VERSION = 1
MAX_SCAN_DEPTH = 8
MAX_CUSTOM_CALL_OPERANDS = 4
MAX_SCAN_CARRIES = 8
GENERATED_PREFIX = "#"

DTYPE_SIZE = {"i1": 1, "i8": 1, "i16": 2, "i32": 4, "i64": 8, "u8": 1, "u16": 2, "u32": 4, "u64": 8,
              "f16": 2, "bf16": 2, "f32": 4, "f64": 8, "key": 8}
FLOAT_DTYPES = ("f16", "bf16", "f32", "f64")
SIGNED_DTYPES = ("i8", "i16", "i32", "i64")
UNSIGNED_DTYPES = ("u8", "u16", "u32", "u64")

# numpy storage type per dtype; bf16 is held as its raw 16 bits.
NUMPY_DTYPE = {"i1": np.bool_, "i8": np.int8, "i16": np.int16, "i32": np.int32, "i64": np.int64,
               "u8": np.uint8, "u16": np.uint16, "u32": np.uint32, "u64": np.uint64, "f16": np.float16,
               "bf16": np.uint16, "f32": np.float32, "f64": np.float64, "key": np.uint64}


class TensorError(Exception):
    """A recording or wire failure, named after the reference's error (e.g. ``AxisExtentMismatch``)."""

    def __init__(self, name: str, detail: str = ""):
        super().__init__(f"{name}: {detail}" if detail else name)
        self.name = name


Dim = Tuple[str, int]


@dataclass(frozen=True)
class Type:
    dtype: str
    dims: Tuple[Dim, ...] = ()

    @property
    def rank(self) -> int:
        return len(self.dims)

    @property
    def shape(self) -> Tuple[int, ...]:
        return tuple(e for _, e in self.dims)

    @property
    def names(self) -> Tuple[str, ...]:
        return tuple(n for n, _ in self.dims)

    def find(self, name: str) -> Optional[int]:
        for i, (n, _) in enumerate(self.dims):
            if n == name:
                return i
        return None

    def element_count(self) -> int:
        count = 1
        for _, e in self.dims:
            if e < 0:
                raise TensorError("InvalidDimension")
            count *= e
        if count >= 1 << 64:
            raise TensorError("ShapeElementOverflow")
        return count

    def byte_count(self) -> int:
        n = self.element_count() * DTYPE_SIZE[self.dtype]
        if n >= 1 << 64:
            raise TensorError("ShapeByteOverflow")
        return n


@dataclass(frozen=True)
class Spec:
    dtype: str
    dims: Tuple[Dim, ...]


def spec(dtype: str, *dims: Dim, **named: int) -> Spec:
    """``tensor.spec(.f32, .{ .guess = 8 })`` (dim.zig:88-95): ``spec("f32", guess=8)``.

    Axis order is the keyword order; ``spec("f32", ("a", 2), ("b", 3))`` is the positional form.
    """
    if dtype not in DTYPES:
        raise TensorError("UnknownTag", f"dtype {dtype}")
    return Spec(dtype, tuple(dims) + tuple(named.items()))


# ---- dims checks (dim.zig:213-241) ----

def _validate_name(name: str) -> None:
    if len(name) == 0:
        raise TensorError("AxisNameEmpty")


def _validate_dims(dims: Sequence[Dim]) -> None:
    for i, (name, extent) in enumerate(dims):
        _validate_name(name)
        if extent < 0:
            raise TensorError("InvalidDimension", name)
        for seen, _ in dims[:i]:
            if seen == name:
                raise TensorError("DuplicateAxis", name)


def _validate_authored_dims(dims: Sequence[Dim]) -> None:
    _validate_dims(dims)
    for name, _ in dims:
        if name[0] == GENERATED_PREFIX:
            raise TensorError("AxisNameReserved", name)


def _validate_axis_groups(rank: int, groups: Sequence[Sequence[int]]) -> None:
    # src/axis/roles.zig:21-41
    for gi, group in enumerate(groups):
        for ai, axis in enumerate(group):
            if axis < 0 or axis >= rank:
                raise TensorError("AxisOutOfRange")
            for prior in groups[:gi]:
                if axis in prior:
                    raise TensorError("DuplicateAxis")
            if axis in group[:ai]:
                raise TensorError("DuplicateAxis")


def _validate_axes(rank: int, axes: Sequence[int]) -> None:
    _validate_axis_groups(rank, [list(axes)])


def _make_type(dtype: str, dims: Sequence[Dim]) -> Type:
    _validate_dims(dims)
    return Type(dtype, tuple((str(n), int(e)) for n, e in dims))


def _find(dims: Sequence[Dim], name: str) -> Optional[int]:
    for i, (n, _) in enumerate(dims):
        if n == name:
            return i
    return None


def _same_type(a: Type, b: Type) -> None:
    if a.dtype != b.dtype:
        raise TensorError("DTypeMismatch", f"{a.dtype} vs {b.dtype}")
    if a.dims != b.dims:
        raise TensorError("ShapeMismatch", f"{a.dims} vs {b.dims}")


# ---- shape algebra (algebra.zig) ----

def union_dims(lhs: Sequence[Dim], rhs: Sequence[Dim]) -> Tuple[Dim, ...]:
    """algebra.zig:10-31: lhs axes in order, then the rhs axes lhs lacks."""
    out = list(lhs)
    for name, extent in rhs:
        i = _find(lhs, name)
        if i is not None:
            if lhs[i][1] != extent:
                raise TensorError("AxisExtentMismatch", name)
        else:
            out.append((name, extent))
    return tuple(out)


def alignment(operand: Sequence[Dim], target: Sequence[Dim]):
    """algebra.zig:42-77: (permutation or None, mapping or None) that aligns operand to target."""
    if tuple(operand) == tuple(target):
        return None, None
    positions = []
    for name, extent in operand:
        i = _find(target, name)
        if i is None:
            raise TensorError("AxisNotFound", name)
        if target[i][1] != extent:
            raise TensorError("AxisExtentMismatch", name)
        positions.append(i)
    if all(positions[i - 1] < positions[i] for i in range(1, len(positions))):
        return None, positions
    order = sorted(range(len(operand)), key=lambda i: positions[i])
    return order, [positions[i] for i in order]


def axis_indices(dims: Sequence[Dim], names: Sequence[str]) -> List[int]:
    """algebra.zig:83-97: indices of the named axes, sorted ascending."""
    if len(names) == 0:
        raise TensorError("AxisNotFound")
    out: List[int] = []
    for name in names:
        i = _find(dims, name)
        if i is None:
            raise TensorError("AxisNotFound", name)
        if i in out:
            raise TensorError("DuplicateAxis", name)
        out.append(i)
    return sorted(out)


def remove_axes(dims: Sequence[Dim], axes: Sequence[int]) -> Tuple[Dim, ...]:
    _validate_axes(len(dims), axes)
    return tuple(d for i, d in enumerate(dims) if i not in axes)


def _contraction(lhs: Sequence[Dim], rhs: Sequence[Dim], names: Sequence[str]):
    """algebra.zig:330-414."""
    if len(names) == 0:
        raise TensorError("AxisNotFound")
    lc, rc = [], []
    for name in names:
        li, ri = _find(lhs, name), _find(rhs, name)
        if li is None or ri is None:
            raise TensorError("AxisNotFound", name)
        if lhs[li][1] != rhs[ri][1]:
            raise TensorError("AxisExtentMismatch", name)
        if li in lc:
            raise TensorError("DuplicateAxis", name)
        lc.append(li)
        rc.append(ri)
    lb, rb = [], []
    for i, (name, extent) in enumerate(lhs):
        if i in lc:
            continue
        ri = _find(rhs, name)
        if ri is not None:
            if extent != rhs[ri][1]:
                raise TensorError("AxisExtentMismatch", name)
            lb.append(i)
            rb.append(ri)
    result = [lhs[i] for i in lb]
    result += [d for i, d in enumerate(lhs) if i not in lc and i not in lb]
    for i, d in enumerate(rhs):
        if i in rc or i in rb:
            continue
        if _find(result, d[0]) is not None:
            raise TensorError("DuplicateAxis", d[0])
        result.append(d)
    return lc, rc, lb, rb, tuple(result)


def _gather_type(inp: Type, idx: Type, axis: int) -> Type:
    if idx.dtype != "i32":
        raise TensorError("DTypeMismatch", "gather indices must be i32")
    _validate_axes(inp.rank, [axis])
    dims = inp.dims[:axis] + idx.dims + inp.dims[axis + 1:]
    return _make_type(inp.dtype, dims)


def _to_bytes(dtype: str, values) -> bytes:
    """Element encoding of constants: f16 rounds to nearest even (Zig ``@floatCast``), bf16 truncates
    an f32 (``Bf16.fromF32``, deps/lib/compiler/gpu/abi/src/dtype.zig:6-9)."""
    arr = np.asarray(values)
    if dtype == "bf16":
        f = np.asarray(arr, dtype=np.float64).astype(np.float32)
        return (f.view(np.uint32) >> 16).astype("<u2").tobytes()
    if dtype == "i1":
        return np.asarray(arr, dtype=np.bool_).astype(np.uint8).tobytes()
    if dtype == "key":
        return np.asarray(arr, dtype="<u8").tobytes()
    return np.asarray(arr, dtype=np.dtype(NUMPY_DTYPE[dtype]).newbyteorder("<")).tobytes()


@dataclass
class Operation:
    kind: str
    result: Type
    code: Optional[str] = None           # unary / binary / reducer / compare name
    args: Tuple[int, ...] = ()
    ints: Tuple[int, ...] = ()           # broadcast_dims / permutation / reduce dimensions / sizes
    dot: Optional[Tuple[Tuple[int, ...], ...]] = None  # lhs_contract, rhs_contract, lhs_batch, rhs_batch
    axis: int = 0                        # iota / gather / scatter / sparse CE axis; scan length
    index: int = 0                       # parameter / projection index; custom_call version
    payload: bytes = b""                 # constant payload / custom_call target
    body: Optional["Program"] = None     # scan body


@dataclass
class Program:
    """A recorded program (src/tensor/program.zig:221-282)."""
    name: str
    operations: List[Operation]
    parameters: List[int]
    outputs: List[int]

    def type_of(self, vid: int) -> Type:
        return self.operations[vid].result

    @property
    def values(self) -> List[Type]:
        return [op.result for op in self.operations]

    def input_types(self) -> List[Type]:
        return [self.type_of(i) for i in self.parameters]

    def output_types(self) -> List[Type]:
        return [self.type_of(i) for i in self.outputs]

    def encode(self) -> bytes:
        return encode(self)


class Value:
    """A recorded value (value.zig:13-193). Binary ops align named axes by union."""

    __slots__ = ("builder", "id", "ty")

    def __init__(self, builder: "Builder", vid: int, ty: Type):
        self.builder = builder
        self.id = vid
        self.ty = ty

    def __repr__(self) -> str:
        return f"Value(%{self.id}: {self.ty.dtype}{list(self.ty.dims)})"

    # elementwise
    def add(self, rhs: "Value") -> "Value":
        return self.builder.aligned_binary("add", self, rhs)

    def sub(self, rhs: "Value") -> "Value":
        return self.builder.aligned_binary("sub", self, rhs)

    def mul(self, rhs: "Value") -> "Value":
        return self.builder.aligned_binary("mul", self, rhs)

    def div(self, rhs: "Value") -> "Value":
        return self.builder.aligned_binary("div", self, rhs)

    def pow(self, rhs: "Value") -> "Value":
        return self.builder.aligned_binary("pow", self, rhs)

    def max(self, other) -> "Value":
        if isinstance(other, Value):
            return self.builder.aligned_binary("max", self, other)
        return self.builder.reduce_named(self, "max", _axes(other))

    def min(self, other) -> "Value":
        if isinstance(other, Value):
            return self.builder.aligned_binary("min", self, other)
        return self.builder.reduce_named(self, "min", _axes(other))

    def sum(self, axes) -> "Value":
        return self.builder.reduce_named(self, "sum", _axes(axes))

    def mean(self, axes) -> "Value":
        return self.builder.mean_named(self, _axes(axes))

    def reduce(self, init: "Value", reducer: str, axes) -> "Value":
        return self.builder.reduce_with(self, init, reducer, _axes(axes))

    def gather(self, indices: "Value", axis: str) -> "Value":
        return self.builder.gather_named(self, indices, axis)

    def scatter_add(self, indices: "Value", updates: "Value", axis: str) -> "Value":
        return self.builder.scatter_add_named(self, indices, updates, axis)

    def sparse_cross_entropy_loss(self, targets: "Value", axis: str) -> "Value":
        return self.builder.sparse_cross_entropy_named(self, targets, axis)

    def contract(self, rhs: "Value", axes) -> "Value":
        return self.builder.contract(self, rhs, _axes(axes))

    def rename(self, old: str, new: str) -> "Value":
        return self.builder.rename_axis(self, old, new)

    def split(self, axis: str, *parts: Dim, **named: int) -> "Value":
        return self.builder.split_axis(self, axis, tuple(parts) + tuple(named.items()))

    def merge(self, axes, merged: str) -> "Value":
        return self.builder.merge_axes(self, _axes(axes), merged)

    def broadcast(self, *added: Dim, **named: int) -> "Value":
        return self.builder.broadcast_axes(self, tuple(added) + tuple(named.items()))

    def neg(self) -> "Value":
        return self.builder.unary("neg", self)

    def abs(self) -> "Value":
        return self.builder.unary("abs", self)

    def exp(self) -> "Value":
        return self.builder.unary("exp", self)

    def log(self) -> "Value":
        return self.builder.unary("log", self)

    def sqrt(self) -> "Value":
        return self.builder.unary("sqrt", self)

    def tanh(self) -> "Value":
        return self.builder.unary("tanh", self)

    def sin(self) -> "Value":
        return self.builder.unary("sin", self)

    def cos(self) -> "Value":
        return self.builder.unary("cos", self)

    def tan(self) -> "Value":
        return self.builder.unary("tan", self)

    def compare(self, direction: str, rhs: "Value") -> "Value":
        return self.builder.aligned_compare(direction, self, rhs)

    def select(self, on_true: "Value", on_false: "Value") -> "Value":
        return self.builder.aligned_select(self, on_true, on_false)

    def is_structural_zero(self) -> bool:
        return self.builder.is_structural_zero(self.id)


def _axes(axes) -> List[str]:
    if isinstance(axes, str):
        return [axes]
    return list(axes)


class Builder:
    """Appends checked operations (builder.zig:62-1047)."""

    def __init__(self, name: str):
        self.name = name
        self.operations: List[Operation] = []
        self.parameters: List[int] = []
        self.finished = False

    # -- internals --
    def _append(self, op: Operation) -> Value:
        if self.finished:
            raise TensorError("BuilderFinished")
        self.operations.append(op)
        vid = len(self.operations) - 1
        return Value(self, vid, op.result)

    def _ensure(self, v: Value) -> None:
        if self.finished:
            raise TensorError("BuilderFinished")
        if v.builder is not self:
            raise TensorError("CrossBuilderValue")

    def value(self, vid: int) -> Value:
        return Value(self, vid, self.operations[vid].result)

    # -- inputs and constants --
    def input(self, dtype: str, *dims: Dim, **named: int) -> Value:
        return self.input_dims(dtype, tuple(dims) + tuple(named.items()))

    def input_dims(self, dtype: str, dims: Sequence[Dim]) -> Value:
        _validate_authored_dims(dims)
        return self.input_typed(Type(dtype, tuple(dims)))

    def input_spec(self, s: Spec) -> Value:
        return self.input_dims(s.dtype, s.dims)

    def inputs(self, specs: Sequence[Spec]) -> List[Value]:
        return [self.input_spec(s) for s in specs]

    def input_typed(self, ty: Type) -> Value:
        ty = _make_type(ty.dtype, ty.dims)
        v = self._append(Operation("parameter", ty, index=len(self.parameters)))
        self.parameters.append(v.id)
        return v

    def constant_bytes(self, ty: Type, payload: bytes) -> Value:
        ty = _make_type(ty.dtype, ty.dims)
        if len(payload) != ty.byte_count():
            raise TensorError("PayloadLengthMismatch")
        return self._append(Operation("constant", ty, payload=bytes(payload)))

    def scalar(self, dtype: str, value) -> Value:
        return self.constant_bytes(Type(dtype, ()), _to_bytes(dtype, [value]))

    def full(self, dtype: str, value, *dims: Dim, **named: int) -> Value:
        dims = tuple(dims) + tuple(named.items())
        _validate_authored_dims(dims)
        ty = _make_type(dtype, dims)
        return self.constant_bytes(ty, _to_bytes(dtype, np.full(ty.element_count(), value)))

    def full_float(self, ty: Type, value: float) -> Value:
        """builder.zig:215-249: f16 rounds, bf16 truncates an f32, other dtypes are refused."""
        if ty.dtype not in FLOAT_DTYPES:
            raise TensorError("NonFloatDType")
        ty = _make_type(ty.dtype, ty.dims)
        return self.constant_bytes(ty, _to_bytes(ty.dtype, np.full(ty.element_count(), value, dtype=np.float64)))

    def zeros(self, ty: Type) -> Value:
        ty = _make_type(ty.dtype, ty.dims)
        return self.constant_bytes(ty, bytes(ty.byte_count()))

    def iota(self, dtype: str, axis: str, *dims: Dim, **named: int) -> Value:
        dims = tuple(dims) + tuple(named.items())
        _validate_authored_dims(dims)
        i = _find(dims, axis)
        if i is None:
            raise TensorError("AxisNotFound", axis)
        return self.iota_typed(Type(dtype, dims), i)

    def iota_typed(self, ty: Type, axis: int) -> Value:
        _validate_axes(ty.rank, [axis])
        return self._append(Operation("iota", _make_type(ty.dtype, ty.dims), axis=axis))

    def is_structural_zero(self, vid: int) -> bool:
        """builder.zig:274-303."""
        if vid >= len(self.operations):
            return False
        op = self.operations[vid]
        k = op.kind
        if k == "constant":
            return not any(op.payload)
        if k == "unary":
            return op.code == "neg" and self.is_structural_zero(op.args[0])
        if k == "binary":
            if op.code in ("add", "sub"):
                return self.is_structural_zero(op.args[0]) and self.is_structural_zero(op.args[1])
            if op.code == "mul":
                return self.is_structural_zero(op.args[0]) or self.is_structural_zero(op.args[1])
            return False
        if k in ("broadcast", "broadcast_in_dim", "reshape", "transpose", "gather"):
            return self.is_structural_zero(op.args[0])
        if k == "scatter_add":
            return self.is_structural_zero(op.args[0]) and self.is_structural_zero(op.args[2])
        if k == "select":
            return self.is_structural_zero(op.args[1]) and self.is_structural_zero(op.args[2])
        return False

    # -- elementwise --
    def unary(self, op: str, a: Value) -> Value:
        self._ensure(a)
        if op not in UNARY:
            raise TensorError("UnknownTag", op)
        return self._append(Operation("unary", a.ty, code=op, args=(a.id,)))

    def binary(self, op: str, lhs: Value, rhs: Value) -> Value:
        self._ensure(lhs)
        self._ensure(rhs)
        if op not in BINARY:
            raise TensorError("UnknownTag", op)
        _same_type(lhs.ty, rhs.ty)
        return self._append(Operation("binary", lhs.ty, code=op, args=(lhs.id, rhs.id)))

    def aligned_binary(self, op: str, lhs: Value, rhs: Value) -> Value:
        self._ensure(lhs)
        self._ensure(rhs)
        if lhs.ty.dtype != rhs.ty.dtype:
            raise TensorError("DTypeMismatch", f"{lhs.ty.dtype} vs {rhs.ty.dtype}")
        target = union_dims(lhs.ty.dims, rhs.ty.dims)
        return self.binary(op, self.align_to(lhs, target), self.align_to(rhs, target))

    def compare(self, direction: str, lhs: Value, rhs: Value) -> Value:
        self._ensure(lhs)
        self._ensure(rhs)
        if direction not in COMPARE:
            raise TensorError("UnknownTag", direction)
        _same_type(lhs.ty, rhs.ty)
        return self._append(Operation("compare", Type("i1", lhs.ty.dims), code=direction, args=(lhs.id, rhs.id)))

    def aligned_compare(self, direction: str, lhs: Value, rhs: Value) -> Value:
        self._ensure(lhs)
        self._ensure(rhs)
        if lhs.ty.dtype != rhs.ty.dtype:
            raise TensorError("DTypeMismatch")
        target = union_dims(lhs.ty.dims, rhs.ty.dims)
        return self.compare(direction, self.align_to(lhs, target), self.align_to(rhs, target))

    def select(self, pred: Value, on_true: Value, on_false: Value) -> Value:
        for v in (pred, on_true, on_false):
            self._ensure(v)
        if pred.ty.dtype != "i1":
            raise TensorError("DTypeMismatch", "select predicate must be i1")
        if on_true.ty.dtype != on_false.ty.dtype:
            raise TensorError("DTypeMismatch")
        if on_true.ty.dims != on_false.ty.dims:
            raise TensorError("ShapeMismatch")
        if pred.ty.rank != 0 and pred.ty.dims != on_true.ty.dims:
            raise TensorError("ShapeMismatch")
        return self._append(Operation("select", on_true.ty, args=(pred.id, on_true.id, on_false.id)))

    def aligned_select(self, pred: Value, on_true: Value, on_false: Value) -> Value:
        for v in (pred, on_true, on_false):
            self._ensure(v)
        if on_true.ty.dtype != on_false.ty.dtype:
            raise TensorError("DTypeMismatch")
        target = union_dims(on_true.ty.dims, on_false.ty.dims)
        if pred.ty.rank != 0:
            target = union_dims(target, pred.ty.dims)
        t = self.align_to(on_true, target)
        f = self.align_to(on_false, target)
        p = pred if pred.ty.rank == 0 else self.align_to(pred, target)
        return self.select(p, t, f)

    # -- shape --
    def align_to(self, v: Value, target: Sequence[Dim]) -> Value:
        """builder.zig:476-485."""
        target = tuple(target)
        if v.ty.dims == target:
            return v
        perm, mapping = alignment(v.ty.dims, target)
        cur = v
        if perm is not None:
            cur = self.transpose(cur, perm)
        if cur.ty.dims == target:
            return cur
        return self.broadcast_in_dim(cur, target, mapping)

    def broadcast_axes(self, v: Value, added: Sequence[Dim]) -> Value:
        self._ensure(v)
        _validate_authored_dims(added)
        for name, _ in added:
            if _find(v.ty.dims, name) is not None:
                raise TensorError("DuplicateAxis", name)
        return self.align_to(v, v.ty.dims + tuple(added))

    def broadcast(self, v: Value, dims: Sequence[Dim]) -> Value:
        self._ensure(v)
        ty = _make_type(v.ty.dtype, dims)
        return self._append(Operation("broadcast", ty, args=(v.id,), ints=ty.shape))

    def broadcast_in_dim(self, v: Value, dims: Sequence[Dim], bdims: Sequence[int]) -> Value:
        self._ensure(v)
        dims = tuple(dims)
        if len(bdims) != v.ty.rank:
            raise TensorError("BroadcastRankMismatch")
        _validate_axes(len(dims), bdims)
        for i, axis in enumerate(bdims):
            if v.ty.dims[i][1] != 1 and v.ty.dims[i][1] != dims[axis][1]:
                raise TensorError("BroadcastDimensionMismatch")
        ty = _make_type(v.ty.dtype, dims)
        return self._append(Operation("broadcast_in_dim", ty, args=(v.id,), ints=tuple(bdims)))

    def reshape(self, v: Value, dims: Sequence[Dim]) -> Value:
        self._ensure(v)
        ty = _make_type(v.ty.dtype, dims)
        if v.ty.element_count() != ty.element_count():
            raise TensorError("ReshapeElementMismatch")
        return self._append(Operation("reshape", ty, args=(v.id,), ints=ty.shape))

    def transpose(self, v: Value, perm: Sequence[int]) -> Value:
        self._ensure(v)
        if len(perm) != v.ty.rank:
            raise TensorError("RankMismatch")
        _validate_axes(v.ty.rank, perm)
        ty = _make_type(v.ty.dtype, tuple(v.ty.dims[p] for p in perm))
        return self._append(Operation("transpose", ty, args=(v.id,), ints=tuple(perm)))

    def rename_axis(self, v: Value, old: str, new: str) -> Value:
        self._ensure(v)
        _validate_name(new)
        if new[0] == GENERATED_PREFIX:
            raise TensorError("AxisNameReserved", new)
        i = _find(v.ty.dims, old)
        if i is None:
            raise TensorError("AxisNotFound", old)
        if _find(v.ty.dims, new) is not None:
            raise TensorError("DuplicateAxis", new)
        dims = list(v.ty.dims)
        dims[i] = (new, dims[i][1])
        return self.reshape(v, dims)

    def split_axis(self, v: Value, axis: str, parts: Sequence[Dim]) -> Value:
        """algebra.zig:190-234."""
        self._ensure(v)
        _validate_authored_dims(parts)
        i = _find(v.ty.dims, axis)
        if i is None:
            raise TensorError("AxisNotFound", axis)
        product = 1
        for name, extent in parts:
            if extent < 0:
                raise TensorError("InvalidDimension")
            product *= extent
        if product != v.ty.dims[i][1]:
            raise TensorError("SplitExtentMismatch")
        for name, _ in parts:
            j = _find(v.ty.dims, name)
            if j is not None and j != i:
                raise TensorError("DuplicateAxis", name)
        dims = v.ty.dims[:i] + tuple(parts) + v.ty.dims[i + 1:]
        return self.reshape(v, dims)

    def merge_axes(self, v: Value, names: Sequence[str], merged: str) -> Value:
        """algebra.zig:241-309: move the merged axes together at the first one's position, then reshape."""
        self._ensure(v)
        _validate_name(merged)
        if merged[0] == GENERATED_PREFIX:
            raise TensorError("AxisNameReserved", merged)
        dims = v.ty.dims
        if len(names) == 0:
            raise TensorError("AxisNotFound")
        idx: List[int] = []
        extent = 1
        for name in names:
            i = _find(dims, name)
            if i is None:
                raise TensorError("AxisNotFound", name)
            if i in idx:
                raise TensorError("DuplicateAxis", name)
            idx.append(i)
            extent *= dims[i][1]
        start = min(idx)
        existing = _find(dims, merged)
        if existing is not None and existing not in idx:
            raise TensorError("DuplicateAxis", merged)
        perm: List[int] = []
        result: List[Dim] = []
        for i in range(len(dims)):
            if i == start:
                perm.extend(idx)
                result.append((merged, extent))
            if i not in idx:
                perm.append(i)
                result.append(dims[i])
        cur = v
        if perm != list(range(len(dims))):
            cur = self.transpose(cur, perm)
        return self.reshape(cur, result)

    # -- reductions --
    def reduce(self, v: Value, init: Value, reducer: str, dims: Sequence[int]) -> Value:
        self._ensure(v)
        self._ensure(init)
        if reducer not in REDUCERS:
            raise TensorError("UnknownTag", reducer)
        if v.ty.dtype != init.ty.dtype:
            raise TensorError("DTypeMismatch")
        if init.ty.rank != 0:
            raise TensorError("ReduceInitNotScalar")
        result = remove_axes(v.ty.dims, dims)
        ty = _make_type(v.ty.dtype, result)
        return self._append(Operation("reduce", ty, code=reducer, args=(v.id, init.id), ints=tuple(dims)))

    def reducer_init(self, dtype: str, reducer: str) -> Value:
        """builder.zig:760-797."""
        ty = Type(dtype, ())
        if reducer == "sum":
            return self.zeros(ty)
        lowest = reducer == "max"
        if dtype in ("f16", "f32", "f64", "bf16"):
            return self.constant_bytes(ty, _to_bytes(dtype, [-math.inf if lowest else math.inf]))
        if dtype in ("i32", "i64"):
            bits = 32 if dtype == "i32" else 64
            v = -(1 << (bits - 1)) if lowest else (1 << (bits - 1)) - 1
            return self.constant_bytes(ty, _to_bytes(dtype, [v]))
        raise TensorError("DTypeMismatch")

    def reduce_named(self, v: Value, reducer: str, names: Sequence[str]) -> Value:
        self._ensure(v)
        idx = axis_indices(v.ty.dims, names)
        init = self.reducer_init(v.ty.dtype, reducer)
        return self.reduce(v, init, reducer, idx)

    def reduce_with(self, v: Value, init: Value, reducer: str, names: Sequence[str]) -> Value:
        self._ensure(v)
        idx = axis_indices(v.ty.dims, names)
        return self.reduce(v, init, reducer, idx)

    def mean_named(self, v: Value, names: Sequence[str]) -> Value:
        """builder.zig:743-758: sum, then divide by the reduced element count."""
        self._ensure(v)
        idx = axis_indices(v.ty.dims, names)
        count = 1
        for i in idx:
            count *= v.ty.dims[i][1]
        init = self.reducer_init(v.ty.dtype, "sum")
        summed = self.reduce(v, init, "sum", idx)
        divisor = self.full_float(Type(v.ty.dtype, ()), float(count))
        return self.aligned_binary("div", summed, divisor)

    # -- indexing --
    def gather_named(self, v: Value, indices: Value, axis: str) -> Value:
        self._ensure(v)
        i = _find(v.ty.dims, axis)
        if i is None:
            raise TensorError("AxisNotFound", axis)
        return self.gather(v, indices, i)

    def gather(self, v: Value, indices: Value, axis: int) -> Value:
        self._ensure(v)
        self._ensure(indices)
        ty = _gather_type(v.ty, indices.ty, axis)
        return self._append(Operation("gather", ty, args=(v.id, indices.id), axis=axis))

    def scatter_add_named(self, v: Value, indices: Value, updates: Value, axis: str) -> Value:
        self._ensure(v)
        i = _find(v.ty.dims, axis)
        if i is None:
            raise TensorError("AxisNotFound", axis)
        return self.scatter_add(v, indices, updates, i)

    def scatter_add(self, v: Value, indices: Value, updates: Value, axis: int) -> Value:
        for x in (v, indices, updates):
            self._ensure(x)
        if v.ty.dtype not in FLOAT_DTYPES + SIGNED_DTYPES + UNSIGNED_DTYPES:
            raise TensorError("DTypeMismatch")
        if updates.ty.dtype != v.ty.dtype:
            raise TensorError("DTypeMismatch")
        expected = _gather_type(v.ty, indices.ty, axis)
        if updates.ty.dims != expected.dims:
            raise TensorError("ShapeMismatch")
        return self._append(Operation("scatter_add", v.ty, args=(v.id, indices.id, updates.id), axis=axis))

    def sparse_cross_entropy_named(self, logits: Value, targets: Value, axis: str) -> Value:
        self._ensure(logits)
        i = _find(logits.ty.dims, axis)
        if i is None:
            raise TensorError("AxisNotFound", axis)
        return self.sparse_cross_entropy(logits, targets, i)

    def sparse_cross_entropy(self, logits: Value, targets: Value, axis: int) -> Value:
        self._ensure(logits)
        self._ensure(targets)
        if logits.ty.dtype not in FLOAT_DTYPES:
            raise TensorError("DTypeMismatch")
        if targets.ty.dtype != "i32":
            raise TensorError("DTypeMismatch")
        _validate_axes(logits.ty.rank, [axis])
        expected = remove_axes(logits.ty.dims, [axis])
        if targets.ty.dims != expected:
            raise TensorError("ShapeMismatch")
        ty = _make_type(logits.ty.dtype, targets.ty.dims)
        return self._append(Operation("sparse_cross_entropy", ty, args=(logits.id, targets.id), axis=axis))

    # -- contraction --
    def contract(self, lhs: Value, rhs: Value, names: Sequence[str]) -> Value:
        """builder.zig:799-865: canonicalise to [batch, free, contract] x [batch, contract, free]."""
        self._ensure(lhs)
        self._ensure(rhs)
        if lhs.ty.dtype != rhs.ty.dtype:
            raise TensorError("ContractDTypeMismatch")
        lc, rc, lb, rb, result = _contraction(lhs.ty.dims, rhs.ty.dims, names)
        ld, rd = lhs.ty.dims, rhs.ty.dims
        lhs_order = [ld[a] for a in lb] + [d for i, d in enumerate(ld) if i not in lb and i not in lc] + [ld[a] for a in lc]
        rhs_order = [rd[a] for a in rb] + [rd[a] for a in rc] + [d for i, d in enumerate(rd) if i not in rb and i not in rc]
        lcan = self.align_to(lhs, lhs_order)
        rcan = self.align_to(rhs, rhs_order)
        nb, nc = len(lb), len(lc)
        lfree = len(ld) - nb - nc
        dot = (tuple(nb + lfree + i for i in range(nc)), tuple(nb + i for i in range(nc)),
               tuple(range(nb)), tuple(range(nb)))
        ty = _make_type(lhs.ty.dtype, result)
        return self._append(Operation("dot_general", ty, args=(lcan.id, rcan.id), dot=dot))

    def dot_general(self, lhs: Value, rhs: Value, lc: Sequence[int], rc: Sequence[int],
                    lb: Sequence[int], rb: Sequence[int]) -> Value:
        """algebra.zig:416-480."""
        self._ensure(lhs)
        self._ensure(rhs)
        if lhs.ty.dtype != rhs.ty.dtype:
            raise TensorError("ContractDTypeMismatch")
        L, R = lhs.ty.dims, rhs.ty.dims
        for rank, group in ((len(L), lc), (len(R), rc), (len(L), lb), (len(R), rb)):
            _validate_axes(rank, group)
        if set(lc) & set(lb) or set(rc) & set(rb):
            raise TensorError("DuplicateAxis")
        if len(lc) != len(rc) or len(lb) != len(rb):
            raise TensorError("RankMismatch")
        for a, b in list(zip(lc, rc)) + list(zip(lb, rb)):
            if L[a][1] != R[b][1]:
                raise TensorError("AxisExtentMismatch")
        dims = [L[a] for a in lb] + [d for i, d in enumerate(L) if i not in lc and i not in lb]
        dims += [d for i, d in enumerate(R) if i not in rc and i not in rb]
        names = [n for n, _ in dims]
        if len(set(names)) != len(names):
            raise TensorError("DuplicateAxis")
        ty = _make_type(lhs.ty.dtype, dims)
        return self._append(Operation("dot_general", ty, args=(lhs.id, rhs.id),
                                       dot=(tuple(lc), tuple(rc), tuple(lb), tuple(rb))))

    # -- misc --
    def custom_call(self, target: str, version: int, operands: Sequence[Value], result: Type) -> Value:
        if len(target) == 0 or version == 0:
            raise TensorError("InvalidCustomCallContract")
        if len(operands) > MAX_CUSTOM_CALL_OPERANDS:
            raise TensorError("UnsupportedCustomCallArity")
        for v in operands:
            self._ensure(v)
        ty = _make_type(result.dtype, result.dims)
        return self._append(Operation("custom_call", ty, args=tuple(v.id for v in operands), index=version,
                                      payload=target.encode()))

    def scan(self, length: int, inits: Sequence[Value], body: Callable[["Builder", List[Value]], Sequence[Value]]) -> Value:
        """Repeat ``body`` ``length`` times carrying ``inits`` (builder.zig:899-990)."""
        if length < 0:
            raise TensorError("ScanLengthNegative")
        if len(inits) == 0:
            raise TensorError("ScanWithoutCarries")
        if len(inits) > MAX_SCAN_CARRIES:
            raise TensorError("ScanArityUnsupported")
        for v in inits:
            self._ensure(v)
        child = Builder("scan_body")
        carries = [child.input_typed(v.ty) for v in inits]
        nxt = list(body(child, carries))
        if len(nxt) != len(inits):
            raise TensorError("ScanArityMismatch")
        sub = child.finish(nxt)
        for i, v in enumerate(inits):
            _same_type(v.ty, sub.type_of(sub.parameters[i]))
            _same_type(v.ty, sub.type_of(sub.outputs[i]))
        return self._append(Operation("scan", inits[0].ty, args=tuple(v.id for v in inits), axis=length, body=sub))

    def projection(self, source: Value, index: int) -> Value:
        self._ensure(source)
        op = self.operations[source.id]
        if op.kind != "scan":
            raise TensorError("ProjectionSourceNotScan")
        if index == 0 or index >= len(op.args):
            raise TensorError("ProjectionIndexInvalid")
        ty = op.body.type_of(op.body.outputs[index])
        return self._append(Operation("projection", ty, args=(source.id,), index=index))

    def finish(self, outputs: Sequence[Value]) -> Program:
        if self.finished:
            raise TensorError("BuilderFinished")
        for v in outputs:
            self._ensure(v)
        self.finished = True
        return Program(self.name, self.operations, self.parameters, [v.id for v in outputs])


def define(name: str, specs: Sequence[Spec], body: Callable[[Builder, List[Value]], Union[Value, Sequence[Value]]]) -> Program:
    """``tensor.define`` (define.zig:8-19): run ``body`` on placeholders and record what it does."""
    b = Builder(name)
    args = b.inputs(specs)
    out = body(b, args)
    if isinstance(out, Value):
        out = [out]
    return b.finish(list(out))


# ---- wire encoding (encode.zig:28-230) ----

class _Sink:
    def __init__(self):
        self.parts: List[bytes] = []

    def word(self, v: int) -> None:
        self.parts.append(struct.pack("<I", v))

    def integer(self, v: int) -> None:
        self.parts.append(struct.pack("<q", v))

    def count(self, n: int) -> None:
        if n > 0xFFFFFFFF:
            raise TensorError("InvalidArtifact")
        self.word(n)

    def bytes_(self, b: bytes) -> None:
        self.count(len(b))
        self.parts.append(bytes(b))

    def ids(self, ids: Sequence[int]) -> None:
        for i in ids:
            self.word(i)

    def id_list(self, ids: Sequence[int]) -> None:
        self.count(len(ids))
        self.ids(ids)

    def integers(self, vals: Sequence[int]) -> None:
        self.count(len(vals))
        for v in vals:
            self.integer(v)

    def dims(self, dims: Sequence[Dim]) -> None:
        self.count(len(dims))
        for name, extent in dims:
            self.bytes_(name.encode())
            self.integer(extent)

    def typed(self, ty: Type) -> None:
        self.word(DTYPES.index(ty.dtype))
        self.dims(ty.dims)

    def graph(self, prog: Program, depth: int) -> None:
        pc = 0
        for i, op in enumerate(prog.operations):
            if op.kind != "parameter":
                continue
            if op.index != pc or pc == len(prog.parameters) or prog.parameters[pc] != i:
                raise TensorError("InvalidProgram")
            pc += 1
        if pc != len(prog.parameters):
            raise TensorError("InvalidProgram")
        self.count(len(prog.operations))
        for op in prog.operations:
            self.operation(op)
            if op.kind == "scan":
                if depth + 1 > MAX_SCAN_DEPTH:
                    raise TensorError("ScanTooDeep")
                self.graph(op.body, depth + 1)
        self.id_list(prog.outputs)

    def operation(self, op: Operation) -> None:
        self.word(KINDS.index(op.kind))
        k = op.kind
        if k == "parameter":
            self.typed(op.result)
        elif k == "constant":
            self.typed(op.result)
            self.bytes_(op.payload)
        elif k == "iota":
            self.typed(op.result)
            self.integer(op.axis)
        elif k == "custom_call":
            self.typed(op.result)
            self.bytes_(op.payload)
            self.word(op.index)
            self.id_list(op.args)
        elif k in ("broadcast", "reshape"):
            self.dims(op.result.dims)
            self.word(op.args[0])
        elif k == "broadcast_in_dim":
            self.dims(op.result.dims)
            self.word(op.args[0])
            self.integers(op.ints)
        elif k == "scan":
            self.integer(op.axis)
            self.id_list(op.args)
        elif k == "unary":
            self.word(UNARY.index(op.code))
            self.ids(op.args)
        elif k == "binary":
            self.word(BINARY.index(op.code))
            self.ids(op.args)
        elif k == "compare":
            self.word(COMPARE.index(op.code))
            self.ids(op.args)
        elif k == "select":
            self.ids(op.args)
        elif k == "projection":
            self.word(op.args[0])
            self.count(op.index)
        elif k == "transpose":
            self.word(op.args[0])
            self.integers(op.ints)
        elif k == "reduce":
            self.ids(op.args)
            self.word(REDUCERS.index(op.code))
            self.integers(op.ints)
        elif k in ("gather", "scatter_add", "sparse_cross_entropy"):
            self.ids(op.args)
            self.integer(op.axis)
        elif k == "dot_general":
            self.ids(op.args)
            for group in op.dot:
                self.integers(group)
        else:
            raise TensorError("UnknownTag", k)


def encode(prog: Program) -> bytes:
    s = _Sink()
    s.word(MAGIC)
    s.word(VERSION)
    s.bytes_(prog.name.encode())
    s.graph(prog, 0)
    return b"".join(s.parts)
