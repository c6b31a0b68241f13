"""Python face of the gfx950 execution target, over the C ABI in include/accy_hip.h.

Mirrors the reference's execution API for the runCpu path:

* ``run_hip(program, inputs, outputs)``  — ``tensor.runCpu`` (src/tensor/execute.zig:54-63);
* ``Hip(program)`` with ``launch`` / ``deinit`` — the ``Cpu`` executor (execute.zig:9-52);
* ``Session`` with ``compile`` / ``input_descriptors`` / ``output_descriptors`` / ``invoke`` /
  ``release`` — src/tensor/session/session.zig:99-246, with the same status numbers.

``program`` is a recorded ``accy_amd.tensor.Program`` or its ACTP v1 wire bytes. Inputs are
bytes-like objects or numpy arrays (their raw bytes are used); outputs are writable buffers
(numpy arrays or bytearrays), each exactly its slot's size. ``launch_device`` takes device pointers
(e.g. ``torch.Tensor.data_ptr()``) and a HIP stream handle, for data already resident in HBM.

The library is built in-tree by ``accy_amd.build``; loading fails loudly if it is missing — there is
no CPU fallback in the product.
"""
from __future__ import annotations

import ctypes
import threading
from dataclasses import dataclass
from pathlib import Path
from typing import List, Optional, Sequence, Tuple, Union

import numpy as np

from . import tensor as _tensor

_LIB_PATH = Path(__file__).resolve().parent / "_build" / "libaccy_hip.so"

# Status numbers (session.zig:33-43).
OK, INVALID_PROGRAM, UNSUPPORTED_VERSION, INVALID_HANDLE, INVALID_BUFFER = 0, 1, 2, 3, 4
TOO_MANY_PROGRAMS, OUT_OF_MEMORY, COMPILE_FAILED, LAUNCH_FAILED = 5, 6, 7, 8
STATUS_NAMES = {0: "ok", 1: "invalid_program", 2: "unsupported_version", 3: "invalid_handle",
                4: "invalid_buffer", 5: "too_many_programs", 6: "out_of_memory", 7: "compile_failed",
                8: "launch_failed"}
MAX_PROGRAMS = 64


class HipError(RuntimeError):
    """A non-zero status from the C ABI; ``status`` is the session status number."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")
        self.status = status
        self.message = message


class Handle(ctypes.Structure):
    _fields_ = [("index", ctypes.c_uint32), ("generation", ctypes.c_uint32)]


class _Descriptor(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_uint32), ("rank", ctypes.c_uint32),
                ("names", ctypes.POINTER(ctypes.c_char_p)), ("extents", ctypes.POINTER(ctypes.c_int64)),
                ("byte_size", ctypes.c_uint64), ("alignment", ctypes.c_uint32)]


class _KernelStats(ctypes.Structure):
    _fields_ = [("label", ctypes.c_char_p), ("klass", ctypes.c_char_p), ("algorithmic_bytes", ctypes.c_double),
                ("algorithmic_flops", ctypes.c_double), ("last_ms", ctypes.c_float), ("mean_ms", ctypes.c_float),
                ("calls", ctypes.c_uint32)]


@dataclass(frozen=True)
class Descriptor:
    """session.zig:66-74: element type, named axes, byte length and alignment of one buffer."""
    dtype: str
    dims: Tuple[Tuple[str, int], ...]
    byte_size: int
    alignment: int


@dataclass
class KernelStats:
    """One kernel: algorithmic work, and (while profiling) the latest and the mean duration over the
    recorded invocations."""
    label: str
    klass: str
    algorithmic_bytes: float
    algorithmic_flops: float
    last_ms: float
    mean_ms: float = 0.0
    calls: int = 0


_lib = None
_lib_lock = threading.Lock()

EXPORTS = ["accy_hip_run", "accy_hip_compile", "accy_hip_counts", "accy_hip_describe", "accy_hip_invoke",
           "accy_hip_invoke_device", "accy_hip_invoke_device_scratch", "accy_hip_release", "accy_hip_last_error", "accy_hip_set_profiling",
           "accy_hip_kernel_count", "accy_hip_kernel_info", "accy_hip_plan_source", "accy_hip_device_arch",
           "accy_hip_malloc", "accy_hip_free", "accy_hip_memcpy", "accy_hip_stream_create",
           "accy_hip_stream_destroy", "accy_hip_stream_synchronize", "accy_hip_event_create",
           "accy_hip_event_destroy", "accy_hip_event_record", "accy_hip_event_elapsed_ms", "accy_hip_tune",
           "accy_hip_tuning_export", "accy_hip_tuning_import", "accy_hip_tuning_count", "accy_hip_tuning_clear"]


def library() -> ctypes.CDLL:
    """Loads libaccy_hip.so (raises if it has not been built)."""
    global _lib
    with _lib_lock:
        if _lib is not None:
            return _lib
        if not _LIB_PATH.exists():
            raise RuntimeError(f"{_LIB_PATH} is missing: run accy_amd.build.build_library() first")
        lib = ctypes.CDLL(str(_LIB_PATH))
        vp, sz, u8p = ctypes.c_void_p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_uint8)
        vpp, szp = ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_size_t)
        lib.accy_hip_run.argtypes = [u8p, sz, vpp, szp, sz, vpp, szp, sz]
        lib.accy_hip_compile.argtypes = [u8p, sz, ctypes.POINTER(Handle)]
        lib.accy_hip_counts.argtypes = [Handle, szp, szp]
        lib.accy_hip_describe.argtypes = [Handle, ctypes.c_int, sz, ctypes.POINTER(_Descriptor)]
        lib.accy_hip_invoke.argtypes = [Handle, vpp, szp, sz, vpp, szp, sz]
        lib.accy_hip_invoke_device.argtypes = [Handle, vpp, sz, vpp, sz, vp]
        lib.accy_hip_invoke_device_scratch.argtypes = [Handle, vpp, sz, vpp, sz, vp]
        lib.accy_hip_release.argtypes = [Handle]
        lib.accy_hip_last_error.restype = ctypes.c_char_p
        lib.accy_hip_set_profiling.argtypes = [Handle, ctypes.c_int]
        lib.accy_hip_kernel_count.argtypes = [Handle, szp]
        lib.accy_hip_kernel_info.argtypes = [Handle, sz, ctypes.POINTER(_KernelStats)]
        lib.accy_hip_plan_source.argtypes = [u8p, sz, ctypes.c_int, ctypes.c_char_p, sz, szp]
        lib.accy_hip_device_arch.argtypes = [ctypes.c_char_p, sz]
        lib.accy_hip_malloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), sz]
        lib.accy_hip_free.argtypes = [vp]
        lib.accy_hip_memcpy.argtypes = [vp, vp, sz, ctypes.c_int]
        lib.accy_hip_stream_create.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        lib.accy_hip_stream_destroy.argtypes = [vp]
        lib.accy_hip_stream_synchronize.argtypes = [vp]
        lib.accy_hip_event_create.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        lib.accy_hip_event_destroy.argtypes = [vp]
        lib.accy_hip_event_record.argtypes = [vp, vp]
        lib.accy_hip_event_elapsed_ms.argtypes = [ctypes.POINTER(ctypes.c_float), vp, vp]
        lib.accy_hip_tune.argtypes = [u8p, sz, vpp, sz, vpp, sz, ctypes.c_uint32, szp]
        lib.accy_hip_tuning_export.argtypes = [ctypes.POINTER(ctypes.c_uint8), sz, szp]
        lib.accy_hip_tuning_import.argtypes = [ctypes.POINTER(ctypes.c_uint8), sz]
        lib.accy_hip_tuning_count.argtypes = [szp]
        lib.accy_hip_tuning_clear.argtypes = []
        for name in EXPORTS:
            if name != "accy_hip_last_error":
                getattr(lib, name).restype = ctypes.c_int
        _lib = lib
        return lib


def _check(status: int) -> None:
    if status != OK:
        raise HipError(status, library().accy_hip_last_error().decode(errors="replace"))


def _wire(program: Union[_tensor.Program, bytes, bytearray]) -> bytes:
    if isinstance(program, _tensor.Program):
        return program.encode()
    return bytes(program)


def _u8(buf: bytes):
    arr = (ctypes.c_uint8 * len(buf)).from_buffer_copy(buf) if buf else (ctypes.c_uint8 * 1)()
    return arr, len(buf)


def _in_ptr(x) -> Tuple[int, int, object]:
    """(address, length, keep-alive) of a read-only host buffer."""
    if isinstance(x, np.ndarray):
        a = np.ascontiguousarray(x)
        return a.ctypes.data, a.nbytes, a
    mv = memoryview(x).cast("B")
    if mv.readonly:
        a = np.frombuffer(mv, dtype=np.uint8)
        return a.ctypes.data if a.size else 0, a.nbytes, a
    a = np.frombuffer(mv, dtype=np.uint8)
    return a.ctypes.data if a.size else 0, a.nbytes, a


def _out_ptr(x) -> Tuple[int, int, object]:
    if isinstance(x, np.ndarray):
        if not x.flags.c_contiguous or not x.flags.writeable:
            raise HipError(INVALID_BUFFER, "outputs must be writable C-contiguous arrays")
        return x.ctypes.data, x.nbytes, x
    mv = memoryview(x).cast("B")
    if mv.readonly:
        raise HipError(INVALID_BUFFER, "outputs must be writable")
    a = np.frombuffer(mv, dtype=np.uint8)
    return a.ctypes.data if a.size else 0, a.nbytes, a


def _lists(items, conv):
    keep, ptrs, lens = [], [], []
    for x in items:
        p, n, k = conv(x)
        keep.append(k)
        ptrs.append(p)
        lens.append(n)
    pa = (ctypes.c_void_p * max(len(ptrs), 1))(*ptrs)
    la = (ctypes.c_size_t * max(len(lens), 1))(*lens)
    return pa, la, keep


def run_hip(program, inputs: Sequence, outputs: Sequence) -> None:
    """``tensor.runCpu`` on the MI355X: compile, launch once, copy outputs back, release."""
    lib = library()
    w, wl = _u8(_wire(program))
    ip, il, k1 = _lists(inputs, _in_ptr)
    op, ol, k2 = _lists(outputs, _out_ptr)
    _check(lib.accy_hip_run(w, wl, ip, il, len(inputs), op, ol, len(outputs)))


class Session:
    """The host-language session (session.zig:99-246): compile wire bytes, describe, invoke, release."""

    def __init__(self):
        self._lib = library()

    def compile(self, program) -> Handle:
        w, wl = _u8(_wire(program))
        h = Handle()
        _check(self._lib.accy_hip_compile(w, wl, ctypes.byref(h)))
        return h

    def _describe(self, h: Handle, which: int) -> List[Descriptor]:
        n_in, n_out = ctypes.c_size_t(), ctypes.c_size_t()
        _check(self._lib.accy_hip_counts(h, ctypes.byref(n_in), ctypes.byref(n_out)))
        out = []
        for i in range(n_in.value if which == 0 else n_out.value):
            d = _Descriptor()
            _check(self._lib.accy_hip_describe(h, which, i, ctypes.byref(d)))
            dims = tuple((d.names[j].decode(), int(d.extents[j])) for j in range(d.rank))
            out.append(Descriptor(_tensor.DTYPES[d.dtype], dims, int(d.byte_size), int(d.alignment)))
        return out

    def input_descriptors(self, h: Handle) -> List[Descriptor]:
        return self._describe(h, 0)

    def output_descriptors(self, h: Handle) -> List[Descriptor]:
        return self._describe(h, 1)

    def invoke(self, h: Handle, inputs: Sequence, outputs: Sequence) -> None:
        ip, il, k1 = _lists(inputs, _in_ptr)
        op, ol, k2 = _lists(outputs, _out_ptr)
        _check(self._lib.accy_hip_invoke(h, ip, il, len(inputs), op, ol, len(outputs)))

    def invoke_device(self, h: Handle, inputs: Sequence[int], outputs: Sequence[int], stream: int = 0) -> None:
        ip = (ctypes.c_void_p * max(len(inputs), 1))(*inputs)
        op = (ctypes.c_void_p * max(len(outputs), 1))(*outputs)
        _check(self._lib.accy_hip_invoke_device(h, ip, len(inputs), op, len(outputs), ctypes.c_void_p(stream)))

    def release(self, h: Handle) -> None:
        _check(self._lib.accy_hip_release(h))

    def set_profiling(self, h: Handle, enable: bool) -> None:
        _check(self._lib.accy_hip_set_profiling(h, 1 if enable else 0))

    def kernels(self, h: Handle) -> List[KernelStats]:
        n = ctypes.c_size_t()
        _check(self._lib.accy_hip_kernel_count(h, ctypes.byref(n)))
        out = []
        for i in range(n.value):
            k = _KernelStats()
            _check(self._lib.accy_hip_kernel_info(h, i, ctypes.byref(k)))
            out.append(KernelStats(k.label.decode(), k.klass.decode(), k.algorithmic_bytes, k.algorithmic_flops,
                                   k.last_ms, k.mean_ms, k.calls))
        return out


class Hip:
    """The executor (``Cpu`` in execute.zig:9-52): compile once with ``Hip(program)``, then ``launch``
    many times; ``deinit`` (or leaving a ``with`` block) releases device memory and kernels."""

    def __init__(self, program):
        self._session = Session()
        self.handle = self._session.compile(program)
        self.inputs = self._session.input_descriptors(self.handle)
        self.outputs = self._session.output_descriptors(self.handle)
        self._live = True

    def launch(self, inputs: Sequence, outputs: Sequence) -> None:
        self._session.invoke(self.handle, inputs, outputs)

    def launch_device(self, inputs: Sequence[int], outputs: Sequence[int], stream: int = 0) -> None:
        self._session.invoke_device(self.handle, inputs, outputs, stream)

    def set_profiling(self, enable: bool) -> None:
        self._session.set_profiling(self.handle, enable)

    def kernels(self) -> List[KernelStats]:
        return self._session.kernels(self.handle)

    def deinit(self) -> None:
        if self._live:
            self._live = False
            self._session.release(self.handle)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.deinit()

    def __del__(self):
        try:
            self.deinit()
        except Exception:
            pass


def plan_source(program, compile: bool = False) -> str:
    """The HIP sources the target generates for ``program`` (host-only; ``compile`` also runs hiprtc)."""
    lib = library()
    w, wl = _u8(_wire(program))
    need = ctypes.c_size_t()
    _check(lib.accy_hip_plan_source(w, wl, 1 if compile else 0, None, 0, ctypes.byref(need)))
    buf = ctypes.create_string_buffer(need.value)
    _check(lib.accy_hip_plan_source(w, wl, 0, buf, need.value, ctypes.byref(need)))
    return buf.value.decode()


# ---- launch tuning (src/executable/tuning.zig: measured candidates, one selection per kernel key) ----

def tune(program, inputs: Sequence[np.ndarray], repeats: int = 20) -> int:
    """Measures every launch candidate of the program's tunable kernels on the device (inputs copied
    to HBM first), checks that each candidate's outputs equal the default's byte for byte, and records
    the fastest candidate per kernel in the process-wide table. Returns the number of kernels tuned."""
    lib = library()
    w, wl = _u8(_wire(program))
    prog = program if isinstance(program, _tensor.Program) else None
    if prog is None:
        raise TypeError("tune needs a traced Program (for its output sizes)")
    ins = [DeviceBuffer.from_array(np.asarray(x)) for x in inputs]
    outs = [DeviceBuffer(int(np.prod(t.shape, dtype=np.int64)) * np.dtype(_tensor.NUMPY_DTYPE[t.dtype]).itemsize)
            for t in prog.output_types()]
    try:
        ip = (ctypes.c_void_p * max(len(ins), 1))(*[b.ptr for b in ins])
        op = (ctypes.c_void_p * max(len(outs), 1))(*[b.ptr for b in outs])
        n = ctypes.c_size_t()
        _check(lib.accy_hip_tune(w, wl, ip, len(ins), op, len(outs), int(repeats), ctypes.byref(n)))
        return int(n.value)
    finally:
        for b in ins + outs:
            b.free()


def tuning_export() -> bytes:
    """The process-wide tuning table as an artifact ("ACTT", version 1)."""
    lib = library()
    need = ctypes.c_size_t()
    _check(lib.accy_hip_tuning_export(None, 0, ctypes.byref(need)))
    buf = (ctypes.c_uint8 * max(need.value, 1))()
    _check(lib.accy_hip_tuning_export(buf, need.value, ctypes.byref(need)))
    return bytes(buf[: need.value])


def tuning_import(artifact: bytes) -> None:
    """Merges an artifact into the table (a record replaces one of the same key only when faster)."""
    data = bytes(artifact)
    buf = (ctypes.c_uint8 * max(len(data), 1)).from_buffer_copy(data if data else b"\0")
    _check(library().accy_hip_tuning_import(buf, len(data)))


def tuning_count() -> int:
    n = ctypes.c_size_t()
    _check(library().accy_hip_tuning_count(ctypes.byref(n)))
    return int(n.value)


def tuning_clear() -> None:
    _check(library().accy_hip_tuning_clear())


def device_arch() -> str:
    buf = ctypes.create_string_buffer(256)
    _check(library().accy_hip_device_arch(buf, 256))
    return buf.value.decode()


class DeviceBuffer:
    """Device memory from the library's own HIP runtime (``accy_hip_malloc``)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        _check(library().accy_hip_malloc(ctypes.byref(p), self.nbytes))
        self.ptr = p.value or 0

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        buf = cls(a.nbytes)
        buf.upload(a)
        return buf

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        if a.nbytes != self.nbytes:
            raise HipError(INVALID_BUFFER, "size mismatch")
        _check(library().accy_hip_memcpy(self.ptr, a.ctypes.data, self.nbytes, 1))

    def download(self, out: np.ndarray) -> np.ndarray:
        if out.nbytes != self.nbytes or not out.flags.c_contiguous:
            raise HipError(INVALID_BUFFER, "size mismatch")
        _check(library().accy_hip_memcpy(out.ctypes.data, self.ptr, self.nbytes, 2))
        return out

    def free(self) -> None:
        if self.ptr:
            library().accy_hip_free(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    """A HIP stream at the default priority."""

    def __init__(self):
        p = ctypes.c_void_p()
        _check(library().accy_hip_stream_create(ctypes.byref(p)))
        self.handle = p.value or 0

    def synchronize(self) -> None:
        _check(library().accy_hip_stream_synchronize(self.handle))

    def destroy(self) -> None:
        if self.handle:
            library().accy_hip_stream_destroy(self.handle)
            self.handle = 0


class Event:
    def __init__(self):
        p = ctypes.c_void_p()
        _check(library().accy_hip_event_create(ctypes.byref(p)))
        self.handle = p.value or 0

    def record(self, stream: "Stream") -> None:
        _check(library().accy_hip_event_record(self.handle, stream.handle if stream else 0))

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        _check(library().accy_hip_event_elapsed_ms(ctypes.byref(ms), self.handle, end.handle))
        return float(ms.value)

    def destroy(self) -> None:
        if self.handle:
            library().accy_hip_event_destroy(self.handle)
            self.handle = 0


def empty_output(desc: Descriptor) -> np.ndarray:
    """A host array sized and typed for one output descriptor."""
    shape = tuple(e for _, e in desc.dims)
    return np.zeros(shape, dtype=_tensor.NUMPY_DTYPE[desc.dtype])
