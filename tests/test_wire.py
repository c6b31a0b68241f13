"""Tracer and ACTP v1 wire format (src/tensor/trace/builder.zig, src/tensor/wire/*.zig)."""
import ctypes
import struct

import numpy as np
import pytest

from accy_amd import tensor as T
from accy_amd import workloads as W
from conftest import oracle_lib, wire_roundtrip


def u32(v):
    return struct.pack("<I", v)


def i64(v):
    return struct.pack("<q", v)


def s(b: bytes):
    return u32(len(b)) + b


def readme_one_guess_bytes() -> bytes:
    """The README's one-guess mismatch program written out by hand from format.zig / encode.zig:
    kind codes parameter=0 constant=1 unary=2 binary=3 broadcast_in_dim=6 reduce=9; dtype f32=11;
    unary sin=6; binary sub=1 mul=2; reducer sum=0."""
    point = s(b"point") + i64(16)
    body = [
        u32(0) + u32(11) + u32(0),                                 # %0 frequency f32 {}
        u32(0) + u32(11) + u32(1) + point,                         # %1 time f32 {point}
        u32(0) + u32(11) + u32(1) + point,                         # %2 sample
        u32(6) + u32(1) + point + u32(0) + u32(0),                 # %3 broadcast_in_dim(%0, [])
        u32(3) + u32(2) + u32(3) + u32(1),                         # %4 mul(%3, %1)
        u32(2) + u32(6) + u32(4),                                  # %5 sin(%4)
        u32(3) + u32(1) + u32(5) + u32(2),                         # %6 sub(%5, %2)
        u32(3) + u32(2) + u32(6) + u32(6),                         # %7 mul(%6, %6)
        u32(1) + u32(11) + u32(0) + s(b"\0\0\0\0"),                # %8 const f32 0
        u32(9) + u32(7) + u32(8) + u32(0) + u32(1) + i64(0),       # %9 reduce sum over [0]
    ]
    return b"ACTP" + u32(1) + s(b"mismatch") + u32(len(body)) + b"".join(body) + u32(1) + u32(9)


def test_tracer_writes_the_hand_encoded_readme_program():
    prog = W.tone_program(points=16, scalar=True)
    assert prog.encode() == readme_one_guess_bytes()


def test_cpp_codec_round_trips_every_config_program_byte_for_byte():
    programs = [W.tone_program(8, 16), W.logsumexp_program(4, 32), W.gemm_program(4, 8, 3),
                W.gemm_program(4, 8, 3, "bf16", "mulsum"), W.attention_program(2, 16, 8),
                W.attention_program(2, 16, 8, causal=True), W.decoder_program(1, 8, 16, 2, 8, 32)]
    for p in programs:
        wire = p.encode()
        st, back = wire_roundtrip(wire)
        assert st == 0, back
        assert back == wire


def test_scan_and_indexing_programs_round_trip():
    def body(b, a):
        idx = a[1]
        g = a[0].gather(idx, "v")
        sc = a[0].scatter_add(idx, g, "v")
        loop = b.scan(3, [sc], lambda bb, c: [c[0].add(c[0])])
        return [loop, g]
    p = T.define("ix", [T.spec("f32", v=5), T.spec("i32", j=5)], body)
    wire = p.encode()
    st, back = wire_roundtrip(wire)
    assert st == 0 and back == wire


@pytest.mark.parametrize("mutate,status,name", [
    (lambda w: b"XCTP" + w[4:], 1, "BadMagic"),
    (lambda w: w[:4] + u32(2) + w[8:], 2, "UnsupportedVersion"),
    (lambda w: w[:-3], 1, "InvalidArtifact"),
    (lambda w: w + b"\0", 1, "InvalidArtifact"),
])
def test_decoder_refuses_bad_bytes(mutate, status, name):
    st, err = wire_roundtrip(mutate(readme_one_guess_bytes()))
    assert st == status and err == name


def test_decoder_refuses_unknown_tag_and_bad_reference():
    w = readme_one_guess_bytes()
    # The first operation's kind code sits after magic, version, name and the op count.
    off = 4 + 4 + 4 + len(b"mismatch") + 4
    bad_tag = w[:off] + u32(99) + w[off + 4:]
    assert wire_roundtrip(bad_tag) == (1, "UnknownTag")
    bad_ref = w[:-4] + u32(10)    # output id past the last value
    assert wire_roundtrip(bad_ref) == (1, "InvalidReference")


def test_decoder_derives_types_instead_of_trusting_bytes():
    # Rewrite %4 = mul(%3, %1) as mul(%3, %0): f32{point} * f32{} is a ShapeMismatch in the builder.
    w = readme_one_guess_bytes()
    good = u32(3) + u32(2) + u32(3) + u32(1)
    bad = u32(3) + u32(2) + u32(3) + u32(0)
    assert w.count(good) == 1
    assert wire_roundtrip(w.replace(good, bad)) == (1, "ShapeMismatch")


# ---- tracer behaviour (builder.zig, algebra.zig; main.zig:230-258) ----

def test_names_keep_guesses_and_points_apart_when_lengths_are_equal():
    p = W.tone_program(guesses=16, points=16)
    out = p.output_types()[0]
    assert out.dims == (("guess", 16),)


def test_samples_and_times_of_different_lengths_are_refused_while_recording():
    with pytest.raises(T.TensorError) as e:
        T.define("mismatch", [T.spec("f32"), T.spec("f32", point=16), T.spec("f32", point=15)], W.mismatch)
    assert e.value.name == "AxisExtentMismatch"


def test_alignment_transposes_then_broadcasts():
    b = T.Builder("t")
    x = b.input("f32", b=3, a=2)
    y = b.input("f32", a=2, c=4)
    z = x.add(y)               # target [b, a, c]
    assert z.ty.dims == (("b", 3), ("a", 2), ("c", 4))
    w = y.add(x)               # target [a, c, b]: x [b, a] needs a transpose to [a, b] first
    kinds = [op.kind for op in b.operations]
    assert "transpose" in kinds and kinds.count("broadcast_in_dim") >= 2
    assert w.ty.dims == (("a", 2), ("c", 4), ("b", 3))


def test_contract_canonicalises_operands():
    b = T.Builder("c")
    a = b.input("f32", k=4, m=3)
    w = b.input("f32", n=5, k=4)
    c = a.contract(w, "k")
    op = b.operations[c.id]
    assert op.kind == "dot_general" and c.ty.dims == (("m", 3), ("n", 5))
    assert op.dot == ((1,), (0,), (), ())
    assert b.operations[op.args[0]].kind == "transpose" and b.operations[op.args[1]].kind == "transpose"


def test_reduce_init_and_mean():
    b = T.Builder("r")
    x = b.input("bf16", r=2, c=3)
    m = x.max("c")
    init = b.operations[b.operations[m.id].args[1]]
    assert init.payload == bytes([0x80, 0xFF])    # Bf16.fromF32(-inf)
    mean = x.mean("c")
    div = b.operations[mean.id]
    assert div.code == "div"
    assert b.operations[b.operations[div.args[1]].args[0]].payload == W.to_dtype(np.array([3.0], np.float32), "bf16").tobytes()


@pytest.mark.parametrize("make,err", [
    (lambda b: b.input("f32", a=2).add(b.input("f16", a=2)), "DTypeMismatch"),
    (lambda b: b.input("f32", a=2).sum("z"), "AxisNotFound"),
    (lambda b: b.input("f32", a=2, c=3).merge(("a", "q"), "m"), "AxisNotFound"),
    (lambda b: b.input("f32", a=6).split("a", x=4, y=2), "SplitExtentMismatch"),
    (lambda b: b.input("f32", **{"#a": 2}), "AxisNameReserved"),
    (lambda b: b.input("f32", a=2).reduce(b.input("f32", z=1), "sum", "a"), "ReduceInitNotScalar"),
    (lambda b: b.input("f32", a=2).gather(b.input("f32", j=2), "a"), "DTypeMismatch"),
])
def test_recording_errors(make, err):
    with pytest.raises(T.TensorError) as e:
        make(T.Builder("e"))
    assert e.value.name == err


# ---- the decoder's derived types against the tracer's (the oracle shares the decoder) ----

def _python_types(prog, depth=0):
    out = []
    for op in prog.operations:
        dims = ",".join(f"{n}={e}" for n, e in op.result.dims)
        out.append(f"{depth} {op.kind} {op.result.dtype}{{{dims}}}")
        if op.body is not None:
            out.extend(_python_types(op.body, depth + 1))
    return out


def _decoder_types(wire: bytes):
    lib = oracle_lib()
    lib.accy_cpu_wire_types.argtypes = [ctypes.POINTER(ctypes.c_uint8), ctypes.c_size_t, ctypes.c_char_p,
                                        ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t)]
    need = ctypes.c_size_t()
    buf = (ctypes.c_uint8 * len(wire)).from_buffer_copy(wire)
    assert lib.accy_cpu_wire_types(buf, len(wire), None, 0, ctypes.byref(need)) == 0
    out = ctypes.create_string_buffer(need.value)
    assert lib.accy_cpu_wire_types(buf, len(wire), out, need.value, ctypes.byref(need)) == 0
    return out.value.decode().splitlines()


def _type_corpus():
    import test_random_programs as R
    progs = [W.tone_program(8192, 16384), W.logsumexp_program(32768, 8192),
             W.gemm_program(8192, 8192, 8192, "bf16", "mulsum"), W.gemm_program(64, 32, 16, "f32", "contract"),
             W.attention_program(32, 4096, 128, "f16"), W.attention_program(2, 256, 64, "bf16", causal=True),
             W.decoder_program(), W.decoder_program(2, 8, 16, 2, 8, 32, dtype="f32")]
    progs += [R._program(s, d)[0] for s in range(40) for d in ("f32", "i32")]
    progs += [R._contraction_program(s, d)[0] for s in range(24) for d in ("f32", "bf16")]
    progs += [R._scan_program(s, d)[0] for s in range(16) for d in ("f32", "i32")]
    return progs


def test_decoder_derives_the_same_types_as_the_tracer():
    """The C++ decoder replays every operation through its own checked builder; the Python tracer
    derived every type independently while recording (tensor.py). Both must give every value of every
    program, scan bodies included, the same dtype, axis names and extents: the oracle and the target
    share the decoder, so this is what pins its type derivation."""
    n = 0
    for prog in _type_corpus():
        want = _python_types(prog)
        got = _decoder_types(prog.encode())
        assert got == want, prog.name
        n += len(want)
    assert n > 2500
