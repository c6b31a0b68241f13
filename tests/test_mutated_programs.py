"""Mutated programs: the wire bytes of traced programs with a few bytes changed.

Most mutations give bytes the decoder refuses; the rest are valid programs the tracer would not write
(other extents, dtypes, operation codes, inits, axes). Both kinds go through the C ABI:

* every mutated program gets a status from accy_hip_plan_source (decode, type derivation, planning;
  no compile), never a crash (CPU);
* valid mutated programs with small values and no scans run on the GPU against the oracle on seeded
  inputs: integer and boolean outputs bit for bit, float outputs with the same NaN and infinity
  positions and within 1e-4 (f32, f64) or 2e-2 (16-bit) of the largest finite output.

Running such programs against the oracle found the row kernel adding a sum's init once per thread.
Float inputs are scaled by 0.1: with unit-scale weights a decoder block's scores reach the hundreds, the
softmax is nearly one-hot, and a one-ulp difference of a score flips which key wins (there the GPU
result was the closer of the two to float64).
"""
import ctypes
import random

import numpy as np
import pytest

from accy_amd import hip, tensor as T, workloads as W
from conftest import _buf, oracle_lib, to_f32
import test_random_programs as R
from test_wire import _decoder_types


def _bases():
    out = [W.tone_program(8, 64), W.logsumexp_program(16, 128), W.gemm_program(64, 96, 32, "bf16", "mulsum"),
           W.gemm_program(64, 32, 48, "f32", "contract"), W.attention_program(2, 64, 64, "bf16", causal=True),
           W.attention_program(1, 64, 64, "f32"), W.decoder_program(1, 32, 64, 2, 32, 128, dtype="bf16")]
    for s in range(8):
        out += [R._program(s, "f32")[0], R._program(s, "i32")[0], R._contraction_program(s, "bf16")[0]]
    return [p.encode() for p in out]


def _mutate(w: bytes, rng: random.Random) -> bytes:
    b = bytearray(w)
    for _ in range(rng.choice([1, 1, 2])):
        if not b:
            break
        pos = rng.randrange(len(b))
        p = pos - pos % 4
        kind = rng.randrange(5)
        if kind == 0:
            b[pos] ^= 1 << rng.randrange(8)
        elif kind == 1:
            b[pos] = rng.randrange(256)
        elif kind == 2:
            b[p:p + 4] = rng.randrange(2 ** 32).to_bytes(4, "little")[:len(b[p:p + 4])]
        elif kind == 3:
            b[p:p + 4] = rng.randrange(9).to_bytes(4, "little")[:len(b[p:p + 4])]
        else:
            b = b[:pos]
    return bytes(b)


def _plan_status(lib, w: bytes) -> int:
    need = ctypes.c_size_t()
    return lib.accy_hip_plan_source(_buf(w), len(w), 0, None, 0, ctypes.byref(need))


def test_every_mutated_program_gets_a_status():
    lib = hip.library()
    rng = random.Random(1)
    bases = _bases()
    seen = set()
    for _ in range(5000):
        st = _plan_status(lib, _mutate(rng.choice(bases), rng))
        assert 0 <= st <= 8
        seen.add(st)
    assert 0 in seen and 1 in seen   # some mutated programs are valid, most are refused


def _small_valid(n: int, seed: int):
    """n valid mutated programs: decoded and planned, no scans, every value at most 2^18 elements."""
    lib = hip.library()
    rng = random.Random(seed)
    bases = _bases()
    out = []
    while len(out) < n:
        w = _mutate(rng.choice(bases), rng)
        if _plan_status(lib, w) != 0:
            continue
        try:
            types = _decoder_types(w)
            sizes = []
            for t in types:
                if t.split()[0] != "0" or t.split()[1] == "scan":
                    raise ValueError("scan")
                inner = t.split(" ", 2)[2]
                inner = inner[inner.index("{") + 1:inner.rindex("}")]
                n_el = 1
                for item in (inner.split(",") if inner else []):
                    n_el *= int(item.rsplit("=", 1)[1])
                sizes.append(n_el)
        except (AssertionError, UnicodeDecodeError, ValueError, IndexError):
            continue
        if max(sizes) <= (1 << 18):
            out.append(w)
    return out


def _input(desc, rng):
    shape = tuple(e for _, e in desc.dims)
    dt = desc.dtype
    if dt in ("f32", "f64"):
        return (0.1 * rng.standard_normal(shape)).astype(T.NUMPY_DTYPE[dt])
    if dt in ("bf16", "f16"):
        return W.to_dtype(0.1 * rng.standard_normal(shape), dt).reshape(shape)
    if dt == "i1":
        return rng.random(shape) < 0.5
    info = np.iinfo(T.NUMPY_DTYPE[dt])
    return rng.integers(max(info.min, -60), min(info.max, 60), size=shape, endpoint=True).astype(T.NUMPY_DTYPE[dt])


@pytest.mark.gpu
def test_valid_mutated_programs_match_the_oracle():
    ses = hip.Session()
    lib = oracle_lib()
    bad = []
    for i, w in enumerate(_small_valid(80, seed=2)):
        print(f"mutated program {i} ({len(w)} bytes)", flush=True)
        h = ses.compile(w)
        ins_d, outs_d = ses.input_descriptors(h), ses.output_descriptors(h)
        rng = np.random.default_rng(i)
        ins = [np.ascontiguousarray(_input(d, rng)) for d in ins_d]
        got = [np.zeros(tuple(e for _, e in d.dims), T.NUMPY_DTYPE[d.dtype]) for d in outs_d]
        ref = [np.zeros_like(g) for g in got]
        ses.invoke(h, ins, got)
        ses.release(h)
        ip = (ctypes.c_void_p * max(len(ins), 1))(*[x.ctypes.data for x in ins])
        il = (ctypes.c_size_t * max(len(ins), 1))(*[x.nbytes for x in ins])
        op = (ctypes.c_void_p * max(len(ref), 1))(*[x.ctypes.data for x in ref])
        ol = (ctypes.c_size_t * max(len(ref), 1))(*[x.nbytes for x in ref])
        if lib.accy_cpu_run(_buf(w), len(w), ip, il, len(ins), op, ol, len(ref)) != 0:
            continue   # an unsupported operation nothing reads: the oracle evaluates every operation
        for j, (g, r, d) in enumerate(zip(got, ref, outs_d)):
            if d.dtype in ("f32", "f64", "bf16", "f16"):
                gf, rf = to_f32(g, d.dtype).astype(np.float64), to_f32(r, d.dtype).astype(np.float64)
                ok = np.array_equal(np.isnan(gf), np.isnan(rf)) and np.array_equal(np.isinf(gf), np.isinf(rf)) \
                    and np.array_equal(gf[np.isinf(gf)], rf[np.isinf(rf)])
                fin = np.isfinite(rf) & np.isfinite(gf)
                if ok and fin.any():
                    tol = 2e-2 if d.dtype in ("bf16", "f16") else 1e-4
                    ok = np.abs(gf[fin] - rf[fin]).max() <= tol * max(np.abs(rf[fin]).max(), 1e-30)
            else:
                ok = np.array_equal(g, r)
            if not ok:
                bad.append(f"program {i} output {j} {d.dtype}{d.dims}")
    assert not bad, bad
