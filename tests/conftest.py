"""Shared fixtures: the CPU oracle (test infrastructure), the HIP target, and parity checks."""
from __future__ import annotations

import ctypes
import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))

from accy_amd import tensor as T  # noqa: E402

# ACCY_ORACLE_LIB names another build of the oracle (a copy with a mistake planted on purpose, to
# show that the pinning tests catch it).
ORACLE_LIB = Path(os.environ.get("ACCY_ORACLE_LIB", ROOT / "oracle" / "build" / "liboracle.so"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")


_oracle = None


def oracle_lib() -> ctypes.CDLL:
    global _oracle
    if _oracle is None:
        if not ORACLE_LIB.exists():
            from accy_amd import build
            build.build_oracle()
        lib = ctypes.CDLL(str(ORACLE_LIB))
        vpp, szp, sz = ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_size_t), ctypes.c_size_t
        u8p = ctypes.POINTER(ctypes.c_uint8)
        lib.accy_cpu_run.argtypes = [u8p, sz, vpp, szp, sz, vpp, szp, sz]
        lib.accy_cpu_run.restype = ctypes.c_int
        lib.accy_cpu_last_error.restype = ctypes.c_char_p
        lib.accy_cpu_error_name.restype = ctypes.c_char_p
        lib.accy_cpu_set_threads.argtypes = [ctypes.c_int]
        lib.accy_cpu_unary_f32.argtypes = [ctypes.c_int, ctypes.c_float]
        lib.accy_cpu_unary_f32.restype = ctypes.c_float
        lib.accy_cpu_wire_roundtrip.argtypes = [u8p, sz, u8p, sz, szp]
        lib.accy_cpu_wire_roundtrip.restype = ctypes.c_int
        _oracle = lib
    return _oracle


def _buf(b: bytes):
    return (ctypes.c_uint8 * max(len(b), 1)).from_buffer_copy(b if b else b"\0")


def out_arrays(program: T.Program):
    return [np.zeros(t.shape, dtype=T.NUMPY_DTYPE[t.dtype]) for t in program.output_types()]


def oracle_run(program, inputs, threads: int = 0):
    """Runs the CPU oracle (runCpu restatement) and returns the outputs as numpy arrays."""
    lib = oracle_lib()
    if threads:
        lib.accy_cpu_set_threads(threads)
    wire = program.encode() if isinstance(program, T.Program) else bytes(program)
    ins = [np.ascontiguousarray(x) for x in inputs]
    outs = out_arrays(program)
    ip = (ctypes.c_void_p * max(len(ins), 1))(*[x.ctypes.data for x in ins])
    il = (ctypes.c_size_t * max(len(ins), 1))(*[x.nbytes for x in ins])
    op = (ctypes.c_void_p * max(len(outs), 1))(*[x.ctypes.data for x in outs])
    ol = (ctypes.c_size_t * max(len(outs), 1))(*[x.nbytes for x in outs])
    st = lib.accy_cpu_run(_buf(wire), len(wire), ip, il, len(ins), op, ol, len(outs))
    if st != 0:
        raise RuntimeError(f"oracle status {st}: {lib.accy_cpu_last_error().decode()}")
    return outs


def wire_roundtrip(wire: bytes):
    """(status, bytes or error name) from the C++ codec's decode -> encode."""
    lib = oracle_lib()
    need = ctypes.c_size_t()
    st = lib.accy_cpu_wire_roundtrip(_buf(wire), len(wire), None, 0, ctypes.byref(need))
    if st != 0:
        return st, lib.accy_cpu_error_name().decode()
    out = (ctypes.c_uint8 * max(need.value, 1))()
    st = lib.accy_cpu_wire_roundtrip(_buf(wire), len(wire), out, need.value, ctypes.byref(need))
    return st, bytes(out[: need.value])


def hip_run(program, inputs):
    from accy_amd import hip
    outs = out_arrays(program)
    hip.run_hip(program, inputs, outs)
    return outs


def to_f32(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return (x.astype(np.uint32) << np.uint32(16)).view(np.float32)
    return x.astype(np.float32)


def assert_rel(got, ref, tol, dtype="f32"):
    """Per-element relative error |g - r| <= tol |r| (f32 reductions, BASELINE parity table)."""
    g = to_f32(np.asarray(got), dtype).astype(np.float64)
    r = to_f32(np.asarray(ref), dtype).astype(np.float64)
    err = np.abs(g - r)
    bound = tol * np.abs(r)
    bad = err > bound
    assert not bad.any(), (f"{bad.sum()} of {bad.size} elements off; worst rel "
                           f"{(err / np.maximum(np.abs(r), 1e-300)).max():.3e} (tol {tol})")


def exact_attention(q, k, v, scale, causal, dtype):
    """softmax(scale * q k^T [key <= query]) v in float64 from the 16-bit inputs: the textbook
    formula the reference's per-op evaluation approximates."""
    q, k, v = (to_f32(np.asarray(x), dtype).astype(np.float64) for x in (q, k, v))
    s = np.matmul(q, np.swapaxes(k, -1, -2)) * scale
    if causal:
        keep = np.arange(s.shape[-1])[None, :] <= np.arange(s.shape[-2])[:, None]
        s = np.where(keep, s, -np.inf)
    e = np.exp(s - s.max(-1, keepdims=True))
    return np.matmul(e / e.sum(-1, keepdims=True), v)


def assert_rowwise(got, ref, tol, dtype, exact=None):
    """Parity of outputs built from long 16-bit op chains (attention, a decoder block). Against
    runCpu's per-op 16-bit evaluation: max|g-r| / max|r| <= tol over the whole output and over every
    row (last axis); where runCpu's own error is the larger (exact given), an output or row beyond tol
    passes only if it is closer to the exact result than runCpu's. Against the float64 formula (when given): the error is at most 1.5x runCpu's own
    plus a 16-bit rounding of the largest output. (Where a result is a small difference of large
    16-bit intermediates, one rounding step of an intermediate moves it by more than a per-element
    relative bound allows, so none is asserted.)"""
    g = to_f32(np.asarray(got), dtype).astype(np.float64)
    r = to_f32(np.asarray(ref), dtype).astype(np.float64)
    assert g.shape == r.shape
    if r.size == 0:
        return
    scale = np.abs(r).max()
    err = np.abs(g - r)
    if exact is None or err.max() <= tol * scale:
        assert err.max() <= tol * scale, f"normwise error {err.max() / scale:.3e} > {tol}"
    else:
        # runCpu's per-op 16-bit evaluation can itself be further than tol from the exact result (bf16
        # attention rows over a few hundred keys: up to 2.9e-2 normwise); then the output passes only
        # if it is no further from the exact result than runCpu's is.
        mine, theirs = np.abs(g - exact).max(), np.abs(r - exact).max()
        assert mine <= theirs, (f"normwise error {err.max() / scale:.3e} > {tol} and error vs exact {mine:.3e} "
                                f"above runCpu's {theirs:.3e}")
    row_scale = np.abs(r).max(-1)
    row_err = err.max(-1)
    bad = row_err > tol * np.maximum(row_scale, 1e-30)
    ulp = 2.0 ** -10 if dtype == "f16" else 2.0 ** -7
    if exact is not None:
        # A row further than tol from runCpu passes only if it is closer to the exact result than
        # runCpu's row is (e.g. few-key attention rows under a causal mask, where runCpu's own
        # rounding dominates).
        mine_rows = np.abs(g - exact).max(-1)
        theirs_rows = np.abs(r - exact).max(-1)
        bad &= mine_rows > 1.5 * theirs_rows + ulp * np.abs(exact).max(-1)
    assert not bad.any(), f"{bad.sum()} of {bad.size} rows beyond {tol}: worst {(row_err / row_scale).max():.3e}"
    if exact is not None:
        mine = np.abs(g - exact).max()
        theirs = np.abs(r - exact).max()
        assert mine <= 1.5 * theirs + ulp * np.abs(exact).max(), f"error vs exact {mine:.3e}, runCpu's {theirs:.3e}"


assert_attention = assert_rowwise


def assert_no_less_accurate(got, ref, exact, dtype):
    """max|got - exact| <= 1.5 max|runCpu - exact| + one 16-bit rounding of max|exact|: the result
    is at least as close to the float64 value as runCpu's own per-op evaluation."""
    g = to_f32(np.asarray(got), dtype).astype(np.float64)
    r = to_f32(np.asarray(ref), dtype).astype(np.float64)
    ulp = {"f16": 2.0 ** -10, "bf16": 2.0 ** -7}.get(dtype, 2.0 ** -23)
    mine, theirs = np.abs(g - exact).max(), np.abs(r - exact).max()
    assert mine <= 1.5 * theirs + ulp * np.abs(exact).max(), f"error vs exact {mine:.3e}, runCpu's {theirs:.3e}"


def assert_normwise(got, ref, tol, dtype="f32", floor=1e-3):
    """GEMM / attention parity: max|g-r| / max|r| <= tol, and per element
    |g-r| <= tol (|r| + floor max|r|) unless floor is None."""
    g = to_f32(np.asarray(got), dtype).astype(np.float64)
    r = to_f32(np.asarray(ref), dtype).astype(np.float64)
    scale = np.abs(r).max() if r.size else 0.0
    err = np.abs(g - r)
    if r.size == 0:
        return
    assert err.max() <= tol * max(scale, 1e-30), f"normwise error {err.max() / max(scale, 1e-30):.3e} > {tol}"
    if floor is None:
        return
    bound = tol * (np.abs(r) + floor * scale)
    bad = err > bound
    assert not bad.any(), f"{bad.sum()} of {bad.size} elements beyond tol {tol} with floor {floor}"
