"""Every output element of every benchmark configuration at its BASELINE size, on an MI355X.

The sampled-row tests compare a few rows with the CPU oracle (runCpu's own arithmetic); these check
the whole output, so that a wrong tile number, batch or head offset anywhere in the grid fails:

* C1 tone: all 8192 guesses against the oracle (run in chunks of guesses; each guess is
  independent), per element relative 1e-5.
* C2 logsumexp: all 32768 rows against the float64 closed form m + log sum exp(x - m), per element
  relative 1e-5 (runCpu's own f32 error against it is below 1e-6 at this size).
* C3 contraction (the benchmarked mul + sum spelling), f32 and bf16: every element of C against the
  float64 product A B: normwise within BASELINE's 1e-3 (f32) / 2e-2 (bf16), and per element within
  the forward error bound of an f32 sum of K products in any order, K u sum_k |a_ik b_kj| (plus the
  truncating bf16 store, under 2^-7 relative). A single-tile fault is about 30x that bound. For
  bf16, 16 rows also against runCpu's plan of this spelling (per-product bf16 truncation) at 2e-2.
* C4 attention: every query row of every head against float64 softmax(scale q k^T) v from the same
  f16 inputs: each row within 2e-3 of its largest magnitude (measured about 5e-4 normwise; runCpu's
  own per-op f16 evaluation is about 1.7e-3 away).
* C5 decoder block: all four batch elements against a float64 formulation of the block (RMSNorm,
  projections, causal softmax attention, GELU with the tanh approximation, residuals) from the same
  bf16 inputs: each batch element no further from it than 1.5x runCpu's own error on batch element 2
  (oracle) plus one bf16 rounding of the largest output.
"""
import math

import numpy as np
import pytest

from accy_amd import workloads as W
from conftest import assert_no_less_accurate, assert_normwise, assert_rel, hip_run, oracle_run, to_f32
from test_cpu_plan import lib as plan_lib

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


def test_c1_tone_every_guess():
    say("C1 tone 8192 x 16384: all guesses against the oracle")
    f, t, s = W.tone_inputs(8192, 16384, seed=1)
    got = hip_run(W.tone_program(8192, 16384), [f, t, s])[0]
    chunk = 1024
    prog = W.tone_program(chunk, 16384)
    for g0 in range(0, 8192, chunk):
        ref = oracle_run(prog, [f[g0:g0 + chunk], t, s])[0]
        assert_rel(got[g0:g0 + chunk], ref, 1e-5)


def test_c2_logsumexp_every_row():
    say("C2 logsumexp 32768 x 8192: all rows against float64")
    x = W.logsumexp_inputs(32768, 8192, seed=2)[0]
    got = hip_run(W.logsumexp_program(32768, 8192), [x])[0]
    for r0 in range(0, 32768, 2048):
        xb = x[r0:r0 + 2048].astype(np.float64)
        m = xb.max(axis=1)
        exact = m + np.log(np.exp(xb - m[:, None]).sum(axis=1))
        err = np.abs(got[r0:r0 + 2048].astype(np.float64) - exact)
        assert (err <= 1e-5 * np.abs(exact)).all(), f"rows {r0}..: worst rel {(err / np.abs(exact)).max():.3e}"


@pytest.mark.parametrize("dtype,tol", [("f32", 1e-3), ("bf16", 2e-2)])
def test_c3_contraction_every_element(dtype, tol):
    say(f"C3 {dtype} 8192^3 mul + sum: every element against the float64 product")
    a, b = W.gemm_inputs(8192, 8192, 8192, dtype)
    got = to_f32(hip_run(W.gemm_program(8192, 8192, 8192, dtype, "mulsum"), [a, b])[0], dtype).astype(np.float64)
    a64, b64 = to_f32(a, dtype).astype(np.float64), to_f32(b, dtype).astype(np.float64)
    del a, b
    exact = a64 @ b64
    scale = np.abs(exact).max()
    err = np.abs(got - exact)
    assert err.max() <= tol * scale, f"normwise {err.max() / scale:.3e} > {tol}"
    # Per element, the forward error bound of an f32 sum of K products in any order,
    # |err| <= K u sum_k |a_ik b_kj| (u = 2^-24), plus for bf16 the truncating store (< 2^-7 relative).
    # A misplaced or missing tile is off by about |C| (~30), against a bound of about 1.
    bound = 8192 * 2.0 ** -24 * (np.abs(a64) @ np.abs(b64))
    if dtype == "bf16":
        bound = 2.0 ** -7 * np.abs(exact) + (1 + 2.0 ** -7) * bound
    bad = err > bound
    assert not bad.any(), f"{bad.sum()} elements beyond the bound; worst ratio {(err / bound).max():.3f}"
    if dtype == "bf16":
        # Against runCpu's own plan of this spelling (oracle/runcpu_plan.cpp, pinned bit for bit to
        # the op-by-op oracle): 16 rows at K = 8192. runCpu truncates every product to bf16 before
        # its serial f32 sum, a noise of about 2^-8 |a b| per product that the matrix cores' exact
        # products do not carry; near-zero sums differ by that noise, so the per-element bound has a
        # floor of 0.1 max|C| (the exact product truncated once measures 0.76 of this bound on these
        # rows), and the result must be at least as close to the float64 product as runCpu's.
        rows = np.sort(np.random.default_rng(1).choice(8192, 16, replace=False))
        a, b = W.gemm_inputs(8192, 8192, 8192, dtype)
        a_rows = np.ascontiguousarray(a[rows])   # held while the C function reads it
        ref = np.zeros((16, 8192), np.uint16)
        plan_lib().accy_cpu_plan_mulsum(a_rows.ctypes.data, b.ctypes.data, 16, 8192, 8192, 1, ref.ctypes.data)
        got16 = (got[rows].astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
        assert_normwise(got16, ref, tol, dtype, floor=0.1)
        assert_no_less_accurate(got16, ref, exact[rows], dtype)


def test_c4_attention_every_head():
    say("C4 attention f16 32 x 4096 x 4096 x 128: every query row of every head against float64")
    q, k, v = W.attention_inputs(32, 4096, 128, "f16")
    got = hip_run(W.attention_program(32, 4096, 128, "f16"), [q, k, v])[0]
    scale = float(np.float16(1.0 / math.sqrt(128)))   # the traced constant is f16
    for h in range(32):
        kh, vh = k[h].astype(np.float64), v[h].astype(np.float64)
        worst = 0.0
        for r0 in range(0, 4096, 1024):
            s = q[h, r0:r0 + 1024].astype(np.float64) @ kh.T * scale
            e = np.exp(s - s.max(-1, keepdims=True))
            exact = (e / e.sum(-1, keepdims=True)) @ vh
            err = np.abs(got[h, r0:r0 + 1024].astype(np.float64) - exact)
            # per row: within 2e-3 of the row's largest magnitude (measured about 5e-4 normwise)
            row = err.max(-1) / np.abs(exact).max(-1)
            assert (row <= 2e-3).all(), f"head {h}, rows {r0 + np.flatnonzero(row > 2e-3)[:4]}: {row.max():.3e}"
            worst = max(worst, float(row.max()))
        say(f"head {h}: worst row {worst:.2e}")


def _bf16_const(v):
    """A constant as the program traces it in bf16: the high half of its f32 value (Bf16.fromF32)."""
    return float(to_f32(np.array([np.float32(v).view(np.uint32) >> 16], np.uint16), "bf16")[0])


def _decoder_f64(ins):
    """The decoder block in float64 from the bf16 inputs (batch x seq x model), with the program's own
    bf16 constants (scale, epsilon, GELU coefficients): the traced program in exact arithmetic."""
    x, g1, wq, wk, wv, wo, g2, w1, w2 = [to_f32(a, "bf16").astype(np.float64) for a in ins]
    B, S, M = x.shape
    H, D = wq.shape[1], wq.shape[2]
    eps, scale = _bf16_const(1e-5), _bf16_const(1.0 / math.sqrt(D))
    c0, c1 = _bf16_const(0.7978845608028654), _bf16_const(0.044715)

    def rms(t, g):
        return t / np.sqrt((t * t).mean(-1, keepdims=True) + eps) * g
    h = rms(x, g1).reshape(B * S, M)
    q = (h @ wq.reshape(M, H * D)).reshape(B, S, H, D)
    k = (h @ wk.reshape(M, H * D)).reshape(B, S, H, D)
    v = (h @ wv.reshape(M, H * D)).reshape(B, S, H, D)
    o = np.empty((B, S, H, D))
    keep = np.tril(np.ones((S, S), bool))
    for bi in range(B):
        for hi in range(H):
            s = q[bi, :, hi] @ k[bi, :, hi].T * scale
            s = np.where(keep, s, -np.inf)
            p = np.exp(s - s.max(-1, keepdims=True))
            o[bi, :, hi] = (p / p.sum(-1, keepdims=True)) @ v[bi, :, hi]
    x1 = x.reshape(B * S, M) + o.reshape(B * S, H * D) @ wo.reshape(H * D, M)
    f = rms(x1, g2) @ w1
    f = 0.5 * f * (1 + np.tanh(c0 * (f + c1 * f ** 3)))
    return (x1 + f @ w2).reshape(B, S, M)


def test_c5_decoder_every_batch_element():
    say("C5 decoder 4 x 2048 x 2048: all batch elements against float64")
    ins = W.decoder_inputs()
    got = to_f32(hip_run(W.decoder_program(), ins)[0], "bf16").astype(np.float64)
    exact = _decoder_f64(ins)
    b = 2
    ref = to_f32(oracle_run(W.decoder_program(batch=1), [ins[0][b:b + 1]] + ins[1:])[0], "bf16").astype(np.float64)
    theirs = np.abs(ref[0] - exact[b]).max()
    for bi in range(4):
        mine = np.abs(got[bi] - exact[bi]).max()
        bound = 1.5 * theirs + 2.0 ** -7 * np.abs(exact[bi]).max()
        assert mine <= bound, f"batch {bi}: error vs float64 {mine:.3e}, runCpu's {theirs:.3e}"
        assert mine <= 2e-2 * np.abs(exact[bi]).max()
