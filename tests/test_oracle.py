"""Pins the CPU oracle (the runCpu restatement) before anything is compared against it.

Each check is chosen so that a plausible mistake in the restatement fails it: a pairwise or f64
accumulation instead of the serial f32 fold, a fused multiply-add, a dropped term, a transposed
operand, a wrong rounding of 16-bit results, unclamped gather indices.
"""
import math

import numpy as np
import pytest

from accy_amd import tensor as T
from accy_amd import workloads as W
from conftest import oracle_lib, oracle_run


def f64_mismatch(time, sample, frequency):
    """examples/consumer/src/main.zig:187-198: the mismatch and its slope in f64."""
    t = time.astype(np.float64)
    d = np.sin(frequency * t) - sample.astype(np.float64)
    return (d * d).sum(), (2 * d * np.cos(frequency * t) * t).sum()


# ---- known answers of the reference (README.md:152-160, 300-304; main.zig:200-228) ----

def test_readme_tone_known_answers():
    time, sample = W.readme_tone()
    one = W.tone_program(points=16, scalar=True)
    v25 = oracle_run(one, [np.array(2.5, np.float32), time, sample])[0]
    v3 = oracle_run(one, [np.array(3.0, np.float32), time, sample])[0]
    assert abs(float(v25) - 8.656) < 5e-4                       # README.md:152, 160 "about 8.656"
    ref, slope = f64_mismatch(time, sample, 2.5)
    assert abs(float(v25) - ref) <= 1e-5 * abs(ref)             # main.zig:208
    assert abs(float(v3)) <= 1e-9                               # main.zig:210
    assert abs(slope - (-31.29)) < 5e-3                         # README.md:300


def test_eight_guesses_equal_eight_single_runs():
    time, sample = W.readme_tone()
    starts = np.array([0.5, 1.5, 2.5, 3.5, 4.5, 5.5, 6.5, 7.5], np.float32)
    eight = oracle_run(W.tone_program(guesses=8, points=16), [starts, time, sample])[0]
    one = W.tone_program(points=16, scalar=True)
    for s, v in zip(starts, eight):
        alone = oracle_run(one, [np.array(s, np.float32), time, sample])[0]
        assert abs(float(alone) - float(v)) <= 1e-6 * abs(float(alone))   # main.zig:213-228
        assert abs(float(v) - f64_mismatch(time, sample, float(s))[0]) <= 1e-5 * abs(float(v))


def test_mismatch_curve_361_points_against_f64():
    """The README's figure data: 361 guesses from -0.5 to 8.5 (main.zig:152-181)."""
    time, sample = W.readme_tone()
    freq = (-0.5 + 0.025 * np.arange(361)).astype(np.float32)
    got = oracle_run(W.tone_program(guesses=361, points=16), [freq, time, sample])[0]
    for f, v in zip(freq, got):
        ref = f64_mismatch(time, sample, float(f))[0]
        assert abs(float(v) - ref) <= 1e-5 * abs(ref) + 1e-9


# ---- fold order (reduction.zig:839-878, 1157-1177) ----

def _sum_program(n, dtype="f32"):
    return T.define("s", [T.spec(dtype, i=n)], lambda b, a: a[0].sum("i"))


def test_sum_is_a_serial_left_to_right_f32_fold():
    # Serial f32: ((1e8 + 1) - 1e8) + 1 = 1; pairwise gives 0; f64 accumulation gives 2.
    x = np.array([1e8, 1.0, -1e8, 1.0], np.float32)
    assert float(oracle_run(_sum_program(4), [x])[0]) == 1.0


def test_sum_matches_explicit_serial_loop_bit_exact():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, 333)).astype(np.float32)
    prog = T.define("s", [T.spec("f32", a=5, b=333)], lambda b, a: a[0].sum("b"))
    got = oracle_run(prog, [x])[0]
    for r in range(5):
        acc = np.float32(0)
        for v in x[r]:
            acc = np.float32(acc + v)
        assert got[r] == acc


def test_multi_axis_reduce_folds_in_row_major_order_of_reduced_axes():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((3, 4, 5)) * 1e4).astype(np.float32)
    prog = T.define("s", [T.spec("f32", a=3, b=4, c=5)], lambda b, a: a[0].sum(("a", "c")))
    got = oracle_run(prog, [x])[0]
    for j in range(4):
        acc = np.float32(0)
        for i in range(3):
            for k in range(5):
                acc = np.float32(acc + x[i, j, k])
        assert got[j] == acc


def test_max_and_min_reduce():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((7, 64)).astype(np.float32)
    mx = T.define("m", [T.spec("f32", r=7, c=64)], lambda b, a: [a[0].max("c"), a[0].min("r")])
    got = oracle_run(mx, [x])
    assert np.array_equal(got[0], x.max(axis=1))
    assert np.array_equal(got[1], x.min(axis=0))


def _maxss_rule(x, y, greater):
    """deps/lib/compiler/choir/src/backends/x64/scalar.zig:675-720: maxss / minss return the second
    operand on a tie or a NaN, then a NaN result is replaced by the first operand."""
    r = x if ((x > y) if greater else (x < y)) else y
    return x if np.isnan(r) else r


def test_float_max_min_follow_maxss_with_nan_fixup():
    a = np.array([np.nan, 1.0, np.nan, 0.0, -0.0, 2.0, -np.inf, 3.0], np.float32)
    b = np.array([1.0, np.nan, np.nan, -0.0, 0.0, 2.0, np.inf, -3.0], np.float32)
    prog = T.define("mm", [T.spec("f32", i=8), T.spec("f32", i=8)],
                    lambda bb, v: [v[0].max(v[1]), v[0].min(v[1])])
    mx, mn = oracle_run(prog, [a, b])
    for i in range(8):
        for got, greater in ((mx[i], True), (mn[i], False)):
            want = np.float32(_maxss_rule(a[i], b[i], greater))
            assert got.view(np.uint32) == want.view(np.uint32) or (np.isnan(got) and np.isnan(want)), (i, got, want)
    # As a fold from -inf, a +0 / -0 tie keeps the later element's sign; NaN is skipped.
    fold = T.define("f", [T.spec("f32", r=3, i=3)], lambda bb, v: v[0].max("i"))
    x = np.array([[0.0, -0.0, -1.0], [-0.0, 0.0, -1.0], [np.nan, -5.0, np.nan]], np.float32)
    got = oracle_run(fold, [x])[0]
    assert np.signbit(got[0]) and not np.signbit(got[1]) and got[0] == 0 and got[2] == -5.0


def test_f16_sum_widens_to_f32_and_rounds_once():
    # 4096 ones in f16: an f16 accumulator sticks at 2048; the f32 accumulator reaches 4096.
    x = np.ones(4096, np.float16)
    assert float(oracle_run(_sum_program(4096, "f16"), [x])[0]) == 4096.0


# ---- elementwise arithmetic and 16-bit rounding (src/eval/root.zig:10-16) ----

@pytest.mark.parametrize("op", ["add", "sub", "mul", "div"])
def test_f16_binary_ops_round_to_nearest_even_after_each_op(op):
    rng = np.random.default_rng(3)
    with np.errstate(all="ignore"):   # magnitudes beyond f16's range overflow to infinity on purpose
        a = (rng.standard_normal(4096) * np.exp(rng.uniform(-12, 12, 4096))).astype(np.float16)
        b = (rng.standard_normal(4096) * np.exp(rng.uniform(-12, 12, 4096))).astype(np.float16)
    prog = T.define("e", [T.spec("f16", i=4096), T.spec("f16", i=4096)], lambda bb, x: getattr(x[0], op)(x[1]))
    got = oracle_run(prog, [a, b])[0]
    # numpy computes float16 arithmetic in f32 and rounds the result to nearest even.
    with np.errstate(all="ignore"):
        ref = getattr(np, {"add": "add", "sub": "subtract", "mul": "multiply", "div": "divide"}[op])(a, b)
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16)) or np.array_equal(
        np.nan_to_num(got.astype(np.float32)), np.nan_to_num(ref.astype(np.float32)))


def _bf16_trunc(x32):
    """Bf16.fromF32 (deps/lib/compiler/gpu/abi/src/dtype.zig:6-9): the high 16 bits of the f32."""
    return (np.asarray(x32, np.float32).view(np.uint32) >> np.uint32(16)).astype(np.uint16)


def _bf16_rne(x32):
    b = np.asarray(x32, np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def test_bf16_ops_truncate():
    """Every bf16 operation result keeps the high half of its f32 value (Bf16.fromF32, applied by the
    reference evaluator to binary ops at src/eval/evaluator.zig:2242-2244, unary at :2338, pow at
    :2384-2386, converts at :2860), not the nearest even. The inputs are chosen so that about half of
    the f32 results round up under nearest even: a nearest-even oracle fails every check."""
    rng = np.random.default_rng(4)
    a32 = rng.standard_normal(2048).astype(np.float32)
    b32 = rng.standard_normal(2048).astype(np.float32)
    a, b = W.to_dtype(a32, "bf16"), W.to_dtype(b32, "bf16")
    fa, fb = W.bf16_to_f32(a), W.bf16_to_f32(b)
    prog = T.define("e", [T.spec("bf16", i=2048), T.spec("bf16", i=2048)],
                    lambda bb, x: [x[0].mul(x[1]), x[0].add(x[1]), x[0].exp(), x[0].abs().pow(x[1])])
    mul, add, ex, pw = oracle_run(prog, [a, b])
    prod = (fa.astype(np.float64) * fb.astype(np.float64)).astype(np.float32)   # exact in f32
    summ = (fa.astype(np.float64) + fb.astype(np.float64)).astype(np.float32)   # exact in f32
    for got, f32 in [(mul, prod), (add, summ), (ex, np.exp(fa)), (pw, np.power(np.abs(fa), fb))]:
        assert np.array_equal(got, _bf16_trunc(f32))
        assert (got != _bf16_rne(f32)).mean() > 0.2


def test_bf16_reduction_and_dot_truncate_at_the_store():
    """A bf16 sum and a bf16 contraction accumulate in f32 (reduction.zig:847, 861; dot.zig:2004,
    2015) and the stored result is Bf16.fromF32 of the f32 accumulator: truncated."""
    rng = np.random.default_rng(14)
    x = W.to_dtype(rng.standard_normal((64, 96)).astype(np.float32), "bf16")
    y = W.to_dtype(rng.standard_normal((96, 32)).astype(np.float32), "bf16")
    fx, fy = W.bf16_to_f32(x), W.bf16_to_f32(y)
    prog = T.define("r", [T.spec("bf16", m=64, k=96), T.spec("bf16", k=96, n=32)],
                    lambda bb, a: [a[0].sum("k"), a[0].contract(a[1], "k")])
    s, d = oracle_run(prog, [x, y])
    acc = np.zeros(64, np.float32)
    for j in range(96):                       # serial f32 fold, left to right
        acc = (acc + fx[:, j]).astype(np.float32)
    assert np.array_equal(s, _bf16_trunc(acc))
    dacc = np.zeros((64, 32), np.float32)
    for j in range(96):                       # serial k, multiply and add rounded separately
        dacc = (dacc + (fx[:, j:j + 1] * fy[j:j + 1, :]).astype(np.float32)).astype(np.float32)
    assert np.array_equal(d, _bf16_trunc(dacc))
    assert (d != _bf16_rne(dacc)).mean() > 0.2


def test_tan_and_pow_against_f64():
    """The oracle's tan and pow (libm tanf / powf, as runCpu binds std.math functions) are within
    2 ulp of the float64 value, including pow's special cases (x^0 = 1, 1^y = 1, negative bases with
    integral exponents, NaN for a negative base with a fractional exponent, 0^-1 = inf)."""
    rng = np.random.default_rng(15)
    x = np.concatenate([rng.uniform(-1.5, 1.5, 2000), rng.uniform(-100, 100, 2000)]).astype(np.float32)
    got = oracle_run(T.define("t", [T.spec("f32", i=len(x))], lambda b, a: a[0].tan()), [x])[0].astype(np.float64)
    ref = np.tan(x.astype(np.float64))
    ulp = np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
    assert (np.abs(got - ref) <= 2 * ulp).all()
    base = np.concatenate([rng.uniform(0.05, 20, 3000), [2.0, 1.0, -2.0, -2.0, 0.0, -8.0, 3.0]]).astype(np.float32)
    expo = np.concatenate([rng.uniform(-8, 8, 3000), [0.0, 123.4, 3.0, 0.5, -1.0, 2.0, 0.0]]).astype(np.float32)
    got = oracle_run(T.define("p", [T.spec("f32", i=len(base))] * 2, lambda b, a: a[0].pow(a[1])),
                     [base, expo])[0].astype(np.float64)
    with np.errstate(all="ignore"):
        ref = np.power(base.astype(np.float64), expo.astype(np.float64))
    fin = np.isfinite(ref) & (np.abs(ref) < 3e38) & (np.abs(ref) > 1e-37)
    ulp = np.spacing(np.abs(ref[fin]).astype(np.float32)).astype(np.float64)
    assert (np.abs(got[fin] - ref[fin]) <= 2 * ulp).all()
    assert got[-7] == 1.0 and got[-6] == 1.0 and got[-5] == -8.0
    assert np.isnan(got[-4]) and got[-3] == np.inf and got[-2] == 64.0 and got[-1] == 1.0


@pytest.mark.parametrize("dtype,top", [("u8", 2 ** 8 - 1), ("u16", 2 ** 16 - 1), ("u32", 2 ** 32 - 1),
                                       ("u64", 2 ** 64 - 1)])
def test_unsigned_division_by_the_all_ones_value(dtype, top):
    """Unsigned division is plain truncating division: x / max is 0 below max and 1 at max (an
    implementation that treats the all-ones divisor as -1 returns 0 - x)."""
    npd = {"u8": np.uint8, "u16": np.uint16, "u32": np.uint32, "u64": np.uint64}[dtype]
    x = np.array([5, 0, top, top - 1, 1, top // 2], npd)
    y = np.array([top] * 6, npd)
    got = oracle_run(T.define("d", [T.spec(dtype, i=6)] * 2, lambda b, a: a[0].div(a[1])), [x, y])[0]
    assert list(got) == [0, 0, 1, 0, 0, 0]


def test_unary_f32_ops_against_f64():
    rng = np.random.default_rng(5)
    x = rng.uniform(0.1, 20.0, 1024).astype(np.float32)
    for name, f in [("exp", np.exp), ("log", np.log), ("sqrt", np.sqrt), ("tanh", np.tanh), ("sin", np.sin),
                    ("cos", np.cos), ("neg", np.negative), ("abs", np.abs)]:
        prog = T.define("u", [T.spec("f32", i=1024)], lambda b, a, n=name: getattr(a[0], n)())
        got = oracle_run(prog, [x])[0].astype(np.float64)
        ref = f(x.astype(np.float64))
        ulp = np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
        assert (np.abs(got - ref) <= 2 * ulp).all(), name


def test_no_fused_multiply_add_in_elementwise_chains():
    # a*b + c with a*b rounded first: chosen so that FMA gives a different f32 result.
    a = np.array([1.0 + 2.0 ** -12], np.float32)
    c = np.array([-(1.0 + 2.0 ** -11)], np.float32)
    prog = T.define("f", [T.spec("f32", i=1)] * 3, lambda b, x: x[0].mul(x[1]).add(x[2]))
    got = oracle_run(prog, [a, a, c])[0]
    separate = np.float32(np.float32(a[0] * a[0]) + c[0])
    fused = np.float32(np.float64(a[0]) * np.float64(a[0]) + np.float64(c[0]))
    assert separate != fused
    assert got[0] == separate


def test_integer_arithmetic_wraps_and_divides_toward_zero():
    x = np.array([2 ** 31 - 1, -7, 7, -(2 ** 31)], np.int32)
    y = np.array([1, 2, -2, -1], np.int32)
    prog = T.define("i", [T.spec("i32", i=4)] * 2, lambda b, a: [a[0].add(a[1]), a[0].div(a[1])])
    s, q = oracle_run(prog, [x, y])
    assert list(s) == [-(2 ** 31), -5, 5, 2 ** 31 - 1]
    assert list(q) == [2 ** 31 - 1, -3, -3, -(2 ** 31)]


# ---- contraction (dot.zig:2049-2115) ----

def test_dot_general_matches_serial_k_loop_bit_exact():
    rng = np.random.default_rng(6)
    a = rng.uniform(-1, 1, (6, 37)).astype(np.float32)
    b = rng.uniform(-1, 1, (37, 5)).astype(np.float32)
    got = oracle_run(W.gemm_program(6, 37, 5), [a, b])[0]
    for i in range(6):
        for j in range(5):
            acc = np.float32(0)
            for k in range(37):
                acc = np.float32(acc + np.float32(a[i, k] * b[k, j]))
            assert got[i, j] == acc
    assert np.abs(got - a.astype(np.float64) @ b.astype(np.float64)).max() < 1e-5


def test_mul_sum_spelling_equals_contract_spelling():
    rng = np.random.default_rng(7)
    a, b = W.gemm_inputs(9, 33, 7, seed=11)
    c1 = oracle_run(W.gemm_program(9, 33, 7, spelling="contract"), [a, b])[0]
    c2 = oracle_run(W.gemm_program(9, 33, 7, spelling="mulsum"), [a, b])[0]
    assert np.array_equal(c1, c2)


def test_batched_transposed_contraction_against_einsum():
    rng = np.random.default_rng(8)
    q = rng.standard_normal((3, 4, 8)).astype(np.float32)    # head, query, dim
    k = rng.standard_normal((3, 5, 8)).astype(np.float32)    # head, key, dim
    prog = T.define("qk", [T.spec("f32", head=3, query=4, dim=8), T.spec("f32", head=3, key=5, dim=8)],
                    lambda b, a: a[0].contract(a[1], "dim"))
    got = oracle_run(prog, [q, k])[0]
    ref = np.einsum("hqd,hkd->hqk", q.astype(np.float64), k.astype(np.float64))
    assert np.abs(got - ref).max() < 1e-5


def test_f16_contraction_accumulates_in_f32():
    # 4096 products of 1*1 in f16: an f16 accumulator would stop at 2048.
    a = np.ones((1, 4096), np.float16)
    b = np.ones((4096, 1), np.float16)
    assert float(oracle_run(W.gemm_program(1, 4096, 1, dtype="f16"), [a, b])[0][0, 0]) == 4096.0


# ---- attention, LSE, GELU closed forms ----

def test_attention_matches_reference_sdpa_closed_form():
    """src/kernel/library/attention.zig:464-509 (2 batches, 2 queries, 3 keys, qk 2, value 2)."""
    rng = np.random.default_rng(9)
    q = rng.standard_normal((2, 2, 2)).astype(np.float32)
    k = rng.standard_normal((2, 3, 2)).astype(np.float32)
    v = rng.standard_normal((2, 3, 2)).astype(np.float32)

    def body(b, a):
        s = a[0].contract(a[1], "qk").mul(b.full_float(T.Type("f32", ()), 1.0 / math.sqrt(2)))
        e = s.sub(s.max("key")).exp()
        return e.div(e.sum("key")).contract(a[2], "key")
    prog = T.define("sdpa", [T.spec("f32", batch=2, query=2, qk=2), T.spec("f32", batch=2, key=3, qk=2),
                             T.spec("f32", batch=2, key=3, value=2)], body)
    got = oracle_run(prog, [q, k, v])[0]
    scale = np.float32(1.0 / math.sqrt(2.0))
    for bi in range(2):
        for qi in range(2):
            sc = [np.float32(np.float32(q[bi, qi, 0] * k[bi, j, 0]) + np.float32(q[bi, qi, 1] * k[bi, j, 1])) * scale
                  for j in range(3)]
            m = max(sc)
            den = np.float32(0)
            for s_ in sc:
                den = np.float32(den + np.exp(np.float32(s_ - m)))
            for vi in range(2):
                acc = np.float32(0)
                for j in range(3):
                    acc = np.float32(acc + np.float32(np.float32(np.exp(np.float32(sc[j] - m)) / den) * v[bi, j, vi]))
                assert abs(got[bi, qi, vi] - acc) <= 1e-6 * max(1.0, abs(acc))


def test_logsumexp_against_f64():
    x = W.logsumexp_inputs(64, 1024, seed=21)[0]
    got = oracle_run(W.logsumexp_program(64, 1024), [x])[0]
    x64 = x.astype(np.float64)
    m = x64.max(axis=1)
    ref = m + np.log(np.exp(x64 - m[:, None]).sum(axis=1))
    assert np.abs(got - ref).max() <= 1e-6 * np.abs(ref).max()


def test_gelu_tanh_approximation_on_eight_values():
    """src/kernel/library/fused.zig:471-478 / elementwise.zig:234-240."""
    x = np.array([-3.0, -1.5, -0.5, -0.1, 0.0, 0.3, 1.0, 2.5], np.float32)
    prog = T.define("g", [T.spec("f32", i=8)], lambda b, a: W.gelu(b, a[0], "f32"))
    got = oracle_run(prog, [x])[0]
    x64 = x.astype(np.float64)
    ref = 0.5 * x64 * (1 + np.tanh(0.7978845608028654 * (x64 + 0.044715 * x64 ** 3)))
    assert np.abs(got - ref).max() <= 1e-6


def test_rms_norm_against_f64():
    rng = np.random.default_rng(10)
    x = rng.standard_normal((4, 64)).astype(np.float32)
    g = rng.uniform(0.5, 1.5, 64).astype(np.float32)
    prog = T.define("n", [T.spec("f32", r=4, model=64), T.spec("f32", model=64)],
                    lambda b, a: W.rms_norm(b, a[0], a[1], "model", "f32"))
    got = oracle_run(prog, [x, g])[0]
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-5) * g
    assert np.abs(got - ref).max() <= 1e-5


# ---- indexing ----

def test_gather_clamps_indices_into_range():
    x = np.arange(10, dtype=np.float32) * 10
    idx = np.array([-5, 0, 3, 9, 12], np.int32)
    prog = T.define("g", [T.spec("f32", v=10), T.spec("i32", j=5)], lambda b, a: a[0].gather(a[1], "v"))
    assert list(oracle_run(prog, [x, idx])[0]) == [0, 0, 30, 90, 90]


def test_scatter_add_accumulates_in_update_order():
    x = np.zeros(4, np.float32)
    idx = np.array([1, 1, 3, 1], np.int32)
    upd = np.array([1e8, 1.0, 5.0, -1e8], np.float32)
    prog = T.define("s", [T.spec("f32", v=4), T.spec("i32", j=4), T.spec("f32", j=4)],
                    lambda b, a: a[0].scatter_add(a[1], a[2], "v"))
    got = oracle_run(prog, [x, idx, upd])[0]
    assert list(got) == [0.0, 0.0, 0.0, 5.0]   # ((1e8 + 1) - 1e8) = 0 in serial f32


def test_decoder_block_small_against_f64():
    """A scaled-down decoder block in f32: every op of the traced program is checked against an
    independent f64 formulation (no dropped residual, mask, or norm)."""
    B, S, M, H, D, F = 2, 8, 16, 2, 8, 32
    ins = W.decoder_inputs(B, S, M, H, D, F, dtype="f32", seed=31)
    got = oracle_run(W.decoder_program(B, S, M, H, D, F, dtype="f32"), ins)[0].astype(np.float64)
    x, g1, wq, wk, wv, wo, g2, w1, w2 = [a.astype(np.float64) for a in ins]

    def rms(t, g):
        return t / np.sqrt((t * t).mean(-1, keepdims=True) + 1e-5) * g
    h = rms(x, g1)
    q = np.einsum("bsm,mhd->bshd", h, wq)
    k = np.einsum("bsm,mhd->bshd", h, wk)
    v = np.einsum("bsm,mhd->bshd", h, wv)
    s = np.einsum("bqhd,bkhd->bhqk", q, k) / math.sqrt(D)
    s = np.where(np.tril(np.ones((S, S), bool)), s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    o = np.einsum("bhqk,bkhd->bhqd", p, v)
    x1 = x + np.einsum("bhsd,hdm->bsm", o, wo)
    f = np.einsum("bsm,mf->bsf", rms(x1, g2), w1)
    f = 0.5 * f * (1 + np.tanh(0.7978845608028654 * (f + 0.044715 * f ** 3)))
    ref = x1 + np.einsum("bsf,fm->bsm", f, w2)
    assert np.abs(got - ref).max() <= 1e-4 * np.abs(ref).max()


def test_oracle_threads_give_identical_results():
    x = W.logsumexp_inputs(256, 512, seed=5)[0]
    prog = W.logsumexp_program(256, 512)
    one = oracle_run(prog, [x], threads=1)[0]
    many = oracle_run(prog, [x], threads=8)[0]
    assert np.array_equal(one, many)


# ---- integer, compare, f64, broadcast and reshape families ----
# Each check recomputes the expected value with Python integers or Python floats (float64), one
# element at a time, independently of the oracle's code: a signed compare on u64, a swapped lt / gt,
# a saturating or widened integer op, f64 evaluated through f32 or a dropped broadcast all fail.

_NP_INT = {"i32": np.int32, "i64": np.int64, "u32": np.uint32, "u64": np.uint64}
_BITS = {"i32": 32, "i64": 64, "u32": 32, "u64": 64}


def _wrap(v, dtype):
    """v reduced to the dtype's width (two's complement for signed types): Zig's +% -% *%."""
    bits = _BITS[dtype]
    v &= (1 << bits) - 1
    if dtype[0] == "i" and v >= 1 << (bits - 1):
        v -= 1 << bits
    return v


def _int_values(dtype, n, seed):
    """Edge values of the type (both ends, around zero and, unsigned, around 2^(bits-1)) followed by
    random values over the whole range."""
    info = np.iinfo(_NP_INT[dtype])
    lo, hi = int(info.min), int(info.max)
    edges = [lo, lo + 1, hi - 1, hi, 0, 1, 2, 3]
    if dtype[0] == "i":
        edges += [-1, -2, -3]
    else:
        edges += [1 << (_BITS[dtype] - 1), (1 << (_BITS[dtype] - 1)) - 1, (1 << (_BITS[dtype] - 1)) + 1]
    rng = np.random.default_rng(seed)
    rand = rng.integers(lo, hi, size=n - len(edges), dtype=_NP_INT[dtype], endpoint=True)
    return np.concatenate([np.array(edges, dtype=_NP_INT[dtype]), rand])


@pytest.mark.parametrize("dtype", ["i32", "i64", "u32", "u64"])
def test_integer_add_sub_mul_wrap_at_the_declared_width(dtype):
    """evalIntBinary (src/eval/evaluator.zig:2254-2263): add, sub and mul wrap (+% -% *%)."""
    x = _int_values(dtype, 96, 40)
    y = np.roll(_int_values(dtype, 96, 41), 5)
    prog = T.define("w", [T.spec(dtype, i=96)] * 2,
                    lambda b, a: [a[0].add(a[1]), a[0].sub(a[1]), a[0].mul(a[1])])
    add, sub, mul = oracle_run(prog, [x, y])
    for i in range(96):
        xi, yi = int(x[i]), int(y[i])
        assert int(add[i]) == _wrap(xi + yi, dtype), (i, xi, yi)
        assert int(sub[i]) == _wrap(xi - yi, dtype), (i, xi, yi)
        assert int(mul[i]) == _wrap(xi * yi, dtype), (i, xi, yi)


@pytest.mark.parametrize("dtype", ["i32", "i64", "u32", "u64"])
def test_integer_max_min_elementwise_and_as_folds(dtype):
    """@max / @min (evaluator.zig:2261-2262) on the type's own order: u64 values above 2^63 are the
    largest, not negative. As folds (reduction.zig:1140-1155) they start from the type's lowest /
    highest value (builder.zig:760-797; explicit inits for unsigned types) and take every element;
    the sum fold wraps."""
    x = _int_values(dtype, 8 * 24, 42).reshape(8, 24)
    y = _int_values(dtype, 8 * 24, 43).reshape(8, 24)[::-1].copy()
    info = np.iinfo(_NP_INT[dtype])

    def body(b, a):
        if dtype[0] == "i":
            return [a[0].max(a[1]), a[0].min(a[1]), a[0].max("c"), a[0].min("c"), a[0].sum("c"), a[0].max("r")]
        # The named max / min have no unsigned init (builder.zig:769-796): explicit inits instead.
        lo, hi = b.full(dtype, int(info.min)), b.full(dtype, int(info.max))
        return [a[0].max(a[1]), a[0].min(a[1]), a[0].reduce(lo, "max", "c"), a[0].reduce(hi, "min", "c"),
                a[0].sum("c"), a[0].reduce(lo, "max", "r")]
    prog = T.define("m", [T.spec(dtype, r=8, c=24)] * 2, body)
    mx, mn, fmax, fmin, fsum, fmax_r = oracle_run(prog, [x, y])
    X, Y = [[int(v) for v in row] for row in x], [[int(v) for v in row] for row in y]
    for r in range(8):
        for c in range(24):
            assert int(mx[r, c]) == max(X[r][c], Y[r][c]) and int(mn[r, c]) == min(X[r][c], Y[r][c])
        assert int(fmax[r]) == max(X[r]) and int(fmin[r]) == min(X[r])
        assert int(fsum[r]) == _wrap(sum(X[r]), dtype)
    for c in range(24):
        assert int(fmax_r[c]) == max(X[r][c] for r in range(8))


@pytest.mark.parametrize("dtype", ["i32", "u64"])
def test_integer_dot_general_wraps_per_output(dtype):
    """dot_general on integers (dot.zig:2049-2115 with the evaluator's wrapping add and multiply):
    out[m, n] = sum over k of a[m, k] * b[k, n], reduced to the type's width."""
    a = _int_values(dtype, 5 * 19, 44).reshape(5, 19)
    bm = _int_values(dtype, 19 * 7, 45).reshape(19, 7)
    got = oracle_run(W.gemm_program(5, 19, 7, dtype=dtype), [a, bm])[0]
    for m in range(5):
        for n in range(7):
            want = _wrap(sum(int(a[m, k]) * int(bm[k, n]) for k in range(19)), dtype)
            assert int(got[m, n]) == want, (m, n)
    # A batched contraction with the contracted axis first in one operand.
    p = _int_values(dtype, 3 * 4 * 6, 46).reshape(3, 4, 6)      # batch, k, m
    q = _int_values(dtype, 3 * 5 * 4, 47).reshape(3, 5, 4)      # batch, n, k
    prog = T.define("bd", [T.spec(dtype, batch=3, k=4, m=6), T.spec(dtype, batch=3, n=5, k=4)],
                    lambda b, v: v[0].contract(v[1], "k"))
    got = oracle_run(prog, [p, q])[0]
    assert got.shape == (3, 6, 5)
    for bi in range(3):
        for m in range(6):
            for n in range(5):
                want = _wrap(sum(int(p[bi, k, m]) * int(q[bi, n, k]) for k in range(4)), dtype)
                assert int(got[bi, m, n]) == want


_CMP = {"lt": lambda x, y: x < y, "le": lambda x, y: x <= y, "gt": lambda x, y: x > y,
        "ge": lambda x, y: x >= y, "eq": lambda x, y: x == y, "ne": lambda x, y: x != y}


@pytest.mark.parametrize("dtype", ["f32", "f64", "i32", "i64", "u32", "u64"])
def test_all_six_compares(dtype):
    """evalFloatCmp / evalIntCmp / evalUnsignedCmp (evaluator.zig:2454-2490): floats compare as
    IEEE values (NaN: only ne is true; -0 == +0), signed integers by value, unsigned integers on
    their unsigned order (u64 above 2^63 is large)."""
    if dtype in ("f32", "f64"):
        npd = np.float32 if dtype == "f32" else np.float64
        base = [np.nan, -np.inf, -3.5, -1.0, -0.0, 0.0, 1e-30, 1.0, 2.5, np.inf]
        x = np.array([u for u in base for _ in base], npd)
        y = np.array([v for _ in base for v in base], npd)
        X, Y = [float(v) for v in x], [float(v) for v in y]
    else:
        vals = _int_values(dtype, 16, 48)
        x = np.repeat(vals, 16)
        y = np.tile(vals, 16)
        X, Y = [int(v) for v in x], [int(v) for v in y]
    n = len(x)
    names = list(_CMP)
    prog = T.define("c", [T.spec(dtype, i=n)] * 2, lambda b, a: [a[0].compare(d, a[1]) for d in names])
    outs = oracle_run(prog, [x, y])
    for d, got in zip(names, outs):
        for i in range(n):
            assert bool(got[i]) == _CMP[d](X[i], Y[i]), (d, X[i], Y[i])


def test_f64_arithmetic_is_float64():
    """f64 runs evalFloatBinary / unary with f64 operands (evaluator.zig:2248-2250): add, sub, mul
    and div are the correctly rounded float64 results bit for bit (Python floats), exp is within
    one float64 ulp of the exact value, and an f64 sum is a serial float64 fold. Inputs are chosen
    so that evaluating through f32 changes every result."""
    rng = np.random.default_rng(49)
    x = (rng.standard_normal(256) * np.exp(rng.uniform(-30, 30, 256))).astype(np.float64)
    y = (rng.standard_normal(256) * np.exp(rng.uniform(-30, 30, 256))).astype(np.float64)
    e = rng.uniform(-700, 700, 256)
    prog = T.define("f", [T.spec("f64", i=256)] * 3,
                    lambda b, a: [a[0].add(a[1]), a[0].sub(a[1]), a[0].mul(a[1]), a[0].div(a[1]), a[2].exp()])
    add, sub, mul, div, ex = oracle_run(prog, [x, y, e])
    for i in range(256):
        xi, yi = float(x[i]), float(y[i])
        assert add[i] == xi + yi and sub[i] == xi - yi and mul[i] == xi * yi and div[i] == xi / yi
        assert float(np.float32(np.float32(xi) * np.float32(yi))) != xi * yi
        ref = math.exp(float(e[i]))
        assert abs(float(ex[i]) - ref) <= math.ulp(ref), (e[i], ex[i], ref)
    s = np.array([1e16, 1.0, -1e16, 1.0, 3.0, 2.0 ** -40], np.float64)
    got = oracle_run(T.define("s", [T.spec("f64", i=6)], lambda b, a: a[0].sum("i")), [s])[0]
    acc = 0.0
    for v in s:
        acc = acc + float(v)
    assert float(got) == acc and acc != float(np.float32(acc))


def test_f64_dot_is_a_serial_float64_fold():
    rng = np.random.default_rng(50)
    a = rng.standard_normal((4, 29)) * 1e10
    bm = rng.standard_normal((29, 3))
    got = oracle_run(W.gemm_program(4, 29, 3, dtype="f64"), [a, bm])[0]
    for m in range(4):
        for n in range(3):
            acc = 0.0
            for k in range(29):
                acc = acc + float(a[m, k]) * float(bm[k, n])
            assert got[m, n] == acc


@pytest.mark.parametrize("dtype", ["f32", "i32", "u64", "bf16"])
def test_broadcast_op_splats_one_element_and_copies_equal_sizes(dtype):
    """`broadcast` (builder.zig:487) lowers only from a splat (elementwise.zig:943-957): a
    one-element operand fills the result; an operand with as many elements is copied in order."""
    npd = T.NUMPY_DTYPE[dtype]
    one = np.array([7], npd).reshape(())
    six = np.arange(1, 7).astype(npd)
    prog = T.define("bc", [T.spec(dtype), T.spec(dtype, i=6)],
                    lambda b, a: [b.broadcast(a[0], [("r", 3), ("c", 5)]),
                                  b.broadcast(a[1], [("r", 2), ("c", 3)])])
    splat, copy = oracle_run(prog, [one, six])
    assert splat.shape == (3, 5) and (splat == npd(7)).all()
    assert copy.shape == (2, 3) and np.array_equal(copy.reshape(-1), six)
    with pytest.raises(RuntimeError):
        oracle_run(T.define("bad", [T.spec(dtype, i=2)], lambda b, a: b.broadcast(a[0], [("r", 4)])),
                   [six[:2]])


def test_split_and_merge_reshape_in_row_major_order():
    """Value.split / merge (builder.zig:438-470; value.zig:88-99): a split is a row-major reshape of
    one axis; a merge moves the merged axes together at the first one's position (algebra.zig:241-309)
    and reshapes. Checked element by element against numpy's reshape / transpose, and through a
    reduction over a split part and a contraction over a merged axis."""
    x = np.arange(2 * 12 * 5, dtype=np.int32).reshape(2, 12, 5)
    prog = T.define("sm", [T.spec("i32", a=2, b=12, c=5)],
                    lambda bb, v: [v[0].split("b", p=3, q=4), v[0].merge(("c", "a"), "m"),
                                   v[0].split("b", p=3, q=4).sum("q"), v[0].merge(("a", "b"), "m")])
    sp, mg, red, mg2 = oracle_run(prog, [x])
    assert np.array_equal(sp, x.reshape(2, 3, 4, 5))
    assert np.array_equal(mg, x.transpose(2, 0, 1).reshape(10, 12))
    for a in range(2):
        for p in range(3):
            for c in range(5):
                assert int(red[a, p, c]) == sum(int(x[a, 4 * p + q, c]) for q in range(4))
    assert np.array_equal(mg2, x.reshape(24, 5))
    y = np.arange(10 * 3, dtype=np.int32).reshape(10, 3) - 7
    prog = T.define("mc", [T.spec("i32", a=2, b=12, c=5), T.spec("i32", m=10, n=3)],
                    lambda bb, v: v[0].merge(("c", "a"), "m").contract(v[1], "m"))
    got = oracle_run(prog, [x, y])[0]
    want = x.transpose(2, 0, 1).reshape(10, 12).astype(np.int64).T @ y.astype(np.int64)
    assert np.array_equal(got, want.astype(np.int32))


def test_iota_broadcast_in_dim_transpose_and_select_against_numpy():
    """iota along one axis of a 2-D shape; an aligned binary of [a, b] with [b] (broadcast_in_dim) and
    with [b, a] (transpose, then elementwise, builder.zig:476-485); select on a compare; integer neg and
    abs wrapping at the most negative value."""
    prog = T.define("ib", [T.spec("f32", a=3, b=5), T.spec("f32", b=5), T.spec("f32", b=5, a=3),
                           T.spec("i32", i=6)],
                    lambda bb, v: [bb.iota("i32", "b", ("a", 3), ("b", 5)), bb.iota("f32", "a", ("a", 3), ("b", 5)),
                                   v[0].add(v[1]), v[0].sub(v[2]),
                                   v[0].compare("lt", v[2]).select(v[0], v[2].neg()),
                                   v[3].neg(), v[3].abs()])
    rng = np.random.default_rng(51)
    x = rng.standard_normal((3, 5)).astype(np.float32)
    y = rng.standard_normal(5).astype(np.float32)
    z = rng.standard_normal((5, 3)).astype(np.float32)
    w = np.array([0, 1, -1, 7, 2 ** 31 - 1, -(2 ** 31)], np.int32)
    ib, ia, add, sub, sel, neg, ab = oracle_run(prog, [x, y, z, w])
    assert np.array_equal(ib, np.broadcast_to(np.arange(5, dtype=np.int32), (3, 5)))
    assert np.array_equal(ia, np.broadcast_to(np.arange(3, dtype=np.float32)[:, None], (3, 5)))
    for i in range(3):
        for j in range(5):
            assert add[i, j] == np.float32(x[i, j] + y[j])
            assert sub[i, j] == np.float32(x[i, j] - z[j, i])
            assert sel[i, j] == (x[i, j] if x[i, j] < z[j, i] else -z[j, i])
    assert [int(v) for v in neg] == [_wrap(-int(v), "i32") for v in w]
    assert [int(v) for v in ab] == [_wrap(abs(int(v)), "i32") for v in w]


@pytest.mark.parametrize("dtype", ["i32", "u64", "f32", "f64"])
def test_sum_with_an_init_adds_it_once(dtype):
    """reduce(x, init, sum) is init + x_0 + x_1 + ... (a fold from the init, reduction.zig:1140-1155):
    the init enters once per output, whatever the reduced extent. Small integers keep the float sums
    exact."""
    npd = T.NUMPY_DTYPE[dtype]
    x = (np.arange(6 * 50) % 13).astype(npd).reshape(6, 50)
    init = 1000

    def body(b, a):
        c = b.full(dtype, init) if dtype[0] in "iu" else b.full_float(T.Type(dtype, ()), float(init))
        return [a[0].reduce(c, "sum", "c"), a[0].reduce(c, "sum", "r")]
    rows, cols = oracle_run(T.define("si", [T.spec(dtype, r=6, c=50)], body), [x])
    assert np.array_equal(rows, (x.astype(np.float64).sum(axis=1) + init).astype(npd))
    assert np.array_equal(cols, (x.astype(np.float64).sum(axis=0) + init).astype(npd))
