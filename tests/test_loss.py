"""sparse_cross_entropy (builder.zig:699-741) in the expanded form runCpu lowers it to
(src/tensor/lower.zig:914-1003): loss = log(sum(exp(x - m))) - sum(select(iota == target, x - m, 0))
over the class axis, m the row max folded from the lowest finite value (lower.zig:1005-1029).

The reference holds no fixture for this op, so the oracle is pinned by closed forms: the float64
log-softmax lse(x) - x[t] for targets in range, lse(x) - max(x) for targets out of range (no class
matches), NaN for an all -inf row with a target in range and -inf without one. The GPU tests compare
the target with the oracle: f32 normwise 1e-5 (per element with a floor of 1e-3 of the largest loss),
bf16 / f16 2e-2, special values (NaN, +-inf) at the same positions.
"""
import numpy as np
import pytest

from accy_amd import hip
from accy_amd import tensor as T
from conftest import assert_normwise, hip_run, oracle_run, to_f32


def loss_program(rows, classes, dtype="f32", class_axis_first=False):
    if class_axis_first:
        specs = [T.spec(dtype, cls=classes, row=rows), T.spec("i32", row=rows)]
    else:
        specs = [T.spec(dtype, row=rows, cls=classes), T.spec("i32", row=rows)]
    return T.define("ce", specs, lambda b, a: a[0].sparse_cross_entropy_loss(a[1], "cls"))


def mean_loss_program(rows, classes):
    """The training objective: the mean of the per-row losses."""
    def body(b, a):
        loss = a[0].sparse_cross_entropy_loss(a[1], "cls")
        return [loss.sum("row").mul(b.full_float(T.Type("f32", ()), 1.0 / rows)), loss]
    return T.define("mean_ce", [T.spec("f32", row=rows, cls=classes), T.spec("i32", row=rows)], body)


def _inputs(rows, classes, seed, dtype="f32", scale=3.0, out_of_range=()):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((rows, classes)) * scale).astype(np.float32)
    t = rng.integers(0, classes, rows).astype(np.int32)
    for i, bad in enumerate(out_of_range):
        t[i] = bad
    if dtype == "bf16":
        x = (x.view(np.uint32) >> 16).astype(np.uint16)
    elif dtype == "f16":
        x = x.astype(np.float16)
    return x, t


def _closed_form(x64, t):
    """float64 loss per row: lse - x[t] in range, lse - max out of range."""
    m = x64.max(axis=1)
    lse = m + np.log(np.exp(x64 - m[:, None]).sum(axis=1))
    rows = np.arange(x64.shape[0])
    hit = (t >= 0) & (t < x64.shape[1])
    picked = np.where(hit, x64[rows, np.clip(t, 0, x64.shape[1] - 1)], m)
    return lse - picked


def _same_specials(got, ref):
    g, r = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    assert np.array_equal(np.isnan(g), np.isnan(r))
    assert np.array_equal(np.isposinf(g), np.isposinf(r)) and np.array_equal(np.isneginf(g), np.isneginf(r))
    return np.isfinite(r)


# ---- the oracle against closed forms ----

def test_oracle_loss_matches_float64_log_softmax():
    x, t = _inputs(37, 1000, seed=1, out_of_range=(-1, 1000, 5000))
    got = oracle_run(loss_program(37, 1000), [x, t])[0]
    want = _closed_form(x.astype(np.float64), t)
    assert np.allclose(got, want, rtol=1e-5, atol=2e-5)
    # rows 0-2 have no matching class: the loss is lse - max
    m = x[:3].astype(np.float64).max(axis=1)
    lse = m + np.log(np.exp(x[:3].astype(np.float64) - m[:, None]).sum(axis=1))
    assert np.allclose(got[:3], lse - m, rtol=1e-5, atol=2e-5)


def test_oracle_loss_class_axis_first_equals_transposed():
    x, t = _inputs(7, 50, seed=2)
    a = oracle_run(loss_program(7, 50), [x, t])[0]
    b = oracle_run(loss_program(7, 50, class_axis_first=True), [np.ascontiguousarray(x.T), t])[0]
    assert np.array_equal(a, b)


def test_oracle_loss_special_rows():
    x, t = _inputs(4, 16, seed=3)
    x[0, :] = -np.inf          # m stays at -floatMax: log(0) - (-inf) is NaN
    x[1, :] = -np.inf
    t[1] = 99                  # ... and without a target: log(0) - 0 = -inf
    x[2, 5] = np.nan           # NaN in the row: the sum of exponentials is NaN
    x[3, 7] = np.inf           # +inf: inf - inf in the shifted row
    got = oracle_run(loss_program(4, 16), [x, t])[0]
    assert np.isnan(got[0]) and np.isneginf(got[1]) and np.isnan(got[2]) and np.isnan(got[3])


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_oracle_loss_16bit_against_float64(dtype):
    x, t = _inputs(16, 300, seed=4, dtype=dtype)
    got = to_f32(oracle_run(loss_program(16, 300, dtype), [x, t])[0], dtype)
    want = _closed_form(to_f32(x, dtype).astype(np.float64), t)
    # each shifted value, exponential and the logarithm round to 8 (bf16) or 11 (f16) bits
    tol = 2e-2 if dtype == "bf16" else 4e-3
    assert np.allclose(got, want, rtol=tol, atol=tol * np.abs(want).max())


def test_loss_plans_one_row_kernel_and_compiles():
    src = hip.plan_source(loss_program(64, 1000), compile=True)
    assert src.count("__global__") == 1 and "// row:" in src
    src = hip.plan_source(loss_program(8, 50, "bf16", class_axis_first=True), compile=True)
    assert "__global__" in src


# ---- the target against the oracle ----

@pytest.mark.gpu
@pytest.mark.parametrize("rows,classes", [(64, 1000), (256, 32000), (3, 5), (1, 1)])
def test_loss_f32_matches_oracle(rows, classes):
    x, t = _inputs(rows, classes, seed=rows + classes, out_of_range=(-3,) if rows > 1 else ())
    prog = loss_program(rows, classes)
    got, ref = hip_run(prog, [x, t])[0], oracle_run(prog, [x, t])[0]
    assert_normwise(got, ref, 1e-5)


@pytest.mark.gpu
def test_loss_class_axis_first_matches_oracle():
    x, t = _inputs(96, 777, seed=8)
    xt = np.ascontiguousarray(x.T)
    prog = loss_program(96, 777, class_axis_first=True)
    got, ref = hip_run(prog, [xt, t])[0], oracle_run(prog, [xt, t])[0]
    assert_normwise(got, ref, 1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_loss_16bit_matches_oracle(dtype):
    x, t = _inputs(128, 4096, seed=9, dtype=dtype)
    prog = loss_program(128, 4096, dtype)
    got, ref = hip_run(prog, [x, t])[0], oracle_run(prog, [x, t])[0]
    assert_normwise(got, ref, 2e-2, dtype)


@pytest.mark.gpu
def test_loss_special_rows_match_oracle():
    x, t = _inputs(6, 16, seed=3)
    x[0, :] = -np.inf
    x[1, :] = -np.inf
    t[1] = 99
    x[2, 5] = np.nan
    x[3, 7] = np.inf
    t[4] = -1
    prog = loss_program(6, 16)
    got, ref = hip_run(prog, [x, t])[0], oracle_run(prog, [x, t])[0]
    finite = _same_specials(got, ref)
    assert_normwise(got[finite], ref[finite], 1e-5)


@pytest.mark.gpu
def test_mean_loss_objective_matches_oracle():
    x, t = _inputs(512, 2048, seed=12)
    prog = mean_loss_program(512, 2048)
    got, ref = hip_run(prog, [x, t]), oracle_run(prog, [x, t])
    assert_normwise(got[1], ref[1], 1e-5)
    assert abs(float(got[0]) - float(ref[0])) <= 1e-5 * abs(float(ref[0]))
