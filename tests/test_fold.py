"""Reductions over leading or middle axes with few outputs and a long reduced range (the fold class,
src/preparation/kernelization/lowering/reduction.zig:839-878).

One serial fold per output cannot fill the GPU there, so the target folds the range in chunks and then
each output's chunk partials in order from the program's init. The chunk identity makes integer folds
and float max / min bit-identical to runCpu's serial fold (NaN is the absent element of the NaN-skipping
max / min; -0 the identity of a float sum); a float sum is associated differently, so it is checked
against the classical bound for any summation order, |error| <= (n - 1) u sum|x| with u = 2^-24 (plus
the final rounding for 16-bit outputs). Small folds keep the serial loop (test_gpu_parity).
"""
import numpy as np
import pytest

from accy_amd import hip
from accy_amd import tensor as T
from accy_amd import workloads as W
from conftest import hip_run, oracle_run, to_f32

U = 2.0 ** -24


def colsum(dtype, r, c, reducer="sum"):
    return T.define("col", [T.spec(dtype, r=r, c=c)], lambda b, a: getattr(a[0], reducer)("r"))


def test_long_leading_folds_are_chunked_and_small_ones_serial():
    src = hip.plan_source(colsum("f32", 8192, 4096), compile=True)
    assert "// fold:%2 chunks grid" in src and "float acc = -0.0f;" in src
    src = hip.plan_source(colsum("f32", 8192, 4096, "max"), compile=True)
    assert '__builtin_nanf("")' in src
    assert "chunks" not in hip.plan_source(colsum("f32", 300, 77))          # small: serial
    assert "chunks" not in hip.plan_source(colsum("i16", 8192, 4096))       # no identity kept: serial
    assert "chunks" not in hip.plan_source(colsum("f32", 64, 1 << 18))      # many outputs: serial


def _sum_bound(x64, n, axis=0):
    return (n - 1) * U * np.abs(x64).sum(axis=axis)


@pytest.mark.gpu
def test_chunked_f32_sum_within_the_summation_bound():
    r, c = 8192, 4096
    x = np.random.default_rng(1).standard_normal((r, c)).astype(np.float32)
    prog = colsum("f32", r, c)
    got, ref = hip_run(prog, [x])[0].astype(np.float64), oracle_run(prog, [x])[0].astype(np.float64)
    exact = x.astype(np.float64).sum(axis=0)
    bound = _sum_bound(x.astype(np.float64), r)
    assert np.all(np.abs(got - exact) <= bound) and np.all(np.abs(ref - exact) <= bound)
    # positive terms (no cancellation): within the reductions' 1e-5 relative bound of the serial fold
    y = np.abs(x)
    got, ref = hip_run(prog, [y])[0], oracle_run(prog, [y])[0]
    assert np.all(np.abs(got.astype(np.float64) - ref) <= 1e-5 * np.abs(ref.astype(np.float64)))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_chunked_16bit_sum(dtype):
    r, c = 4096, 2048
    x = W.to_dtype(np.abs(np.random.default_rng(2).standard_normal((r, c))), dtype)
    prog = colsum(dtype, r, c)
    got, ref = to_f32(hip_run(prog, [x])[0], dtype), to_f32(oracle_run(prog, [x])[0], dtype)
    # f32 accumulation in either order, one rounding to 8 (11) bits at the end: one 16-bit step apart
    step = 2.0 ** -7 if dtype == "bf16" else 2.0 ** -10
    assert np.all(np.abs(got - ref) <= step * np.abs(ref))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,reducer", [("i32", "sum"), ("i32", "max"), ("i32", "min"), ("i64", "sum"),
                                           ("u32", "sum")])
def test_chunked_integer_folds_bit_exact(dtype, reducer):
    r, c = 4096, 1024
    nd = np.dtype(T.NUMPY_DTYPE[dtype])
    info = np.iinfo(nd)
    x = np.random.default_rng(3).integers(info.min // 2, info.max // 2, (r, c), dtype=nd, endpoint=True)
    prog = colsum(dtype, r, c, reducer)
    assert "chunks" in hip.plan_source(prog)
    assert np.array_equal(hip_run(prog, [x])[0], oracle_run(prog, [x])[0])   # sums wrap


@pytest.mark.gpu
@pytest.mark.parametrize("reducer", ["max", "min"])
@pytest.mark.parametrize("r,c", [(4096, 1024), (300, 16)])   # chunked, serial
def test_float_max_min_folds_bit_exact_with_nan_inf_and_signed_zeros(reducer, r, c):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((r, c)).astype(np.float32)
    x[:, 0] = np.nan                                   # all NaN: NaN
    x[::7, 1] = np.nan                                 # NaN skipped
    x[:, 2] = 0.0
    x[rng.integers(0, r, 50), 2] = -0.0               # +0 / -0 ties: the later element's sign
    x[:, 3] = -0.0
    x[:, 4] = -np.inf if reducer == "max" else np.inf  # all infinite
    x[100, 5] = np.inf
    x[200, 5] = -np.inf
    x[:, 6] = np.nan
    x[r - 7, 6] = 1.5                                  # one number among NaNs
    prog = colsum("f32", r, c, reducer)
    assert ("chunks" in hip.plan_source(prog)) == (r == 4096)
    got, ref = hip_run(prog, [x])[0], oracle_run(prog, [x])[0]
    assert np.array_equal(got.view(np.uint32)[~np.isnan(ref)], ref.view(np.uint32)[~np.isnan(ref)])
    assert np.array_equal(np.isnan(got), np.isnan(ref))


@pytest.mark.gpu
def test_chunked_fold_starts_from_the_program_init_and_spans_several_axes():
    def body(b, a):
        init = b.full_float(T.Type("f32", ()), 5.0)
        return [a[0].reduce(init, "sum", ("a", "b")), a[0].reduce(b.full_float(T.Type("f32", ()), 3.0), "max", ("a", "b"))]
    prog = T.define("mid", [T.spec("f32", a=64, b=256, c=512)], body)
    assert "chunks" in hip.plan_source(prog)
    x = np.abs(np.random.default_rng(5).standard_normal((64, 256, 512))).astype(np.float32)
    got, ref = hip_run(prog, [x]), oracle_run(prog, [x])
    assert np.all(np.abs(got[0].astype(np.float64) - ref[0]) <= 1e-5 * np.abs(ref[0].astype(np.float64)))
    assert np.array_equal(got[1], ref[1])
    assert np.all(ref[1] >= 3.0)
