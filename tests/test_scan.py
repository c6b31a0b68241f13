"""Scans (builder.zig:899-990; runCpu's loop, src/tensor/lower.zig:119-167) on the gfx950 target.

The target runs a scan as a host loop: the body's own plan is launched `length` times, reading one
set of carry buffers and writing the other. The CPU tests pin the oracle's scan against closed forms
and check the planned loop; the GPU tests compare the target with the oracle — bit-exact for
elementwise and integer bodies, relative 1e-5 for the f32 row sums, normwise 1e-5 for the f32
contraction carried through the loop.
"""
import numpy as np
import pytest

from accy_amd import hip
from accy_amd import tensor as T
from conftest import assert_normwise, assert_rel, hip_run, oracle_run, out_arrays

F32 = T.Type("f32", ())


def doubling(length):
    return T.define("double", [T.spec("f32", v=1000)],
                    lambda b, a: b.scan(length, [a[0]], lambda bb, c: [c[0].add(c[0])]))


def two_carries(length):
    """Carry 0 relaxes towards 2 (y/2 + 1); carry 1 adds up the row sums of carry 0 it saw; the
    final sums are read twice, once scaled and exponentiated."""
    def step(bb, c):
        y, s = c
        return [y.mul(bb.full_float(F32, 0.5)).add(bb.full_float(F32, 1.0)), s.add(y.sum("c"))]

    def body(b, a):
        loop = b.scan(length, [a[0], a[1]], step)
        return [loop, b.projection(loop, 1), b.projection(loop, 1).mul(b.full_float(F32, 1e-3)).exp()]
    return T.define("relax", [T.spec("f32", r=64, c=1000), T.spec("f32", r=64)], body)


def nested(outer, inner):
    def body(b, a):
        def outer_step(bb, c):
            return [bb.scan(inner, [c[0]], lambda b3, d: [d[0].add(b3.full_float(F32, 1.0))])]
        return b.scan(outer, [a[0]], outer_step)
    return T.define("nested", [T.spec("f32", v=333)], body)


def power(length):
    """A·B^length with B passed through unchanged, then a row sum of the result read later."""
    def step(bb, c):
        return [c[0].contract(c[1], "k").rename("n", "k"), c[1]]

    def body(b, a):
        loop = b.scan(length, [a[0], a[1]], step)
        return [loop, loop.sum("k")]
    return T.define("power", [T.spec("f32", m=64, k=64), T.spec("f32", k=64, n=64)], body)


def integer_counter(length):
    """Three carries, the last never read: an i32 doubling, an i32 step counter and an f32 scale."""
    def step(bb, c):
        return [c[0].add(c[0]), c[1].add(bb.full("i32", 1)), c[2].mul(bb.full_float(F32, 3.0))]

    def body(b, a):
        loop = b.scan(length, [a[0], a[1], a[2]], step)
        return [loop, b.projection(loop, 1)]
    return T.define("count", [T.spec("i32", j=100), T.spec("i32"), T.spec("f32", j=8)], body)


def _relax_inputs(seed=5):
    rng = np.random.default_rng(seed)
    return [rng.standard_normal((64, 1000)).astype(np.float32), np.zeros(64, np.float32)]


def _power_inputs(seed=9):
    rng = np.random.default_rng(seed)
    a = rng.standard_normal((64, 64)).astype(np.float32)
    b = (rng.standard_normal((64, 64)) / 8.0).astype(np.float32)
    return [a, b]


# ---- the oracle's scan against closed forms ----

@pytest.mark.parametrize("length", [0, 1, 5])
def test_oracle_scan_doubling_closed_form(length):
    x = np.linspace(-3, 3, 1000).astype(np.float32)
    assert np.array_equal(oracle_run(doubling(length), [x])[0], x * np.float32(2.0 ** length))


def test_oracle_scan_carries_and_projections():
    x, s = _relax_inputs()
    out = oracle_run(two_carries(3), [x, s])
    y1 = x * np.float32(0.5) + np.float32(1.0)
    y2 = y1 * np.float32(0.5) + np.float32(1.0)
    y3 = y2 * np.float32(0.5) + np.float32(1.0)
    assert np.array_equal(out[0], y3)
    sums = x.astype(np.float64).sum(1) + y1.astype(np.float64).sum(1) + y2.astype(np.float64).sum(1)
    assert np.allclose(out[1], sums, rtol=1e-5, atol=1e-3)
    assert np.allclose(out[2], np.exp(out[1].astype(np.float64) * 1e-3), rtol=1e-6)
    zero = oracle_run(two_carries(0), [x, s])
    assert np.array_equal(zero[0], x) and np.array_equal(zero[1], s)


def test_oracle_nested_scan_and_pass_through_carry():
    x = np.arange(333, dtype=np.float32) - 100
    assert np.array_equal(oracle_run(nested(3, 4), [x])[0], x + 12)
    a, b = _power_inputs()
    out = oracle_run(power(3), [a, b])
    want = a.astype(np.float64) @ np.linalg.matrix_power(b.astype(np.float64), 3)
    assert np.allclose(out[0], want, rtol=1e-4, atol=1e-4)
    i, n, f = np.arange(100, dtype=np.int32), np.array(7, np.int32), np.ones(8, np.float32)
    got = oracle_run(integer_counter(6), [i, n, f])
    assert np.array_equal(got[0], i * 64) and int(got[1]) == 13


# ---- the planned loop (host only) ----

def test_scan_plans_a_loop_over_the_body_and_compiles():
    src = hip.plan_source(two_carries(6), compile=True)
    assert "// loop 6 times over 2 carries {" in src
    body = src[src.index("{\n"):src.index("// }")]
    assert "__global__" in body          # the body's kernels are planned and compiled
    src = hip.plan_source(nested(3, 4), compile=True)
    assert "// loop 3 times over 1 carries {" in src and "  // loop 4 times over 1 carries {" in src


# ---- the target against the oracle ----

@pytest.mark.gpu
@pytest.mark.parametrize("length", [0, 1, 5])
def test_scan_doubling_on_gpu(length):
    x = np.linspace(-3, 3, 1000).astype(np.float32)
    prog = doubling(length)
    assert np.array_equal(hip_run(prog, [x])[0], oracle_run(prog, [x])[0])


@pytest.mark.gpu
@pytest.mark.parametrize("length", [0, 6])
def test_scan_carries_projections_and_later_readers_on_gpu(length):
    prog, inputs = two_carries(length), _relax_inputs()
    got, ref = hip_run(prog, inputs), oracle_run(prog, inputs)
    assert np.array_equal(got[0], ref[0])
    assert_rel(got[1], ref[1], 1e-5)
    assert_rel(got[2], ref[2], 1e-5)


@pytest.mark.gpu
def test_nested_scan_on_gpu():
    x = np.arange(333, dtype=np.float32) - 100
    prog = nested(3, 4)
    assert np.array_equal(hip_run(prog, [x])[0], oracle_run(prog, [x])[0])


@pytest.mark.gpu
def test_scan_with_contraction_and_pass_through_carry_on_gpu():
    prog, inputs = power(3), _power_inputs()
    got, ref = hip_run(prog, inputs), oracle_run(prog, inputs)
    assert_normwise(got[0], ref[0], 1e-5)
    assert_rel(got[1], ref[1], 1e-4)


@pytest.mark.gpu
def test_scan_integer_carries_and_unread_carry_on_gpu():
    i, n, f = np.arange(100, dtype=np.int32), np.array(7, np.int32), np.ones(8, np.float32)
    prog = integer_counter(6)
    got, ref = hip_run(prog, [i, n, f]), oracle_run(prog, [i, n, f])
    assert np.array_equal(got[0], ref[0]) and np.array_equal(got[1], ref[1])


@pytest.mark.gpu
def test_scan_program_invoked_repeatedly_reuses_its_carry_buffers():
    prog, inputs = two_carries(4), _relax_inputs(seed=11)
    ref = oracle_run(prog, inputs)
    with hip.Hip(prog) as p:
        for _ in range(3):
            got = out_arrays(prog)
            p.launch(inputs, got)
            assert np.array_equal(got[0], ref[0])
            assert_rel(got[1], ref[1], 1e-5)


# ---- long scans ----

@pytest.mark.gpu
@pytest.mark.parametrize("case", ["relax", "power", "count"])
def test_long_scans_invoked_repeatedly(case):
    """Loops of 40-100 iterations (relaxation 100, matrix power 40, counter 70) against the oracle,
    the same executor invoked three times with
    another program's work and a synchronisation between the invocations; every invocation equals
    the first bit for bit."""
    if case == "relax":
        prog, inputs = two_carries(100), _relax_inputs(seed=21)
    elif case == "power":
        prog, inputs = power(40), _power_inputs(seed=22)
        inputs[1] = inputs[1] * np.float32(0.9)  # keep A B^40 finite
    else:
        i, n, f = np.arange(100, dtype=np.int32), np.array(7, np.int32), np.ones(8, np.float32)
        prog, inputs = integer_counter(70), [i, n, f]
    ref = oracle_run(prog, inputs)
    other = doubling(3)
    x = np.linspace(-1, 1, 1000).astype(np.float32)
    first = None
    with hip.Hip(prog) as p:
        for _ in range(3):
            got = out_arrays(prog)
            p.launch(inputs, got)
            if first is None:
                first = [np.array(g, copy=True) for g in got]
            for g, e in zip(got, first):
                assert np.array_equal(np.asarray(g).reshape(-1).view(np.uint8), np.asarray(e).reshape(-1).view(np.uint8))
            hip_run(other, [x])  # other work between the invocations
    if case == "relax":
        assert np.array_equal(got[0], ref[0])
        assert_rel(got[1], ref[1], 1e-5)
    elif case == "power":
        assert_normwise(got[0], ref[0], 1e-4)
    else:
        assert np.array_equal(got[0], ref[0]) and np.array_equal(got[1], ref[1])
