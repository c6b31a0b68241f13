"""Differential test over seeded random programs: elementwise chains, named-axis broadcasts and
transposes (aligned binaries), compare / select, and reductions over one or two axes, in f32 and
i32, on extents that are and are not multiples of four. Each program runs on the target and on the
oracle (the runCpu restatement): integer results bit-exact; f32 results within 1e-5 of the largest
magnitude of the output (reductions may be associated differently, and the values stay in a moderate
range: no exp / log, divisions by |x| + 1).
"""
import numpy as np
import pytest

from accy_amd import hip
from accy_amd import tensor as T
from accy_amd import workloads as W
from conftest import assert_normwise, hip_run, oracle_run


def _program(seed, dtype):
    rng = np.random.default_rng(seed)
    ext = {n: int(rng.choice([1, 3, 4, 7, 16, 33, 64, 130])) for n in "abc"}
    specs = [T.spec(dtype, a=ext["a"], b=ext["b"]), T.spec(dtype, b=ext["b"], c=ext["c"]), T.spec(dtype, c=ext["c"], a=ext["a"])]

    def body(b, args):
        vals = list(args)
        outs = []
        one = b.full_float(T.Type("f32", ()), 1.0) if dtype == "f32" else b.full("i32", 1)
        for _ in range(int(rng.integers(3, 8))):
            x = vals[int(rng.integers(len(vals)))]
            y = vals[int(rng.integers(len(vals)))]
            op = str(rng.choice(["add", "sub", "mul", "max", "min", "neg", "abs", "div", "select", "sum", "rmax"]))
            if op in ("add", "sub", "mul", "max", "min"):
                v = getattr(x, op)(y)
            elif op == "neg":
                v = x.neg()
            elif op == "abs":
                v = x.abs()
            elif op == "div":
                v = x.div(y.abs().add(one)) if dtype == "f32" else x.div(y.abs().add(one))
            elif op == "select":
                v = x.compare("gt", y).select(x, y.neg())
            else:
                names = [n for n, _ in x.ty.dims]
                k = int(rng.integers(1, len(names) + 1)) if len(names) > 1 else 1
                axes = tuple(rng.choice(names, size=min(k, len(names)), replace=False))
                if len(axes) == len(names):
                    axes = axes[:-1] if len(axes) > 1 else axes
                v = x.sum(axes) if op == "sum" else x.max(axes)
            if dtype == "i32" and op == "mul":
                v = v.max(b.full("i32", -100000)).min(b.full("i32", 100000))   # keep products in range
            vals.append(v)
            if rng.random() < 0.4:
                outs.append(v)
        outs.append(vals[-1])
        return outs

    prog = T.define(f"rand{seed}", specs, body)
    inputs = []
    for t in prog.input_types():
        shape = t.shape
        if dtype == "f32":
            inputs.append(rng.standard_normal(shape).astype(np.float32))
        else:
            inputs.append(rng.integers(-50, 50, shape).astype(np.int32))
    return prog, inputs


SEEDS = list(range(40))


@pytest.mark.parametrize("seed", SEEDS[:10])
def test_random_programs_plan_and_compile(seed):
    for dtype in ("f32", "i32"):
        prog, _ = _program(seed, dtype)
        assert isinstance(hip.plan_source(prog, compile=True), str)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", SEEDS)
@pytest.mark.parametrize("dtype", ["f32", "i32"])
def test_random_programs_match_the_oracle(seed, dtype):
    prog, inputs = _program(seed, dtype)
    print(f"seed {seed} {dtype}: {[t.shape for t in prog.output_types()]}", flush=True)
    got, ref = hip_run(prog, inputs), oracle_run(prog, inputs)
    for i, (g, r) in enumerate(zip(got, ref)):
        if dtype == "i32":
            assert np.array_equal(g, r), f"output {i}"
        else:
            scale = float(np.abs(r).max()) if r.size else 0.0
            assert np.all(np.abs(g.astype(np.float64) - r) <= 1e-5 * max(scale, 1e-30)), f"output {i}"


def _contraction_program(seed, dtype):
    """A[m, k] . B[k, n] on whichever contraction path the extents select (direct-to-LDS MFMA,
    register-staged MFMA with edge guards, or the serial-k dot), followed by random elementwise work
    (some of it fused into the contraction's epilogue), a transposed operand and a reduction."""
    rng = np.random.default_rng(1000 + seed)
    m, k, n = (int(rng.choice([16, 48, 128, 160, 256, 512])) for _ in range(3))
    specs = [T.spec(dtype, m=m, k=k), T.spec(dtype, k=k, n=n), T.spec(dtype, n=n, m=m)]
    scalar = T.Type(dtype, ())

    def body(b, a):
        x, w, c = a
        d = x.contract(w, "k")
        for _ in range(int(rng.integers(0, 4))):
            op = str(rng.choice(["add_c", "mul_half", "max0", "tanh", "sub_c"]))
            if op == "add_c":
                d = d.add(c)                      # c is [n, m]: a transposed operand
            elif op == "sub_c":
                d = d.sub(c)
            elif op == "mul_half":
                d = d.mul(b.full_float(scalar, 0.5))
            elif op == "max0":
                d = d.max(b.full_float(scalar, 0.0))
            else:
                d = d.tanh()
        outs = [d]
        if rng.random() < 0.5:
            outs.append(d.sum(str(rng.choice(["m", "n"]))))
        return outs

    prog = T.define(f"mm{seed}", specs, body)
    inputs = [W.to_dtype(rng.standard_normal(t.shape) * sc, dtype)
              for t, sc in zip(prog.input_types(), (1.0, 1.0 / np.sqrt(k), 1.0))]
    return prog, inputs


@pytest.mark.parametrize("seed", range(6))
def test_random_contraction_programs_plan_and_compile(seed):
    for dtype in ("f32", "bf16"):
        prog, _ = _contraction_program(seed, dtype)
        assert isinstance(hip.plan_source(prog, compile=True), str)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(24))
@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
def test_random_contraction_programs_match_the_oracle(seed, dtype):
    prog, inputs = _contraction_program(seed, dtype)
    print(f"seed {seed} {dtype}: inputs {[t.shape for t in prog.input_types()]}", flush=True)
    got, ref = hip_run(prog, inputs), oracle_run(prog, inputs)
    tol = 1e-3 if dtype == "f32" else 2e-2
    for g, r in zip(got, ref):
        assert_normwise(g, r, tol, dtype, floor=None)
