"""Differential test over seeded random programs: elementwise chains, named-axis broadcasts and
transposes (aligned binaries), compare / select, reductions over one or two axes, extent-changing
reshapes (split / merge) and the `broadcast` op (a splat or an equal-size copy), in f32 and i32, on extents that are and are not multiples of four. Each program runs on the target and on the
oracle (the runCpu restatement): integer results bit-exact; f32 results within 1e-5 of the largest
magnitude of the output (reductions may be associated differently, and the values stay in a moderate
range: no exp / log, divisions by |x| + 1). The same for random contraction programs (matrix-core
and serial-k paths) and random scans (two carries, elementwise chains and folds in the body).
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
            op = str(rng.choice(["add", "sub", "mul", "max", "min", "neg", "abs", "div", "select", "sum", "rmax",
                                 "split", "merge", "splat"]))
            names = [n for n, _ in x.ty.dims]
            if op == "split":
                # An extent-changing reshape pair (builder.zig:438-470): axis n split as (hi, lo), then
                # merged back in the order (lo, hi), which permutes n's elements.
                cand = [(n, e, p) for n, e in x.ty.dims for p in (2, 3, 4, 5, 13) if e % p == 0 and e > p]
                if cand:
                    n, e, p = cand[int(rng.integers(len(cand)))]
                    v = x.split(n, (n + "h", p), (n + "l", e // p)).merge((n + "l", n + "h"), n)
                else:
                    v = x.neg()
            elif op == "merge":
                # Two axes merged in a random order, then either split back (a transpose of x through
                # reshapes) or reduced over the merged axis.
                if len(names) >= 2:
                    u, w = (str(t) for t in rng.choice(names, size=2, replace=False))
                    m = x.merge((u, w), "m")
                    if rng.random() < 0.5 or len(names) == 2:
                        v = m.split("m", (u, x.ty.dims[names.index(u)][1]), (w, x.ty.dims[names.index(w)][1]))
                    else:
                        v = m.sum("m") if rng.random() < 0.5 else m.max("m")
                else:
                    v = x.abs()
            elif op == "splat":
                # The `broadcast` op (builder.zig:487): a one-element value spread over y's axes, or an
                # equal-size value copied in order into reversed axes.
                if rng.random() < 0.5:
                    v = b.broadcast(x.max(tuple(names)), y.ty.dims).add(y)
                else:
                    v = b.broadcast(x, tuple(reversed(x.ty.dims)))
            elif op in ("add", "sub", "mul", "max", "min"):
                v = getattr(x, op)(y)
            elif op == "neg":
                v = x.neg()
            elif op == "abs":
                v = x.abs()
            elif op == "div":
                v = x.div(y.abs().add(one)) if dtype == "f32" else x.div(y.abs().add(one))
            elif op == "select":
                v = x.compare("gt", y).select(x, y.neg())
            elif not names:
                v = x.neg()                       # nothing left to reduce over
            else:
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


def _scan_program(seed, dtype):
    """A scan over two carries, x [a, b] and s [b], for a random number of steps (0-6): x is updated by
    a random chain of elementwise operations with s broadcast over a, s by a fold of x over a. Read
    back: the loop, a projection of s, and a value computed from both after the loop."""
    rng = np.random.default_rng(2000 + seed)
    ea, eb = (int(rng.choice([1, 5, 64, 130, 1000])) for _ in range(2))
    length = int(rng.integers(0, 7))
    scalar = T.Type(dtype, ())
    ops = [str(rng.choice(["add_s", "sub_s", "max_s", "min_s", "neg", "half", "abs"])) for _ in range(int(rng.integers(1, 5)))]
    fold = str(rng.choice(["sum", "max", "min"]))

    def const(bb, v):
        return bb.full_float(scalar, v) if dtype == "f32" else bb.full("i32", int(v))

    def step(bb, c):
        x, s = c
        for op in ops:
            if op == "add_s":
                x = x.add(s)
            elif op == "sub_s":
                x = x.sub(s)
            elif op == "max_s":
                x = x.max(s)
            elif op == "min_s":
                x = x.min(s)
            elif op == "neg":
                x = x.neg()
            elif op == "abs":
                x = x.abs()
            else:   # keep magnitudes bounded: f32 halves, i32 clamps
                x = x.mul(const(bb, 0.5)) if dtype == "f32" else x.max(const(bb, -10 ** 6)).min(const(bb, 10 ** 6))
        r = getattr(x, fold)("a")
        if dtype == "f32" and fold == "sum":
            r = r.mul(const(bb, 1.0 / ea))
        return [x, s.add(r) if fold == "sum" else s.max(r) if fold == "max" else s.min(r)]

    def body(b, a):
        loop = b.scan(length, [a[0], a[1]], step)
        s = b.projection(loop, 1)
        return [loop, s, loop.sum("a").add(s)]

    prog = T.define(f"scan{seed}", [T.spec(dtype, a=ea, b=eb), T.spec(dtype, b=eb)], body)
    if dtype == "f32":
        inputs = [rng.standard_normal((ea, eb)).astype(np.float32), rng.standard_normal(eb).astype(np.float32)]
    else:
        inputs = [rng.integers(-1000, 1000, (ea, eb)).astype(np.int32), rng.integers(-1000, 1000, eb).astype(np.int32)]
    return prog, inputs


@pytest.mark.parametrize("seed", range(4))
def test_random_scan_programs_plan_and_compile(seed):
    for dtype in ("f32", "i32"):
        prog, _ = _scan_program(seed, dtype)
        assert "// loop " in hip.plan_source(prog, compile=True)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(16))
@pytest.mark.parametrize("dtype", ["f32", "i32"])
def test_random_scan_programs_match_the_oracle(seed, dtype):
    prog, inputs = _scan_program(seed, dtype)
    print(f"scan seed {seed} {dtype}: inputs {[t.shape for t in prog.input_types()]}", flush=True)
    got, ref = hip_run(prog, inputs), oracle_run(prog, inputs)
    for i, (g, r) in enumerate(zip(got, ref)):
        if dtype == "i32":
            assert np.array_equal(g, r), f"output {i}"
        else:
            # f32 sums are associated differently on the target; the carries feed them back each step
            scale = float(np.abs(r).max()) if r.size else 0.0
            assert np.all(np.abs(g.astype(np.float64) - r) <= 1e-4 * max(scale, 1e-30)), f"output {i}"


def test_random_programs_draw_reshapes_and_broadcasts():
    """At least a third of the seeds of the elementwise family carry an extent-changing reshape
    (split / merge) or a `broadcast` op, so the GPU differential test covers them."""
    drawn = 0
    for dtype in ("f32", "i32"):
        for seed in SEEDS:
            prog, _ = _program(seed, dtype)
            ops = prog.operations
            drawn += any(op.kind == "broadcast" or (op.kind == "reshape" and prog.type_of(op.args[0]).shape
                                                    != op.result.shape) for op in ops)
    assert drawn >= 2 * len(SEEDS) / 3, drawn
