"""Elementwise (map) kernels: four consecutive elements per thread when the innermost extent is a
multiple of 4, with operands read at `rest + c` loaded as one vector (non-temporal when read once);
otherwise one element per thread. Elementwise arithmetic without transcendentals is bit-exact with
the oracle (runCpu's per-operation arithmetic; src/preparation/kernelization/lowering/elementwise.zig);
the device's transcendentals are checked against float64 elsewhere."""
import numpy as np
import pytest

from accy_amd import hip
from accy_amd import tensor as T
from accy_amd import workloads as W
from conftest import hip_run, oracle_run

F32 = T.Type("f32", ())


def mixed(rows, cols):
    """Each element size (i1 / u8 storage 1 B, bf16 2 B, f32 and i32 4 B, f64 8 B), a row operand
    broadcast over the rows, and a transposed operand (innermost stride not 1: element loads)."""
    def body(b, a):
        x, y, row, h, d, k, xt = a
        s = x.mul(y).add(row).mul(x)
        m = x.compare("gt", y)
        return [s, m, m.select(x, y), h.add(h).mul(h), d.mul(d).add(d), k.add(k),
                x.add(xt)]
    specs = [T.spec("f32", r=rows, c=cols), T.spec("f32", r=rows, c=cols), T.spec("f32", c=cols),
             T.spec("bf16", r=rows, c=cols), T.spec("f64", r=rows, c=cols), T.spec("i32", r=rows, c=cols),
             T.spec("f32", c=cols, r=rows)]
    return T.define("mixed", specs, body)


def mixed_inputs(rows, cols, seed):
    rng = np.random.default_rng(seed)
    f = lambda *s: rng.standard_normal(s).astype(np.float32)
    return [f(rows, cols), f(rows, cols), f(cols), W.to_dtype(rng.standard_normal((rows, cols)), "bf16"),
            rng.standard_normal((rows, cols)), rng.integers(-2 ** 30, 2 ** 30, (rows, cols)).astype(np.int32),
            f(cols, rows)]


def test_map_kernels_take_four_elements_per_thread():
    src = hip.plan_source(mixed(64, 1024), compile=True)
    assert "for (I i0 = " in src and "accy::ld_quad_stream(" in src
    # the row operand is shared by all rows: a plain vector load
    assert "*(const accy::Quad<float>*)(" in src
    # an innermost extent that is not a multiple of 4: one element per thread
    src = hip.plan_source(mixed(8, 30), compile=True)
    assert "for (I i0 = " not in src and "for (I i = " in src


@pytest.mark.gpu
@pytest.mark.parametrize("rows,cols", [(64, 1024), (3, 8), (8, 30), (1, 4), (257, 132)])
def test_map_kernels_bit_exact(rows, cols):
    prog, ins = mixed(rows, cols), mixed_inputs(rows, cols, seed=rows * 1000 + cols)
    got, ref = hip_run(prog, ins), oracle_run(prog, ins)
    for i, (g, r) in enumerate(zip(got, ref)):
        assert np.array_equal(g, r, equal_nan=True), f"output {i}"


@pytest.mark.gpu
def test_large_copy_through_the_vector_map():
    n = 1 << 26
    prog = T.define("copy", [T.spec("f32", n=n)], lambda b, a: a[0].mul(b.full_float(F32, 1.0)))
    x = np.random.default_rng(3).standard_normal(n).astype(np.float32)
    assert np.array_equal(hip_run(prog, [x])[0], x)


def test_transposes_are_copied_through_lds_tiles():
    p = T.define("tr", [T.spec("f32", r=256, c=512)], lambda b, a: b.transpose(a[0], [1, 0]))
    src = hip.plan_source(p, compile=True)
    assert "// permute:" in src and "tile[64][65]" in src
    assert "ext_vector_type(4)" in src           # extents and strides multiples of 4: 4 elements per access
    # 16 bytes per lane access for small elements when the extents allow it
    p = T.define("tr8", [T.spec("u8", r=512, c=272)], lambda b, a: b.transpose(a[0], [1, 0]))
    assert "ext_vector_type(16)" in hip.plan_source(p, compile=True)
    p = T.define("tr16", [T.spec("bf16", r=200, c=1000)], lambda b, a: b.transpose(a[0], [1, 0]))
    assert "ext_vector_type(8)" in hip.plan_source(p, compile=True) and "u32_t tile[64][33]" in hip.plan_source(p)
    p = T.define("odd", [T.spec("f32", r=256, c=510)], lambda b, a: b.transpose(a[0], [1, 0]))
    src = hip.plan_source(p, compile=True)
    assert "// permute:" in src and "ext_vector_type" not in src
    # the innermost axis contiguous in the source already: the vector map
    p = T.define("same", [T.spec("f32", a=4, b=64, c=128)], lambda b, a: b.transpose(a[0], [1, 0, 2]))
    assert "// permute:" not in hip.plan_source(p)
    # 2^24 tiles of 256 threads would pass 2^32 work items in one launch: the grid-strided map
    p = T.define("huge", [T.spec("u8", r=1 << 18, c=1 << 18)], lambda b, a: b.transpose(a[0], [1, 0]))
    assert "// permute:" not in hip.plan_source(p) and "// map:" in hip.plan_source(p)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,dims,perm", [
    ("f32", (("r", 1000), ("c", 3000)), (1, 0)),
    ("bf16", (("a", 4), ("b", 300), ("c", 130)), (2, 0, 1)),
    ("f64", (("a", 3), ("b", 65), ("c", 70)), (0, 2, 1)),
    ("i32", (("a", 2), ("b", 3), ("c", 100), ("d", 64)), (3, 1, 0, 2)),
    ("i1", (("r", 77), ("c", 129)), (1, 0)),
    ("u8", (("r", 516), ("c", 260)), (1, 0)),
    ("bf16", (("r", 100), ("c", 4096)), (1, 0)),
    ("f64", (("a", 2), ("b", 128), ("c", 68)), (0, 2, 1)),
    ("u8", (("r", 512), ("c", 272)), (1, 0)),                 # 16 per lane access, ragged tiles
    ("bf16", (("r", 200), ("c", 1000)), (1, 0)),              # 8 per lane access
    ("bf16", (("a", 3), ("b", 64), ("c", 136)), (0, 2, 1)),
    ("i16", (("r", 128), ("c", 72)), (1, 0)),                 # two 16-bit elements per LDS word
    ("f16", (("a", 2), ("b", 200), ("c", 64)), (2, 0, 1)),
])
def test_transposes_bit_exact(dtype, dims, perm):
    p = T.define("perm", [T.spec(dtype, *dims)], lambda b, a: b.transpose(a[0], list(perm)))
    rng = np.random.default_rng(len(dims) * 10 + perm[0])
    shape = tuple(e for _, e in dims)
    if dtype == "bf16":
        x = W.to_dtype(rng.standard_normal(shape), "bf16")
    elif dtype == "i1":
        x = rng.random(shape) < 0.5
    elif dtype == "u8":
        x = rng.integers(0, 256, shape).astype(np.uint8)
    elif dtype == "i16":
        x = rng.integers(-32768, 32768, shape).astype(np.int16)
    elif dtype == "i32":
        x = rng.integers(-10 ** 9, 10 ** 9, shape).astype(np.int32)
    else:
        x = rng.standard_normal(shape).astype(T.NUMPY_DTYPE[dtype])
    got, ref = hip_run(p, [x])[0], oracle_run(p, [x])[0]
    assert np.array_equal(got, ref) and np.array_equal(ref, np.transpose(x, perm))
