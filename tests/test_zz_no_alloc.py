"""accy_hip_invoke_device_scratch, the allocation-free entry point, through the C ABI on an MI355X.

Its kernels are the ones accy_hip_invoke_device launches, with every intermediate buffer taken from
the library's static device scratch instead of the program's allocations, so its outputs must equal
invoke_device's bit for bit. Two calls in a row, the second on a smaller program, check that a call
does not depend on what the previous one left in the shared scratch; the programs cover temporaries
between kernels (decoder blocks, up to the full-size C5 block), chunked-fold partials and scan
carries with a body that has its own temporaries. A program whose intermediates exceed the scratch is refused before any launch.
"""
import ctypes

import numpy as np
import pytest

from accy_amd import hip
from accy_amd import tensor as T
from accy_amd import workloads as W

pytestmark = pytest.mark.gpu

F32 = T.Type("f32", ())


def _colsum(rows, cols):
    return T.define("colsum", [T.spec("f32", r=rows, c=cols)], lambda b, a: a[0].sum("r"))


def _scan_with_contraction(length, n):
    """A B^length with a row sum read afterwards: the body's contraction result is a temporary."""
    def step(bb, c):
        return [c[0].contract(c[1], "k").rename("n", "k").mul(bb.full_float(F32, 0.5)), c[1]]

    def body(b, a):
        loop = b.scan(length, [a[0], a[1]], step)
        return [loop, loop.sum("k")]
    return T.define("power", [T.spec("f32", m=n, k=n), T.spec("f32", k=n, n=n)], body)


def _inputs(prog, seed):
    rng = np.random.default_rng(seed)
    out = []
    for t in prog.input_types():
        if t.dtype == "bf16":
            out.append(W.to_dtype(rng.standard_normal(t.shape) * 0.5, "bf16"))
        else:
            out.append(rng.standard_normal(t.shape).astype(T.NUMPY_DTYPE[t.dtype]))
    return out


def _run(session, h, prog, ins, scratch, stream):
    """Device buffers in and out; one invocation (invoke_device or the scratch variant); host copies of
    the outputs."""
    dins = [hip.DeviceBuffer.from_array(x) for x in ins]
    outs = [np.zeros(t.shape, T.NUMPY_DTYPE[t.dtype]) for t in prog.output_types()]
    douts = [hip.DeviceBuffer(max(o.nbytes, 1)) for o in outs]
    ip = (ctypes.c_void_p * max(len(dins), 1))(*[d.ptr for d in dins])
    op = (ctypes.c_void_p * max(len(douts), 1))(*[d.ptr for d in douts])
    lib = hip.library()
    fn = lib.accy_hip_invoke_device_scratch if scratch else lib.accy_hip_invoke_device
    st = fn(h, ip, len(dins), op, len(douts), ctypes.c_void_p(stream.handle))
    assert st == hip.OK, lib.accy_hip_last_error().decode()
    stream.synchronize()
    for o, d in zip(outs, douts):
        d.download(o)
    for d in dins + douts:
        d.free()
    return outs


@pytest.mark.parametrize("big,small", [
    (lambda: W.decoder_program(1, 256, 256, 2, 128, 512), lambda: W.decoder_program(1, 128, 256, 2, 128, 512)),
    (lambda: _colsum(8192, 4096), lambda: _colsum(4096, 2048)),
    (lambda: _scan_with_contraction(5, 256), lambda: _scan_with_contraction(3, 128)),
    (lambda: W.decoder_program(), lambda: W.decoder_program(1, 256, 256, 2, 128, 512)),   # C5 at full size fits
])
def test_scratch_entry_point_matches_invoke_device(big, small):
    s = hip.Session()
    stream = hip.Stream()
    progs = [big(), small()]
    handles = [s.compile(p) for p in progs]
    try:
        for i, (p, h) in enumerate(zip(progs, handles)):
            print(f"program {i}: {p.name}", flush=True)
            ins = _inputs(p, seed=10 + i)
            ref = _run(s, h, p, ins, False, stream)
            got = _run(s, h, p, ins, True, stream)
            for g, r in zip(got, ref):
                assert g.shape == r.shape and np.array_equal(g.view(np.uint8), r.view(np.uint8))
    finally:
        for h in handles:
            s.release(h)
        stream.destroy()


def test_scratch_entry_point_refuses_programs_beyond_the_scratch():
    # an f32 contraction with A stored [k, m] repacks A into a temporary of m * k * 4 bytes = 576 MiB
    n = 12288
    prog = T.define("tn", [T.spec("f32", k=n, m=n), T.spec("f32", k=n, n=256)], lambda b, a: a[0].contract(a[1], "k"))
    assert "pack" in hip.plan_source(prog)
    s = hip.Session()
    h = s.compile(prog)
    try:
        dummy = hip.DeviceBuffer(256)
        ip = (ctypes.c_void_p * 2)(dummy.ptr, dummy.ptr)
        op = (ctypes.c_void_p * 1)(dummy.ptr)
        lib = hip.library()
        st = lib.accy_hip_invoke_device_scratch(h, ip, 2, op, 1, ctypes.c_void_p(0))
        assert st == hip.OUT_OF_MEMORY
        assert "scratch holds 536870912" in lib.accy_hip_last_error().decode()
        dummy.free()
    finally:
        s.release(h)


# ---- HIP graph capture ----

def _hip_runtime():
    """The HIP runtime the library links (stream capture and graph calls are not part of its C ABI)."""
    rt = ctypes.CDLL("/opt/rocm/lib/libamdhip64.so")
    vp = ctypes.c_void_p
    rt.hipStreamBeginCapture.argtypes = [vp, ctypes.c_int]
    rt.hipStreamEndCapture.argtypes = [vp, ctypes.POINTER(vp)]
    rt.hipGraphInstantiate.argtypes = [ctypes.POINTER(vp), vp, vp, ctypes.c_char_p, ctypes.c_size_t]
    rt.hipGraphLaunch.argtypes = [vp, vp]
    rt.hipGraphExecDestroy.argtypes = [vp]
    rt.hipGraphDestroy.argtypes = [vp]
    for f in ("hipStreamBeginCapture", "hipStreamEndCapture", "hipGraphInstantiate", "hipGraphLaunch",
              "hipGraphExecDestroy", "hipGraphDestroy"):
        getattr(rt, f).restype = ctypes.c_int
    return rt


class _Bound:
    """Device copies of one invocation's inputs and outputs, kept for several invocations."""

    def __init__(self, prog, ins):
        self.dins = [hip.DeviceBuffer.from_array(x) for x in ins]
        self.outs = [np.zeros(t.shape, T.NUMPY_DTYPE[t.dtype]) for t in prog.output_types()]
        self.douts = [hip.DeviceBuffer(max(o.nbytes, 1)) for o in self.outs]
        self.ip = (ctypes.c_void_p * max(len(self.dins), 1))(*[d.ptr for d in self.dins])
        self.op = (ctypes.c_void_p * max(len(self.douts), 1))(*[d.ptr for d in self.douts])

    def call(self, h, scratch, stream):
        lib = hip.library()
        fn = lib.accy_hip_invoke_device_scratch if scratch else lib.accy_hip_invoke_device
        st = fn(h, self.ip, len(self.dins), self.op, len(self.douts), ctypes.c_void_p(stream.handle))
        assert st == hip.OK, lib.accy_hip_last_error().decode()

    def clear(self):
        for o, d in zip(self.outs, self.douts):
            d.upload(np.zeros_like(o))

    def read(self):
        return [d.download(np.zeros_like(o)) for o, d in zip(self.outs, self.douts)]

    def free(self):
        for d in self.dins + self.douts:
            d.free()


def _capture(rt, stream, fn):
    graph, exe = ctypes.c_void_p(), ctypes.c_void_p()
    assert rt.hipStreamBeginCapture(ctypes.c_void_p(stream.handle), 1) == 0   # thread-local mode
    fn()
    assert rt.hipStreamEndCapture(ctypes.c_void_p(stream.handle), ctypes.byref(graph)) == 0
    return graph


def _same(got, ref):
    for g, r in zip(got, ref):
        assert g.shape == r.shape and np.array_equal(g.view(np.uint8), r.view(np.uint8))


@pytest.mark.parametrize("scratch", [False, True])
def test_invocations_captured_into_hip_graphs(scratch):
    """A decoder block whose MLP-up epilogue is a lookup table filled by a run-once kernel. The first
    invocation of a fresh executor is captured into a graph that is destroyed without being launched;
    a later eager invocation must still find the table filled. Then an invocation (invoke_device, or
    the allocation-free variant) is captured and the graph replayed three times, with eager work of
    another program between the replays (which, on the scratch path, overwrites the shared scratch);
    every replay must equal an eager invoke_device of a separately compiled executor bit for bit."""
    prog = W.decoder_program(1, 256, 256, 2, 128, 512)
    assert "accy_lut_" in hip.plan_source(prog)
    other = W.decoder_program(1, 128, 256, 2, 128, 512)
    rt = _hip_runtime()
    s, stream = hip.Session(), hip.Stream()
    ins = _inputs(prog, seed=30)
    href = s.compile(prog)
    ref = _run(s, href, prog, ins, False, stream)
    s.release(href)
    h, ho = s.compile(prog), s.compile(other)
    bound, obound = _Bound(prog, ins), _Bound(other, _inputs(other, seed=31))
    try:
        print(f"capture of the first invocation, scratch={scratch}", flush=True)
        rt.hipGraphDestroy(_capture(rt, stream, lambda: bound.call(h, scratch, stream)))
        bound.clear()
        bound.call(h, False, stream)
        stream.synchronize()
        _same(bound.read(), ref)
        graph = _capture(rt, stream, lambda: bound.call(h, scratch, stream))
        exe = ctypes.c_void_p()
        assert rt.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0) == 0
        for r in range(3):
            print(f"replay {r}", flush=True)
            bound.clear()
            assert rt.hipGraphLaunch(exe, ctypes.c_void_p(stream.handle)) == 0
            stream.synchronize()
            _same(bound.read(), ref)
            obound.call(ho, scratch, stream)
            stream.synchronize()
        rt.hipGraphExecDestroy(exe)
        rt.hipGraphDestroy(graph)
    finally:
        bound.free()
        obound.free()
        s.release(h)
        s.release(ho)
        stream.destroy()
