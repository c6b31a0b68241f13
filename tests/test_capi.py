"""The C ABI on a host without a GPU: the library loads, exports every declared entry point, lowers
every config program into kernels that hiprtc compiles for gfx950, and maps failures to the
reference session's status numbers (src/tensor/session/session.zig:33-56)."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from accy_amd import hip
from accy_amd import tensor as T
from accy_amd import workloads as W
from test_wire import readme_one_guess_bytes, u32

HEADER = Path(__file__).resolve().parent.parent / "include" / "accy_hip.h"


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^(?:int|const char\*)\s+(accy_hip_\w+)\(", text, re.M)))


def test_library_exports_every_declared_entry_point():
    lib = hip.library()
    names = declared_functions()
    assert len(names) >= 13
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(hip.EXPORTS)


SMALL_PROGRAMS = {
    "readme": lambda: W.tone_program(points=16, scalar=True),
    "tone": lambda: W.tone_program(64, 1024),
    "lse": lambda: W.logsumexp_program(16, 8192),
    "lse-bf16": lambda: W.logsumexp_program(16, 256, dtype="bf16"),
    "gemm-f32": lambda: W.gemm_program(64, 64, 64),
    "gemm-bf16-mulsum": lambda: W.gemm_program(64, 64, 64, "bf16", "mulsum"),
    "attention": lambda: W.attention_program(2, 128, 64),
    "attention-causal": lambda: W.attention_program(2, 128, 64, causal=True),
    "attention-fused": lambda: W.attention_program(2, 256, 128, "f16"),
    "attention-fused-causal-bf16": lambda: W.attention_program(1, 128, 128, "bf16", causal=True),
    "decoder": lambda: W.decoder_program(1, 64, 128, 2, 64, 256),
}


@pytest.mark.parametrize("name", sorted(SMALL_PROGRAMS))
def test_every_config_program_lowers_and_compiles_for_gfx950(name):
    src = hip.plan_source(SMALL_PROGRAMS[name](), compile=True)
    assert "__global__" in src


@pytest.mark.parametrize("prog,fused", [
    (lambda: W.attention_program(32, 4096, 128, "f16"), True),
    (lambda: W.attention_program(2, 384, 128, "bf16", causal=True), True),
    (lambda: W.decoder_program(), True),
    (lambda: W.attention_program(2, 128, 64), True),      # head dimension 64 (16-bit)
    (lambda: W.attention_program(2, 96, 64), True),       # 96 queries: one-wave workgroups
    (lambda: W.attention_program(2, 96, 128), False),     # one-wave workgroups at head dimension 128 spill
    (lambda: W.attention_program(2, 192, 128), True),     # two-wave workgroups
    (lambda: W.attention_program(2, 192, 128, "bf16", causal=True), False),  # causal: four loop tails spill
    (lambda: W.attention_program(2, 80, 128), False),     # 80 queries: not a multiple of 32
    (lambda: W.attention_program(2, 256, 256), False),    # head dimension 256 spills: unfused kernels
    (lambda: W.attention_program(2, 128, 512), False),    # head dimension 512: unfused kernels
    (lambda: W.attention_program(2, 128, 64, "f32"), True),          # the reference's flash pattern
    (lambda: W.attention_program(1, 96, 64, "f32", causal=True), True),
    (lambda: W.attention_program(2, 128, 128, "f32"), False),        # f32 fuses at head dimension 64
])
def test_attention_fusion_decision(prog, fused):
    src = hip.plan_source(prog(), compile=False)
    assert ("accy::attn::flash" in src) == fused
    if fused:
        # scores, softmax and the product with V in one kernel: no score buffer is planned
        assert src.count("accy::attn::flash<") + src.count("accy::attn::flash_f32<") == 1


def test_decoder_gelu_epilogue_is_a_lookup_table():
    """The decoder's MLP-up contraction ends in GELU (ten bf16 operations on the contraction value and
    constants): a table kernel evaluates them once per 16-bit pattern and the epilogue looks them up;
    the contractions whose epilogues read other tensors (the residual adds) keep direct epilogues."""
    src = hip.plan_source(W.decoder_program(1, 256, 512, 4, 128, 1024), compile=False)
    assert src.count("accy_lut_") == 1 and "// lut:%" in src
    assert src.count("[accy::f32_to_bf16(v)]") == 1


def test_contraction_tile_walk_follows_the_larger_operand():
    """The direct-to-LDS contraction walks its tiles in groups of 4 tile rows when A is the larger
    operand (M > N: each XCD reads each A panel once per round where B is at least 8 tiles wide) and
    of 8 otherwise."""
    def cfg(m, k, n):
        src = hip.plan_source(W.gemm_program(m, k, n, "bf16", "contract"), compile=False)
        return [line for line in src.split("\n") if "STAGES = 4" in line][0]
    assert "GROUP_M = 4" in cfg(8192, 512, 2048)
    assert "GROUP_M = 8" in cfg(2048, 512, 8192)
    assert "GROUP_M = 8" in cfg(4096, 512, 4096)


def test_attention_fusion_keeps_values_read_elsewhere():
    # the probabilities are also an output, so they must be materialised: no fusion
    def body(b, a):
        q, k, v = a
        s = q.contract(k.rename("query", "key"), "dim").mul(b.full_float(T.Type("f16", ()), 0.125))
        e = s.sub(s.max("key")).exp()
        p = e.div(e.sum("key"))
        return [p.contract(v.rename("query", "key"), "key"), p]
    specs = [T.spec("f16", head=1, query=128, dim=128)] * 3
    src = hip.plan_source(T.define("twice", specs, body), compile=False)
    assert "accy::attn::flash" not in src


@pytest.mark.parametrize("dtype,spelling,kernel", [
    ("f32", "contract", "mma32f"), ("f32", "mulsum", "mma32f"),
    ("bf16", "contract", "mma16_dma"), ("bf16", "mulsum", "mma16_dma")])
def test_contractions_plan_onto_matrix_cores(dtype, spelling, kernel):
    src = hip.plan_source(W.gemm_program(8192, 8192, 8192, dtype, spelling), compile=False)
    assert ("accy::gemm::" + kernel + "<") in src
    assert src.count("__global__") == 1


def test_small_or_ragged_f32_contractions_keep_serial_order():
    for m, k, n in [(33, 65, 17), (256, 30, 256), (300, 64, 256)]:
        src = hip.plan_source(W.gemm_program(m, k, n, "f32", "mulsum"), compile=False)
        assert "accy::gemm::" not in src


def test_contractions_with_more_batches_than_the_grid_holds_take_the_dot():
    # the matrix-core kernels index the batch by blockIdx.y, at most 65535 on gfx950
    def batched(dtype, nb):
        return T.define("bb", [T.spec(dtype, b=nb, m=128, k=128), T.spec(dtype, b=nb, k=128, n=128)],
                        lambda b, a: a[0].contract(a[1], "k"))
    assert "accy::gemm::mma16_dma<" in hip.plan_source(batched("bf16", 65535), compile=False)
    src = hip.plan_source(batched("bf16", 65536), compile=False)
    assert "accy::gemm::" not in src and "// dot:" in src


def test_operands_sharing_one_buffer_compile():
    # x . x^T on the matrix cores and self-attention with q = k = v: one kernel parameter each
    gram = T.define("gram", [T.spec("bf16", m=256, k=128)],
                    lambda b, a: a[0].contract(a[0].rename("m", "n"), "k"))
    assert "accy::gemm::" in hip.plan_source(gram, compile=True)
    specs = [T.spec("f16", head=2, query=128, dim=128)]
    self_attn = T.define("self", specs, lambda b, a: W.attention_body("f16", 128)(b, [a[0], a[0], a[0]]))
    assert "accy::attn::flash" in hip.plan_source(self_attn, compile=True)


def test_values_larger_than_a_device_holds_are_refused_before_planning():
    # a 2^20 x 2^19 f32 parameter (2 TiB): OUT_OF_MEMORY when the program is decoded, as an
    # allocation would fail
    big = T.define("big", [T.spec("f32", m=1 << 20, n=1 << 19)], lambda b, a: [a[0].exp()])
    with pytest.raises(hip.HipError) as e:
        hip.plan_source(big)
    assert e.value.status == 6 and "more than one device holds" in str(e.value)
    # 1 TiB exactly is planned
    edge = T.define("edge", [T.spec("u8", m=1 << 20, n=1 << 20)], lambda b, a: [a[0].add(a[0])])
    assert "__global__" in hip.plan_source(edge)
    # an intermediate past 2^50 elements (a fused product of 2^17 x 2^17 x 2^17) is refused too
    mm = W.gemm_program(1 << 17, 1 << 17, 1 << 17, "bf16", "mulsum")
    with pytest.raises(hip.HipError) as e:
        hip.plan_source(mm)
    assert e.value.status == 6 and "more than this target plans" in str(e.value)
    # the C3 spelling's 2 TiB intermediate (8192^3 f32) is fused away and planned
    assert "mma32f" in hip.plan_source(W.gemm_program(8192, 8192, 8192, "f32", "mulsum"))


def test_indexing_and_integer_programs_compile():
    def body(b, a):
        g = a[0].gather(a[1], "v")
        return [a[0].scatter_add(a[1], g, "v"), a[2].add(a[2]).max("j")]
    p = T.define("ix", [T.spec("f32", v=8), T.spec("i32", j=8), T.spec("i32", j=8)], body)
    assert "__global__" in hip.plan_source(p, compile=True)


def test_row_leaves_read_once_are_streamed():
    # C2 reads each element once (the row is cached in registers): non-temporal vector loads.
    assert hip.plan_source(W.logsumexp_program(32768, 8192)).count("accy::ld_quad_stream(") == 1
    # C1's time and sample are broadcast along the rows: every workgroup rereads them, plain loads.
    assert "ld_quad_stream" not in hip.plan_source(W.tone_program(8192, 16384))
    # A row too long for the register cache is read by two passes: plain loads.
    assert "ld_quad_stream" not in hip.plan_source(W.logsumexp_program(64, 102400))
    # One pass over a row that is not cached (a plain sum): streamed, and it builds for gfx950.
    p = T.define("rowsum", [T.spec("bf16", r=64, c=65536)], lambda b, a: a[0].sum("c"))
    assert "accy::ld_quad_stream(" in hip.plan_source(p, compile=True)


def test_row_fusion_gives_one_kernel_for_logsumexp():
    src = hip.plan_source(W.logsumexp_program(32, 8192))
    assert src.count("__global__") == 1
    assert "cache0" in src   # the row stays in registers between the max pass and the sum pass


def _status_of_plan(wire: bytes) -> int:
    lib = hip.library()
    buf = (ctypes.c_uint8 * len(wire)).from_buffer_copy(wire)
    need = ctypes.c_size_t()
    return lib.accy_hip_plan_source(buf, len(wire), 0, None, 0, ctypes.byref(need))


def test_bad_wire_bytes_map_to_session_statuses():
    good = readme_one_guess_bytes()
    assert _status_of_plan(good) == hip.OK
    assert _status_of_plan(b"XCTP" + good[4:]) == hip.INVALID_PROGRAM
    assert _status_of_plan(good[:4] + u32(7) + good[8:]) == hip.UNSUPPORTED_VERSION
    assert _status_of_plan(good[:-2]) == hip.INVALID_PROGRAM


def test_unknown_handles_are_refused():
    lib = hip.library()
    for h in (hip.Handle(0, 12345), hip.Handle(64, 0), hip.Handle(1000, 0)):
        assert lib.accy_hip_release(h) == hip.INVALID_HANDLE
        assert lib.accy_hip_counts(h, None, None) == hip.INVALID_HANDLE


def test_unsupported_operations_fail_to_compile_with_a_named_reason():
    # a custom call names a host-registered target runCpu itself has no kernel for
    p = T.define("cc", [T.spec("f32", r=2, c=3)],
                 lambda b, a: b.custom_call("user.fn", 1, [a[0]], a[0].ty))
    with pytest.raises(hip.HipError) as e:
        hip.plan_source(p)
    assert e.value.status == hip.COMPILE_FAILED and "custom_call" in e.value.message


def test_compile_without_a_device_fails_loudly():
    if hip.library().accy_hip_device_arch(None, 0) == hip.OK:
        pytest.skip("a HIP device is present")
    with pytest.raises(hip.HipError) as e:
        hip.Hip(W.tone_program(8, 16))
    assert e.value.status == hip.COMPILE_FAILED
