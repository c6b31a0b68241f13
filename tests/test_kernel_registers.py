"""Generated matrix-core kernels fit in their registers (CPU test).

A kernel that spills registers to scratch memory is slow, and compiling a spilling kernel has crashed
the device compiler (a segmentation fault in its pass that rewrites MFMAs around AGPR spill copies),
which ends the calling process. So:

* fused attention is planned only for shapes whose kernel fits (planner_attention.cpp,
  attention_layout); the 16-bit kernel forces its MFMA results into VGPRs, so any AGPR it uses is a
  spill slot;
* the contraction kernels keep their accumulators in AGPRs and must not touch scratch, whatever
  their epilogue (the f32 kernel spilled its K loop's offsets once its epilogue computed on the
  values, before its accumulators were pinned to AGPRs after the loop).

Each case compiles the planned kernel as the runtime does (the template text in place of its
#include lines, the runtime's compiler options; offline hipcc here) and reads the compiler's resource
report.
"""
import math
import re
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

from accy_amd import hip, tensor as T, workloads as W
from accy_amd.build import KERNELS, ROCM

HIPCC = ROCM / "bin" / "hipcc"
MARKER = "// accy: mfma-vgpr-form\n"
OPTIONS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-mllvm", "-pragma-unroll-threshold=65536"]


def _attention(dtype, heads, sq, sk, hd, causal):
    specs = [T.spec(dtype, head=heads, query=sq, dim=hd), T.spec(dtype, head=heads, key=sk, dim=hd),
             T.spec(dtype, head=heads, key=sk, dim=hd)]
    return T.define("fa", specs, W.attention_body(dtype, hd, causal))


# (name, program): every one plans its attention as one fused kernel
FUSED = [
    ("c4 f16 32 x 4096 x 128", lambda: W.attention_program(32, 4096, 128, "f16")),
    ("c5 decoder block bf16", lambda: W.decoder_program()),
    ("f16 128 x 512 x 128, four waves", lambda: _attention("f16", 2, 128, 512, 128, False)),
    ("bf16 192 x 320 x 128, two waves", lambda: _attention("bf16", 2, 192, 320, 128, False)),
    ("bf16 384 x 384 x 128 causal, four waves", lambda: _attention("bf16", 2, 384, 384, 128, True)),
    ("bf16 512 x 256 x 128 causal, eight waves", lambda: _attention("bf16", 2, 512, 256, 128, True)),
    ("f16 1024 x 384 x 128 causal, eight waves", lambda: _attention("f16", 2, 1024, 384, 128, True)),
    ("bf16 96 x 96 x 64 causal, one wave", lambda: _attention("bf16", 2, 96, 96, 64, True)),
    ("f16 224 x 320 x 64 causal, one wave", lambda: _attention("f16", 3, 224, 320, 64, True)),
    ("f16 32 x 384 x 64, one wave", lambda: _attention("f16", 1, 32, 384, 64, False)),
    ("bf16 192 x 320 x 64 causal, two waves", lambda: _attention("bf16", 2, 192, 320, 64, True)),
    ("f16 768 x 320 x 64 causal, eight waves", lambda: _attention("f16", 2, 768, 320, 64, True)),
    ("f32 96 x 96 x 64 causal", lambda: _attention("f32", 2, 96, 96, 64, True)),
    ("f32 1024 x 1024 x 64", lambda: _attention("f32", 4, 1024, 1024, 64, False)),
]

# Shapes whose kernel spilled (or, for 352 x 384 at head dimension 256, computed wrong values with an
# earlier version of the kernel; and 224 x 320 x 256 crashed the compiler): they run unfused.
UNFUSED = [
    ("f16 224 x 320 x 256 causal", lambda: _attention("f16", 3, 224, 320, 256, True)),
    ("bf16 352 x 384 x 256 causal", lambda: _attention("bf16", 3, 352, 384, 256, True)),
    ("f16 256 x 256 x 256", lambda: _attention("f16", 2, 256, 256, 256, False)),
    ("bf16 352 x 384 x 128 causal, one wave", lambda: _attention("bf16", 2, 352, 384, 128, True)),
    ("f16 32 x 384 x 128, one wave", lambda: _attention("f16", 1, 32, 384, 128, False)),
    ("bf16 192 x 224 x 128 causal, two waves", lambda: _attention("bf16", 2, 192, 224, 128, True)),
    ("f16 384 x 320 x 128 causal, keys not a multiple of 128", lambda: _attention("f16", 2, 384, 320, 128, True)),
    ("f16 768 x 320 x 128 causal, keys not a multiple of 128", lambda: _attention("f16", 2, 768, 320, 128, True)),
]


def _kernels(src: str, marker: str):
    """The planned kernels whose source contains marker, each with the template text in place of its
    #include lines (as the runtime's full_kernel_source assembles it)."""
    parts = re.split(r"^// \S+ grid \d+ block \d+\n", src, flags=re.M)
    out = []
    for body in parts:
        if marker not in body:
            continue
        for line, name in (('#include "gemm"\n', "gemm.h"), ('#include "attention"\n', "attention.h")):
            body = body.replace(line, (KERNELS / name).read_text() + "\n", 1)
        out.append((KERNELS / "common.h").read_text() + "\n" + body)
    return out


def _attention_kernel(src: str) -> str:
    found = _kernels(src, "accy::attn::flash")
    assert len(found) == 1
    return found[0]


def _resources(name: str, source: str, tmp: Path) -> dict:
    path = tmp / (re.sub(r"\W+", "_", name) + ".hip")
    path.write_text(source)
    opts = OPTIONS + (["-mllvm", "-amdgpu-mfma-vgpr-form"] if MARKER in source else [])
    proc = subprocess.run([str(HIPCC)] + opts + ["--cuda-device-only", "--no-gpu-bundle-output", "-c",
                                                 "-Rpass-analysis=kernel-resource-usage", str(path),
                                                 "-o", str(path.with_suffix(".o"))], capture_output=True, text=True)
    assert proc.returncode == 0, f"{name}: hipcc failed\n{proc.stderr[-2000:]}"
    out = {}
    for key, pat in (("vgpr", r"VGPRs: (\d+)"), ("agpr", r"AGPRs: (\d+)"), ("scratch", r"ScratchSize \[bytes/lane\]: (\d+)")):
        vals = [int(v) for v in re.findall(pat, proc.stderr)]
        assert vals, f"{name}: no resource report"
        out[key] = max(vals)
    out["vgpr_form"] = MARKER in source
    return out


@pytest.mark.skipif(not HIPCC.exists(), reason="needs the ROCm compiler")
def test_fused_attention_kernels_do_not_spill(tmp_path):
    sources = []
    for name, prog in FUSED:
        src = hip.plan_source(prog(), compile=False)
        sources.append((name, _attention_kernel(src)))
    with ThreadPoolExecutor(4) as ex:
        results = list(ex.map(lambda c: (c[0], _resources(c[0], c[1], tmp_path)), sources))
    bad = []
    for name, r in results:
        if r["scratch"] or (r["vgpr_form"] and r["agpr"]):
            bad.append(f"{name}: {r}")
    assert not bad, "spilling fused attention kernels:\n" + "\n".join(bad)


@pytest.mark.parametrize("name,prog", UNFUSED, ids=[n for n, _ in UNFUSED])
def test_attention_shapes_that_would_spill_run_unfused(name, prog):
    # plans without the fused kernel and compiles (hiprtc, in this process)
    src = hip.plan_source(prog(), compile=True)
    assert "accy::attn::flash" not in src


def _contraction(dtype, m, k, n, epi, ta=False):
    sc = T.Type(dtype, ())
    a_spec = T.spec(dtype, k=k, m=m) if ta else T.spec(dtype, m=m, k=k)
    specs = [a_spec, T.spec(dtype, k=k, n=n), T.spec(dtype, m=m, n=n)]

    def body(b, a):
        x, w, r = a
        d = x.contract(w, "k")
        if epi == "scale":
            d = d.mul(b.full_float(sc, 0.5))
        elif epi == "gelu":
            d = d.mul(b.full_float(sc, 0.5)).mul(d.mul(b.full_float(sc, 0.7978845608028654)).tanh().add(b.full_float(sc, 1.0)))
        elif epi == "resid":
            d = d.add(r)
        elif epi == "tanh":
            d = d.tanh()
        return [d]
    return T.define("mm", specs, body)


CONTRACTIONS = [
    ("c3 bf16 8192^3", lambda: W.gemm_program(8192, 8192, 8192, "bf16", "mulsum")),
    ("c3 f32 8192^3", lambda: W.gemm_program(8192, 8192, 8192, "f32", "mulsum")),
    ("c5 decoder block", lambda: W.decoder_program()),
    ("f32 1024^2 x 256, scale", lambda: _contraction("f32", 1024, 256, 1024, "scale")),
    ("f32 1184 x 256 x 768, residual", lambda: _contraction("f32", 1184, 256, 768, "resid")),
    ("f32 512 x 224 x 1024, gelu", lambda: _contraction("f32", 512, 224, 1024, "gelu")),
    ("f32 256 x 2048 x 272, tanh", lambda: _contraction("f32", 256, 2048, 272, "tanh")),
    ("bf16 512^3, gelu table", lambda: _contraction("bf16", 512, 512, 512, "gelu")),
    ("bf16 1024 x 32 x 1024, residual", lambda: _contraction("bf16", 1024, 32, 1024, "resid")),
    ("f16 483 x 192 x 512, residual (register-staged)", lambda: _contraction("f16", 483, 192, 512, "resid")),
    ("bf16 944 x 2048 x 256, scale", lambda: _contraction("bf16", 944, 2048, 256, "scale", ta=True)),
]


@pytest.mark.skipif(not HIPCC.exists(), reason="needs the ROCm compiler")
def test_contraction_kernels_do_not_spill(tmp_path):
    sources = []
    for name, prog in CONTRACTIONS:
        found = _kernels(hip.plan_source(prog(), compile=False), "accy::gemm::")
        assert found, name
        sources += [(f"{name} #{i}", src) for i, src in enumerate(found)]
    with ThreadPoolExecutor(4) as ex:
        results = list(ex.map(lambda c: (c[0], _resources(c[0], c[1], tmp_path)), sources))
    bad = [f"{name}: {r}" for name, r in results if r["scratch"]]
    assert not bad, "contraction kernels using scratch memory:\n" + "\n".join(bad)
