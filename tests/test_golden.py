"""The committed golden fixtures (tests/golden): pinned against the mathematics, reproduced by the CPU
oracle bit for bit, and matched by the HIP target.

The fixtures were written by tests/golden/make_golden.py from the oracle. The CPU tests below check
them independently of the oracle first (float64 closed forms, the README's known answers, serial f32
folds written out in numpy), then that the oracle still produces exactly those bits, and that the
tracer still writes the committed ACTP v1 bytes of every benchmark program. The GPU tests run the
same inputs through runHip.
"""
import json
import math
import sys
from pathlib import Path

import numpy as np
import pytest

from accy_amd import hip
from accy_amd import workloads as W
from conftest import hip_run, oracle_run, wire_roundtrip

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))
import make_golden as MG  # noqa: E402

CONFIGS = ["c1-tone", "c2-lse", "c3-gemm-f32", "c3-gemm-bf16", "c4-attention", "c5-decoder"]


def load(name: str) -> dict:
    return json.loads((GOLDEN / f"{name}.json").read_text())


def f32(bits) -> np.ndarray:
    return np.array(bits, np.uint32).view(np.float32)


def f64_mismatch(time, sample, frequency):
    t = time.astype(np.float64)
    d = np.sin(frequency * t) - sample.astype(np.float64)
    return (d * d).sum(), (2 * d * np.cos(frequency * t) * t).sum()


# ---- the fixtures against the mathematics (no oracle involved) ----

def test_golden_tone_matches_readme_and_f64():
    g = load("tone_readme")
    time, sample = f32(g["time"]), f32(g["sample"])
    rt, rs = W.readme_tone()
    assert np.array_equal(time, rt) and np.array_equal(sample, rs)
    v25, v3 = f32(g["one_guess"]["mismatch"])
    assert abs(float(v25) - 8.656) < 5e-4 and abs(float(v3)) <= 1e-9          # README.md:152-160
    for key in ("eight_guesses", "value_and_slope"):
        for f, v in zip(f32(g[key]["frequency"]), f32(g[key]["mismatch"])):
            ref = f64_mismatch(time, sample, float(f))[0]
            assert abs(float(v) - ref) <= 1e-5 * abs(ref)
    vs = g["value_and_slope"]
    for f, d in zip(f32(vs["frequency"]), f32(vs["slope"])):
        ref = f64_mismatch(time, sample, float(f))[1]
        assert abs(float(d) - ref) <= 1e-4 * max(1.0, abs(ref))
    assert abs(float(f32(vs["slope"])[2]) - (-31.29)) < 5e-3                    # README.md:300


def test_golden_curve_matches_f64():
    g = load("mismatch_curve")
    time, sample = f32(g["time"]), f32(g["sample"])
    freq, got = f32(g["frequency"]), f32(g["mismatch"])
    assert len(freq) == 361 and freq[0] == np.float32(-0.5) and abs(float(freq[-1]) - 8.5) < 1e-5
    for f, v in zip(freq, got):
        ref = f64_mismatch(time, sample, float(f))[0]
        assert abs(float(v) - ref) <= 1e-5 * abs(ref) + 1e-9


def test_golden_folds_are_serial_f32_folds():
    for c in load("serial_folds")["cases"]:
        x = f32(c["x"]).reshape(c["shape"])
        out = f32(c["out"])
        if c["name"].startswith("sum"):
            rows = x.reshape(len(out), -1) if len(c["shape"]) > 1 else x.reshape(1, -1)
            for r, o in zip(rows, out):
                acc = np.float32(0)
                for v in r:
                    acc = np.float32(acc + v)
                assert acc.view(np.uint32) == o.view(np.uint32)
        else:
            assert np.array_equal(x.max(axis=-1), out)
    assert float(f32(load("serial_folds")["cases"][0]["out"])[0]) == 1.0   # pairwise would give 0


def test_golden_sdpa_matches_closed_form():
    g = load("sdpa")
    sh = g["shape"]
    q = f32(g["q"]).reshape(sh["batch"], sh["query"], sh["qk"]).astype(np.float64)
    k = f32(g["k"]).reshape(sh["batch"], sh["key"], sh["qk"]).astype(np.float64)
    v = f32(g["v"]).reshape(sh["batch"], sh["key"], sh["value"]).astype(np.float64)
    s = np.einsum("bqd,bkd->bqk", q, k) / math.sqrt(sh["qk"])
    p = np.exp(s - s.max(-1, keepdims=True))
    ref = np.einsum("bqk,bkv->bqv", p / p.sum(-1, keepdims=True), v)
    assert np.abs(f32(g["out"]).reshape(ref.shape) - ref).max() <= 1e-6


def test_golden_gelu_matches_tanh_formula():
    g = load("gelu")
    x = f32(g["x"]).astype(np.float64)
    ref = 0.5 * x * (1 + np.tanh(0.7978845608028654 * (x + 0.044715 * x ** 3)))
    assert np.abs(f32(g["out"]) - ref).max() <= 1e-6


# ---- the oracle and the tracer reproduce the fixtures exactly ----

@pytest.mark.parametrize("name", ["tone_readme", "mismatch_curve", "serial_folds", "sdpa", "gelu"])
def test_oracle_reproduces_golden_bits(name):
    assert getattr(MG, name)() == load(name)


@pytest.mark.parametrize("config", CONFIGS)
def test_tracer_and_codec_reproduce_committed_wire_bytes(config):
    wire = (GOLDEN / "wire" / f"{config}.actp").read_bytes()
    assert MG.config_programs()[config].encode() == wire
    st, back = wire_roundtrip(wire)
    assert st == 0 and back == wire


@pytest.mark.parametrize("config,kernels", [
    ("c1-tone", ["row"]), ("c2-lse", ["row"]), ("c3-gemm-f32", ["gemm"]), ("c3-gemm-bf16", ["gemm"]),
    ("c4-attention", ["attention"]),
])
def test_committed_programs_plan_onto_the_expected_kernels(config, kernels):
    src = hip.plan_source((GOLDEN / "wire" / f"{config}.actp").read_bytes(), compile=False)
    labels = [line.split()[1].split(":")[0] for line in src.splitlines() if line.startswith("// ") and ":%" in line]
    assert labels == kernels, labels


def test_committed_decoder_plans_fused_attention_and_epilogue_gemms():
    src = hip.plan_source((GOLDEN / "wire" / "c5-decoder.actp").read_bytes(), compile=False)
    labels = [line.split()[1] for line in src.splitlines() if line.startswith("// ") and ":%" in line]
    assert sum(lab.startswith("attention:") for lab in labels) == 1
    assert sum(lab.startswith("gemm:") and "+" in lab for lab in labels) >= 2   # GELU and residual epilogues


# ---- the HIP target on the fixture inputs ----

def _rel_ok(got, ref, rel, floor=0.0):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    return np.all(np.abs(got - ref) <= rel * np.abs(ref) + floor)


@pytest.mark.gpu
def test_hip_matches_golden_tone_and_curve():
    g = load("tone_readme")
    time, sample = f32(g["time"]), f32(g["sample"])
    one = W.tone_program(points=16, scalar=True)
    for f, v in zip(f32(g["one_guess"]["frequency"]), f32(g["one_guess"]["mismatch"])):
        got = hip_run(one, [np.array(f, np.float32), time, sample])[0]
        assert _rel_ok(got, v, 1e-5, 1e-9)
    e = g["eight_guesses"]
    got = hip_run(W.tone_program(guesses=8, points=16), [f32(e["frequency"]), time, sample])[0]
    assert _rel_ok(got, f32(e["mismatch"]), 1e-5)
    vs = g["value_and_slope"]
    val, slope = hip_run(W.tone_value_and_slope_program(8, 16), [f32(vs["frequency"]), time, sample])
    assert _rel_ok(val, f32(vs["mismatch"]), 1e-5)
    assert _rel_ok(slope, f32(vs["slope"]), 1e-5, 1e-5 * np.abs(f32(vs["slope"])).max())
    c = load("mismatch_curve")
    got = hip_run(W.tone_program(guesses=361, points=16), [f32(c["frequency"]), f32(c["time"]), f32(c["sample"])])[0]
    assert _rel_ok(got, f32(c["mismatch"]), 1e-5, 1e-9)


@pytest.mark.gpu
def test_hip_matches_golden_serial_folds_exactly():
    from accy_amd import tensor as T
    for c in load("serial_folds")["cases"]:
        x = f32(c["x"]).reshape(c["shape"])
        names = ["i"] if len(c["shape"]) == 1 else (["r", "a", "c"] if len(c["shape"]) == 3 else ["r", "i"])
        spec = T.spec("f32", **dict(zip(names, c["shape"])))
        axes = tuple(c["axes"]) if len(c["axes"]) > 1 else c["axes"][0]
        if c["name"].startswith("sum"):
            prog = T.define("s", [spec], lambda b, a, axes=axes: a[0].sum(axes))
        else:
            prog = T.define("m", [spec], lambda b, a, axes=axes: a[0].max(axes))
        got = np.asarray(hip_run(prog, [x])[0], np.float32).reshape(-1)
        want = f32(c["out"])
        if c["name"].startswith("sum"):
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (c["name"], got, want)
        else:
            assert np.array_equal(got, want), (c["name"], got, want)


@pytest.mark.gpu
def test_hip_matches_golden_sdpa_and_gelu():
    g = load("sdpa")
    sh = g["shape"]
    ins = [f32(g["q"]).reshape(sh["batch"], sh["query"], sh["qk"]), f32(g["k"]).reshape(sh["batch"], sh["key"], sh["qk"]),
           f32(g["v"]).reshape(sh["batch"], sh["key"], sh["value"])]
    got = hip_run(MG.sdpa_program(), ins)[0]
    want = f32(g["out"]).reshape(got.shape)
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()
    gg = load("gelu")
    got = hip_run(MG.gelu_program(), [f32(gg["x"])])[0]
    want = f32(gg["out"])
    assert np.all(np.abs(got - want) <= 1e-5 * np.maximum(1.0, np.abs(want)))
