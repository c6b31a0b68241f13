"""Writes the golden fixtures of this directory from the CPU oracle (the runCpu restatement).

Every fixture is checked against the mathematics that fixes it (a closed form in float64, a known
answer of the reference's README / example, or a brute-force serial loop) before it is written, so a
mistake in the oracle cannot become a fixture. The fixtures hold inputs and outputs only, f32 values
as their IEEE bit patterns (exact), and the ACTP v1 bytes of every benchmark program.

    python tests/golden/make_golden.py        # rewrites tests/golden/*.json and wire/*.actp

Cases (reference anchors):
  tone_readme.json      README tone, 16 points: one guess at 2.5 and 3.0, eight guesses, value and
                        slope (README.md:152-160, 300-304; examples/consumer/src/main.zig:187-228)
  mismatch_curve.json   361 guesses from -0.5 to 8.5 (main.zig:152-181)
  serial_folds.json     tiny reductions whose value depends on the serial f32 fold order
                        (reduction.zig:839-878, 1157-1177)
  sdpa.json             2 x 2 x 3 x 2 x 2 scaled dot-product attention (library/attention.zig:464-509)
  gelu.json             tanh GELU on 8 values (library/fused.zig:471-478; elementwise.zig:234-240)
  wire/<config>.actp    the traced programs of the benchmark configurations (wire/encode.zig)
"""
from __future__ import annotations

import json
import math
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
sys.path.insert(0, str(HERE.parent.parent))

from accy_amd import tensor as T  # noqa: E402
from accy_amd import workloads as W  # noqa: E402
from conftest import oracle_run  # noqa: E402


def bits(x) -> list:
    return np.asarray(x, np.float32).reshape(-1).view(np.uint32).tolist()


def f64_mismatch(time, sample, frequency):
    t = time.astype(np.float64)
    d = np.sin(frequency * t) - sample.astype(np.float64)
    return float((d * d).sum()), float((2 * d * np.cos(frequency * t) * t).sum())


def tone_readme() -> dict:
    time, sample = W.readme_tone()
    one = W.tone_program(points=16, scalar=True)
    v25 = float(oracle_run(one, [np.array(2.5, np.float32), time, sample])[0])
    v3 = float(oracle_run(one, [np.array(3.0, np.float32), time, sample])[0])
    ref25, slope_ref = f64_mismatch(time, sample, 2.5)
    assert abs(v25 - 8.656) < 5e-4 and abs(v25 - ref25) <= 1e-5 * ref25 and abs(v3) <= 1e-9
    starts = np.array([0.5, 1.5, 2.5, 3.5, 4.5, 5.5, 6.5, 7.5], np.float32)
    eight = oracle_run(W.tone_program(guesses=8, points=16), [starts, time, sample])[0]
    for s, v in zip(starts, eight):
        r = f64_mismatch(time, sample, float(s))[0]
        assert abs(float(v) - r) <= 1e-5 * abs(r)
    val, slope = oracle_run(W.tone_value_and_slope_program(8, 16), [starts, time, sample])
    for s, v, d in zip(starts, val, slope):
        r, dr = f64_mismatch(time, sample, float(s))
        assert abs(float(v) - r) <= 1e-5 * abs(r) and abs(float(d) - dr) <= 1e-4 * max(1.0, abs(dr))
    assert abs(float(slope[2]) - (-31.29)) < 5e-3
    return {"time": bits(time), "sample": bits(sample),
            "one_guess": {"frequency": bits([2.5, 3.0]), "mismatch": bits([v25, v3])},
            "eight_guesses": {"frequency": bits(starts), "mismatch": bits(eight)},
            "value_and_slope": {"frequency": bits(starts), "mismatch": bits(val), "slope": bits(slope)}}


def mismatch_curve() -> dict:
    time, sample = W.readme_tone()
    freq = (-0.5 + 0.025 * np.arange(361)).astype(np.float32)
    got = oracle_run(W.tone_program(guesses=361, points=16), [freq, time, sample])[0]
    for f, v in zip(freq, got):
        r = f64_mismatch(time, sample, float(f))[0]
        assert abs(float(v) - r) <= 1e-5 * abs(r) + 1e-9
    return {"time": bits(time), "sample": bits(sample), "frequency": bits(freq), "mismatch": bits(got)}


def serial_fold(x: np.ndarray) -> np.float32:
    acc = np.float32(0)
    for v in x.reshape(-1):
        acc = np.float32(acc + np.float32(v))
    return acc


def serial_folds() -> dict:
    cases = []
    # Left to right in f32: ((1e8 + 1) - 1e8) + 1 = 1 (pairwise: 0, f64: 2).
    x = np.array([1e8, 1.0, -1e8, 1.0], np.float32)
    got = oracle_run(T.define("s", [T.spec("f32", i=4)], lambda b, a: a[0].sum("i")), [x])[0]
    assert float(got) == 1.0 == float(serial_fold(x))
    cases.append({"name": "sum_1e8", "shape": [4], "axes": ["i"], "x": bits(x), "out": bits(got)})
    # Two reduced axes fold in row-major order of the reduced axes; a kept axis in front.
    rng = np.random.default_rng(41)
    x = (rng.standard_normal((3, 4, 5)) * np.array([1e6, 1.0, 1e-3, 1e4, 1e2])[None, None, :]).astype(np.float32)
    prog = T.define("s", [T.spec("f32", r=3, a=4, c=5)], lambda b, a: a[0].sum(("a", "c")))
    got = oracle_run(prog, [x])[0]
    for r in range(3):
        assert got[r] == serial_fold(x[r])
    cases.append({"name": "sum_two_axes", "shape": [3, 4, 5], "axes": ["a", "c"], "x": bits(x), "out": bits(got)})
    # Max over the inner axis; -inf and +0 / -0 ties.
    x = np.array([[-np.inf, -3.0, -0.0, 0.0], [2.5, 7.0, -1.0, 7.0]], np.float32)
    prog = T.define("m", [T.spec("f32", r=2, i=4)], lambda b, a: a[0].max("i"))
    got = oracle_run(prog, [x])[0]
    assert float(got[1]) == 7.0 and float(got[0]) == 0.0
    cases.append({"name": "max_inner", "shape": [2, 4], "axes": ["i"], "x": bits(x), "out": bits(got)})
    return {"cases": cases}


def sdpa_program() -> T.Program:
    """softmax(Q K^T / sqrt(2)) V with 2 batches, 2 queries, 3 keys, qk 2, value 2."""
    def body(b, a):
        s = a[0].contract(a[1], "qk").mul(b.full_float(T.Type("f32", ()), 1.0 / math.sqrt(2)))
        e = s.sub(s.max("key")).exp()
        return e.div(e.sum("key")).contract(a[2], "key")
    return T.define("sdpa", [T.spec("f32", batch=2, query=2, qk=2), T.spec("f32", batch=2, key=3, qk=2),
                             T.spec("f32", batch=2, key=3, value=2)], body)


def gelu_program() -> T.Program:
    return T.define("g", [T.spec("f32", i=8)], lambda b, a: W.gelu(b, a[0], "f32"))


def sdpa() -> dict:
    rng = np.random.default_rng(9)
    q = rng.standard_normal((2, 2, 2)).astype(np.float32)
    k = rng.standard_normal((2, 3, 2)).astype(np.float32)
    v = rng.standard_normal((2, 3, 2)).astype(np.float32)
    got = oracle_run(sdpa_program(), [q, k, v])[0]
    s = np.einsum("bqd,bkd->bqk", q.astype(np.float64), k.astype(np.float64)) / math.sqrt(2)
    p = np.exp(s - s.max(-1, keepdims=True))
    ref = np.einsum("bqk,bkv->bqv", p / p.sum(-1, keepdims=True), v.astype(np.float64))
    assert np.abs(got - ref).max() <= 1e-6
    return {"q": bits(q), "k": bits(k), "v": bits(v), "shape": {"batch": 2, "query": 2, "key": 3, "qk": 2, "value": 2},
            "scale": bits([1.0 / math.sqrt(2)]), "out": bits(got)}


def gelu() -> dict:
    x = np.array([-3.0, -1.5, -0.5, -0.1, 0.0, 0.3, 1.0, 2.5], np.float32)
    got = oracle_run(gelu_program(), [x])[0]
    x64 = x.astype(np.float64)
    ref = 0.5 * x64 * (1 + np.tanh(0.7978845608028654 * (x64 + 0.044715 * x64 ** 3)))
    assert np.abs(got - ref).max() <= 1e-6
    return {"x": bits(x), "out": bits(got)}


def config_programs() -> dict:
    """The traced program of every benchmark configuration, at its benchmark size."""
    return {
        "c1-tone": W.tone_program(8192, 16384),
        "c2-lse": W.logsumexp_program(32768, 8192),
        "c3-gemm-f32": W.gemm_program(8192, 8192, 8192, "f32", "mulsum"),
        "c3-gemm-bf16": W.gemm_program(8192, 8192, 8192, "bf16", "mulsum"),
        "c4-attention": W.attention_program(32, 4096, 128, "f16"),
        "c5-decoder": W.decoder_program(),
    }


def main() -> None:
    for name, make in [("tone_readme", tone_readme), ("mismatch_curve", mismatch_curve),
                       ("serial_folds", serial_folds), ("sdpa", sdpa), ("gelu", gelu)]:
        (HERE / f"{name}.json").write_text(json.dumps(make(), indent=1) + "\n")
    (HERE / "wire").mkdir(exist_ok=True)
    for name, prog in config_programs().items():
        (HERE / "wire" / f"{name}.actp").write_bytes(prog.encode())
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main()
