"""Launch tuning (src/executable/tuning.zig): candidate selection per kernel key, the artifact, and
measurement on the device.

The CPU tests drive the process-wide table through the C ABI without a device: artifacts are
imported and exported, malformed ones are refused without touching the table, and the planner's
sources follow an imported selection. The GPU test measures real candidates.
"""
import re
import struct

import numpy as np
import pytest

from accy_amd import hip
from accy_amd import tensor as T
from accy_amd import workloads as W
from conftest import assert_normwise, assert_rowwise, hip_run, oracle_run

MAGIC, VERSION = 0x54544341, 1


def artifact(records, magic=MAGIC, version=VERSION, count=None) -> bytes:
    out = struct.pack("<III", magic, version, len(records) if count is None else count)
    for key, cc, cand, ns, samples in records:
        k = key.encode()
        out += struct.pack("<I", len(k)) + k + struct.pack("<IIQI", cc, cand, ns, samples)
    return out


@pytest.fixture(autouse=True)
def clean_table():
    hip.tuning_clear()
    yield
    hip.tuning_clear()


def tuning_lines(src):
    return re.findall(r"// tuning (\S+) candidate (\d+) of (\d+)", src)


def test_artifact_round_trip_sorted_by_key():
    recs = [("gfx950/row/b/x", 4, 1, 1000, 5), ("gfx950/gemm/a/y", 2, 0, 2000, 7)]
    hip.tuning_import(artifact(recs))
    assert hip.tuning_count() == 2
    assert hip.tuning_export() == artifact(sorted(recs))
    hip.tuning_clear()
    assert hip.tuning_count() == 0 and hip.tuning_export() == artifact([])


def test_a_record_replaces_another_only_when_faster():
    hip.tuning_import(artifact([("k", 3, 1, 100, 5)]))
    hip.tuning_import(artifact([("k", 3, 0, 200, 5)]))
    assert hip.tuning_export() == artifact([("k", 3, 1, 100, 5)])
    hip.tuning_import(artifact([("k", 3, 2, 50, 5)]))
    assert hip.tuning_export() == artifact([("k", 3, 2, 50, 5)])
    # Same key with another candidate count is another record.
    hip.tuning_import(artifact([("k", 2, 0, 70, 5)]))
    assert hip.tuning_count() == 2


@pytest.mark.parametrize("bad,status", [
    (artifact([("k", 2, 0, 1, 1)], magic=0x12345678), hip.INVALID_PROGRAM),
    (artifact([("k", 2, 0, 1, 1)], version=2), hip.UNSUPPORTED_VERSION),
    (artifact([("k", 2, 0, 1, 1)])[:-3], hip.INVALID_PROGRAM),             # truncated
    (artifact([("k", 2, 0, 1, 1)]) + b"\0", hip.INVALID_PROGRAM),          # trailing bytes
    (artifact([("k", 2, 2, 1, 1)]), hip.INVALID_PROGRAM),                  # candidate out of range
    (artifact([("k", 2, 0, 1, 0)]), hip.INVALID_PROGRAM),                  # no samples
    (artifact([("", 2, 0, 1, 1)]), hip.INVALID_PROGRAM),                   # empty key
    (artifact([("a", 2, 0, 1, 1), ("b", 2, 5, 1, 1)]), hip.INVALID_PROGRAM),  # all or nothing
])
def test_malformed_artifacts_are_refused_and_leave_the_table(bad, status):
    hip.tuning_import(artifact([("keep", 2, 1, 9, 3)]))
    before = hip.tuning_export()
    with pytest.raises(hip.HipError) as e:
        hip.tuning_import(bad)
    assert e.value.status == status
    assert hip.tuning_export() == before


def test_row_kernel_follows_the_imported_unroll():
    prog = W.tone_program(8192, 16384)
    src = hip.plan_source(prog)
    (key, cand, count), = tuning_lines(src)
    assert key.startswith("gfx950/row/") and key.endswith("/rows=8192,cols=16384")
    # 128 threads per row: 32 element groups per thread, not cached (one pass), candidates {2, 1, 4}
    assert (cand, count) == ("0", "3") and "#pragma unroll 2\n" in src
    hip.tuning_import(artifact([(key, 3, 1, 10, 3)]))
    src = hip.plan_source(prog)
    assert tuning_lines(src) == [(key, "1", "3")]
    assert "#pragma unroll 1\n" in src and "#pragma unroll 2\n" not in src
    hip.plan_source(prog, compile=True)  # the selected candidate builds for gfx950


def test_contraction_follows_the_imported_n_tile():
    prog = W.gemm_program(8192, 8192, 8192, "bf16", "mulsum")
    src = hip.plan_source(prog)
    (key, cand, count), = tuning_lines(src)
    assert key.startswith("gfx950/gemm/") and (cand, count) == ("0", "2")
    assert "BN = 256, STAGES = 4," in src and "grid 1024 " in src
    hip.tuning_import(artifact([(key, 2, 1, 10, 3)]))
    src = hip.plan_source(prog, compile=True)   # the selected candidate builds for gfx950
    assert "BN = 128, STAGES = 4," in src and "grid 2048 " in src
    # A record for another key (or candidate count) changes nothing.
    hip.tuning_clear()
    hip.tuning_import(artifact([(key + "x", 2, 1, 10, 3), (key, 3, 1, 10, 3)]))
    assert "BN = 256, STAGES = 4," in hip.plan_source(prog)


def test_which_config_kernels_are_tunable():
    counts = {name: [int(c) for _, _, c in tuning_lines(hip.plan_source(p))] for name, p in [
        ("c1", W.tone_program(8192, 16384)), ("c2", W.logsumexp_program(32768, 8192)),
        ("c3-bf16", W.gemm_program(8192, 8192, 8192, "bf16", "mulsum")),
        ("c3-f32", W.gemm_program(8192, 8192, 8192, "f32", "mulsum")),
        ("c4", W.attention_program(32, 4096, 128, "f16"))]}
    # C2's rows are cached in registers across passes (always fully unrolled); f32 contractions and
    # attention have one launch shape.
    assert counts == {"c1": [3], "c2": [], "c3-bf16": [2], "c3-f32": [], "c4": []}


@pytest.mark.gpu
def test_tune_on_device_then_compile_takes_the_selection():
    tone = W.tone_program(64, 16384)
    tone_in = W.tone_inputs(64, 16384, seed=12)
    gemm = W.gemm_program(512, 512, 512, "bf16", "mulsum")
    gemm_in = W.gemm_inputs(512, 512, 512, "bf16", seed=13)
    assert hip.tune(tone, tone_in, repeats=5) == 1
    assert hip.tune(gemm, gemm_in, repeats=5) == 1
    assert hip.tuning_count() == 2
    art = hip.tuning_export()
    hip.tuning_clear()
    hip.tuning_import(art)
    assert hip.tuning_export() == art
    # The selected candidates still match the oracle.
    got = hip_run(tone, tone_in)[0]
    ref = oracle_run(tone, tone_in)[0]
    assert np.all(np.abs(got - ref) <= 1e-5 * np.abs(ref))
    assert_normwise(hip_run(gemm, gemm_in)[0], oracle_run(gemm, gemm_in)[0], 2e-2, "bf16", floor=None)


@pytest.mark.gpu
def test_contraction_candidate_matches_the_default_and_the_oracle():
    # The 128-column tile against the default 256, with the decoder's GELU epilogue.
    candidate = 1
    m, k, n = 512, 2048, 1024
    prog = T.define("gelu_mm", [T.spec("bf16", m=m, k=k), T.spec("bf16", k=k, n=n)],
                    lambda b, a: W.gelu(b, a[0].contract(a[1], "k"), "bf16"))
    rng = np.random.default_rng(21)
    x = W.to_dtype(rng.standard_normal((m, k)) * 0.5, "bf16")
    w = W.to_dtype(rng.standard_normal((k, n)) * 0.03, "bf16")
    default = hip_run(prog, [x, w])[0]
    (key, cand, count), = tuning_lines(hip.plan_source(prog))
    assert (cand, count) == ("0", "2")
    hip.tuning_import(artifact([(key, 2, candidate, 10, 3)]))
    assert tuning_lines(hip.plan_source(prog)) == [(key, str(candidate), "2")]
    got = hip_run(prog, [x, w])[0]
    assert np.array_equal(got, default)       # every output keeps its k order: bit-identical
    # per row, as for the decoder: GELU's negative tail sits near zero, where one bf16 step of the
    # pre-activation (a different summation order) is a large relative change of a tiny output
    assert_rowwise(got, oracle_run(prog, [x, w])[0], 2e-2, "bf16")
