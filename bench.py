"""Benchmark of the MI355X execution target on the reference's measured configurations.

``python bench.py [--gpus 1] [--steps K] [--warmup W] [--config all]`` prints ONE JSON line.

* A step is one launch of the compiled program (``Hip.launch_device``) over inputs already resident
  in HBM, on one HIP stream; K steps are timed between two synchronisations.
* ``value`` is the whole-job throughput of the step: algorithmic bytes (HBM-bound configs) or
  algorithmic FLOP (MFMA / VALU-bound configs) per second, with the per-config figures of the
  measurement plan.
* ``roofline`` is for the dominant kernel: its algorithmic bytes or FLOP per launch divided by its
  average duration, from HIP events on the launch stream: around the timed region for a one-kernel
  program, around that kernel in each of K back-to-back steps otherwise. ``traffic`` is the HBM
  bytes per launch measured with rocprofv3 counters (FETCH_SIZE, WRITE_SIZE, calibrated on a copy
  kernel) and committed in profiles/traffic.json; null for a workload not measured there.
* ``cpu_baseline`` is the runCpu restatement (oracle/) timed on this host on a bounded sample of the
  same workload, then scaled to the metric's unit (kind "port"): runCpu's kernel plan as fused loops
  (oracle/runcpu_plan.cpp); min(nproc, 16) host threads and one thread.

The headline workload is C2 (row-wise logsumexp, x f32[32768, 8192]), the configuration the metric
is quoted on that fits one GPU: ``value``, ``roofline`` and ``cpu_baseline`` are C2's. The default run
(``--config all``) measures every config in the same process and adds ``configs``: per config the step
time, throughput, the dominant kernel's roofline fraction and HBM traffic, and a bounded CPU baseline.
``--config NAME`` measures one config alone (its line then has no ``configs``).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import re
import subprocess
import sys
import threading
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from accy_amd import hip  # noqa: E402
from accy_amd import tensor as T  # noqa: E402
from accy_amd import workloads as W  # noqa: E402

METRIC = "GB/s & TFLOP/s per config as % of MI355X roofline; speedup vs runCpu"
HBM_PEAK_GBS = 8000.0
# Dense peaks of MI355X as BASELINE.md's roofline table states them (bf16 / f16 2516.6 TFLOP/s: 256 CUs x
# 4 SIMDs x 1024 FLOP per clock x 2.4 GHz).
MFMA_PEAK_TFLOPS = {"f32": 157.3, "bf16": 2516.6, "f16": 2516.6}
VALU_PEAK_TFLOPS = 157.3


TRAFFIC = Path(__file__).resolve().parent / "profiles" / "traffic.json"


def measured_traffic(config: str, label: str):
    """HBM bytes per launch of one kernel from the committed rocprofv3 counter measurement
    (FETCH_SIZE and WRITE_SIZE, calibrated on a copy kernel), or None when not measured. A label with
    a fused epilogue (+) or a grouped launch (&) is keyed by its first value."""
    try:
        table = json.loads(TRAFFIC.read_text()).get(config, {})
    except (OSError, ValueError):
        return None
    return table.get(label, table.get(re.split("[+&]", label)[0]))


VALU = Path(__file__).resolve().parent / "profiles" / "valu.json"
# Wave64 VALU instructions per second at the published FP32 vector peak: 157.3 TFLOP/s is 2 FLOP x 64
# lanes x 2 FMA instructions per CU per clock (256 CUs at 2.4 GHz); two waves on a SIMD reach about
# that rate with independent FMAs.
VALU_ISSUE_PEAK = 2 * 256 * 2.4e9


def measured_valu(config: str, label: str):
    """VALU instructions (wave64) per launch of one kernel from the committed rocprofv3
    SQ_INSTS_VALU measurement, or None."""
    try:
        table = json.loads(VALU.read_text()).get(config, {})
    except (OSError, ValueError):
        return None
    return table.get(label, table.get(re.split("[+&]", label)[0]))


def decoder_flops(batch, seq, model, heads, hd, ffn):
    """Useful flops of one decoder block: the four projections, the two MLP contractions, and causal
    attention over the key <= query pairs (scores and P.V, 2 flops per multiply-add each)."""
    tokens = batch * seq
    proj = 2.0 * tokens * model * heads * hd * 4
    mlp = 2.0 * tokens * model * ffn * 2
    pairs = seq * (seq + 1) / 2.0
    attn = 4.0 * batch * heads * pairs * hd
    return proj + mlp + attn


def config_table():
    """Per config: program, inputs, algorithmic work, unit, bound, oracle sample."""
    return {
        "c1-tone": dict(
            make=lambda: (W.tone_program(8192, 16384), W.tone_inputs(8192, 16384, seed=1)),
            dtype="f32", unit="GFLOP/s", bound="valu", work=4.0 * 8192 * 16384, peak=VALU_PEAK_TFLOPS * 1000,
            sample=lambda: (W.tone_program(256, 16384), W.tone_inputs(256, 16384, seed=1), 4.0 * 256 * 16384),
            sample_desc="256 of 8192 guesses x 16384 points", workload=dict(guesses=8192, points=16384)),
        "c2-lse": dict(
            make=lambda: (W.logsumexp_program(32768, 8192), W.logsumexp_inputs(32768, 8192, seed=2)),
            dtype="f32", unit="GB/s", bound="hbm", work=32768 * 8192 * 4 + 32768 * 4, peak=HBM_PEAK_GBS,
            sample=lambda: (W.logsumexp_program(4096, 8192), W.logsumexp_inputs(4096, 8192, seed=2),
                            4096 * 8192 * 4 + 4096 * 4),
            sample_desc="4096 of 32768 rows x 8192 features", workload=dict(rows=32768, features=8192)),
        "c3-gemm-f32": dict(
            make=lambda: (W.gemm_program(8192, 8192, 8192, "f32", "mulsum"), W.gemm_inputs(8192, 8192, 8192, "f32")),
            dtype="f32", unit="TFLOP/s", bound="mfma", work=2.0 * 8192 ** 3, peak=MFMA_PEAK_TFLOPS["f32"],
            sample=lambda: (W.gemm_program(16, 8192, 8192, "f32", "mulsum"), W.gemm_inputs(16, 8192, 8192, "f32"),
                            2.0 * 16 * 8192 * 8192),
            sample_desc="16 of 8192 rows of A", workload=dict(m=8192, k=8192, n=8192, spelling="mul+sum")),
        "c3-gemm-bf16": dict(
            make=lambda: (W.gemm_program(8192, 8192, 8192, "bf16", "mulsum"), W.gemm_inputs(8192, 8192, 8192, "bf16")),
            dtype="bf16", unit="TFLOP/s", bound="mfma", work=2.0 * 8192 ** 3, peak=MFMA_PEAK_TFLOPS["bf16"],
            sample=lambda: (W.gemm_program(16, 8192, 8192, "bf16", "mulsum"), W.gemm_inputs(16, 8192, 8192, "bf16"),
                            2.0 * 16 * 8192 * 8192),
            sample_desc="16 of 8192 rows of A", workload=dict(m=8192, k=8192, n=8192, spelling="mul+sum")),
        "c4-attention": dict(
            make=lambda: (W.attention_program(32, 4096, 128, "f16"), W.attention_inputs(32, 4096, 128, "f16")),
            dtype="f16", unit="TFLOP/s", bound="mfma", work=4.0 * 32 * 4096 * 4096 * 128,
            peak=MFMA_PEAK_TFLOPS["f16"],
            sample=lambda: (W.attention_program(1, 1024, 128, "f16"), W.attention_inputs(1, 1024, 128, "f16"),
                            4.0 * 1 * 1024 * 1024 * 128),
            sample_desc="1 head x 1024 queries x 1024 keys", workload=dict(heads=32, seq=4096, dim=128)),
        # Not a measured config: a plain copy of 1 GiB (y = x * 1), whose HBM counters calibrate the
        # FETCH_SIZE / WRITE_SIZE readings of the other kernels.
        "calib-copy": dict(
            make=lambda: (T.define("copy", [T.spec("f32", row=32768, feature=8192)],
                                   lambda b, a: a[0].mul(b.full_float(T.Type("f32", ()), 1.0))),
                          W.logsumexp_inputs(32768, 8192, seed=2)),
            dtype="f32", unit="GB/s", bound="hbm", work=2 * 32768 * 8192 * 4, peak=HBM_PEAK_GBS,
            sample=lambda: (T.define("copy", [T.spec("f32", row=1024, feature=8192)],
                                     lambda b, a: a[0].mul(b.full_float(T.Type("f32", ()), 1.0))),
                            W.logsumexp_inputs(1024, 8192, seed=2), 2 * 1024 * 8192 * 4),
            sample_desc="1024 rows", workload=dict(rows=32768, features=8192)),
        # Not a measured config: a kernel with almost no work (y = x * 1 over 64 f32, one workgroup),
        # whose GRBM_GUI_ACTIVE reading is the counter window around a dispatch beyond the kernel itself.
        "calib-empty": dict(
            make=lambda: (T.define("empty", [T.spec("f32", i=64)],
                                   lambda b, a: a[0].mul(b.full_float(T.Type("f32", ()), 1.0))),
                          [np.arange(64, dtype=np.float32)]),
            dtype="f32", unit="GB/s", bound="hbm", work=2 * 64 * 4, peak=HBM_PEAK_GBS,
            sample=lambda: (T.define("empty", [T.spec("f32", i=64)],
                                     lambda b, a: a[0].mul(b.full_float(T.Type("f32", ()), 1.0))),
                            [np.arange(64, dtype=np.float32)], 2 * 64 * 4),
            sample_desc="64 elements", workload=dict(elements=64)),
        "c5-decoder": dict(
            make=lambda: (W.decoder_program(), W.decoder_inputs()),
            dtype="bf16", unit="TFLOP/s", bound="mfma", work=decoder_flops(4, 2048, 2048, 16, 128, 8192), peak=MFMA_PEAK_TFLOPS["bf16"],
            sample=lambda: (W.decoder_program(1, 128), W.decoder_inputs(1, 128), decoder_flops(1, 128, 2048, 16, 128, 8192)),
            sample_desc="batch 1 x seq 128", workload=dict(batch=4, seq=2048, model=2048, heads=16, hd=128, ffn=8192)),
    }


CPU_SHARE = 16   # host threads one GPU's job may use on the measurement boxes


def host_cores() -> dict:
    """What the host reports: `nproc` (the cores this process may run on) and os.cpu_count()."""
    try:
        nproc = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        nproc = os.cpu_count() or 1
    return dict(nproc=nproc, cpu_count=os.cpu_count() or 1)


def cpu_threads() -> int:
    """Host threads for the CPU legs: $ACCY_CPU_THREADS, else `nproc` capped at 16. The boxes this
    runs on give one GPU's job a share of 16 host threads whatever `nproc` reports (the rest belong to
    the other GPUs' jobs), so more threads would time contention, not runCpu."""
    return min(int(os.environ.get("ACCY_CPU_THREADS", "0")) or host_cores()["nproc"], CPU_SHARE)


def plan_runner(name: str, lib, prog, ins):
    """The CPU baseline's computation for one config: runCpu's kernel plan as fused loops
    (oracle/runcpu_plan.cpp: intermediates only where the plan has them; each output's arithmetic is
    the op-by-op oracle's, which tests/test_cpu_plan.py checks bit for bit) for C1-C5, the op-by-op
    oracle otherwise. Returns (callable, description)."""
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    ptr = lambda x: ctypes.c_void_p(x.ctypes.data)
    if name == "c1-tone":
        f, t, s = ins
        out = np.zeros(f.shape[0], np.float32)
        lib.accy_cpu_plan_tone.argtypes = [vp, i64, vp, vp, i64, vp]
        return (lambda: lib.accy_cpu_plan_tone(ptr(f), f.shape[0], ptr(t), ptr(s), t.shape[0], ptr(out)),
                "fused reduction (runCpu's plan)")
    if name == "c2-lse":
        x = ins[0]
        out = np.zeros(x.shape[0], np.float32)
        lib.accy_cpu_plan_logsumexp.argtypes = [vp, i64, i64, vp]
        return (lambda: lib.accy_cpu_plan_logsumexp(ptr(x), x.shape[0], x.shape[1], ptr(out)),
                "max reduction, fused exp-sum reduction, log + add (runCpu's plan)")
    if name in ("c3-gemm-f32", "c3-gemm-bf16"):
        a, b = ins
        out = np.zeros((a.shape[0], b.shape[1]), a.dtype)
        lib.accy_cpu_plan_mulsum.argtypes = [vp, vp, i64, i64, i64, ctypes.c_int, vp]
        bf = int(name.endswith("bf16"))
        return (lambda: lib.accy_cpu_plan_mulsum(ptr(a), ptr(b), a.shape[0], a.shape[1], b.shape[1], bf, ptr(out)),
                "interior reduction of rounded products, serial k (runCpu's plan)")
    if name == "c4-attention":
        q, k, v = ins
        out = np.zeros_like(q)
        scale = int(np.array([1.0 / math.sqrt(q.shape[2])], np.float16).view(np.uint16)[0])
        lib.accy_cpu_plan_attention_f16.argtypes = [vp, vp, vp, i64, i64, i64, ctypes.c_uint16, ctypes.c_int, vp]
        return (lambda: lib.accy_cpu_plan_attention_f16(ptr(q), ptr(k), ptr(v), q.shape[0], q.shape[1], q.shape[2],
                                                         scale, 0, ptr(out)),
                "per query row: scores, per-op f16 softmax, P.V (runCpu's operations, f16 extension)")
    if name == "c5-decoder":
        B, S, M = ins[0].shape
        H, D = ins[2].shape[1], ins[2].shape[2]
        FF = ins[7].shape[1]
        out = np.zeros((B, S, M), np.uint16)
        lib.accy_cpu_plan_decoder_bf16.argtypes = [vp] * 9 + [i64] * 6 + [vp]
        return (lambda: lib.accy_cpu_plan_decoder_bf16(*[ptr(a) for a in ins], B, S, M, H, D, FF, ptr(out)),
                "norm rows with the squared prologue fused, serial-k dots, per-row causal softmax, GELU, "
                "residuals (runCpu's plan, bf16 extension)")
    sys.path.insert(0, str(ROOT / "tests"))
    from conftest import oracle_run
    return (lambda: oracle_run(prog, ins)), "op-by-op oracle (every intermediate materialised)"


def oracle_time(name: str, cfg, budget_s: float):
    """Times the CPU baseline on the config's bounded sample, with all host threads and with one
    thread (runCpu launches single-threaded); each leg until `budget_s` is spent (at most 50 runs).
    Per-output order makes both legs bit-identical."""
    sys.path.insert(0, str(ROOT / "tests"))
    from conftest import oracle_lib
    prog, ins, work = cfg["sample"]()
    lib = oracle_lib()
    run, plan = plan_runner(name, lib, prog, ins)
    threads = cpu_threads()
    scale = 1e9 if cfg["unit"] in ("GB/s", "GFLOP/s") else 1e12

    def timed(n):
        lib.accy_cpu_set_threads(n)
        times = []
        start = time.perf_counter()
        while True:
            t0 = time.perf_counter()
            run()
            times.append(time.perf_counter() - t0)
            if time.perf_counter() - start >= budget_s or len(times) >= 50:
                break
        return float(np.median(times)), len(times)

    t_all, n_all = timed(threads)
    t_one, n_one = timed(1)
    lib.accy_cpu_set_threads(threads)
    hc = host_cores()
    return dict(value=work / t_all / scale, unit=cfg["unit"], cores=threads, kind="port", plan=plan,
                nproc=hc["nproc"], cpu_count=hc["cpu_count"],
                cores_note=f"min(nproc, {CPU_SHARE}): the host-thread share of one GPU's job on these boxes",
                sample=f"{cfg['sample_desc']}; median of {n_all} runs, {t_all:.3f} s each",
                single_core=dict(value=work / t_one / scale, cores=1,
                                 sample=f"median of {n_one} runs, {t_one:.3f} s each"))


def board_sample():
    """Board power (W) and the mean graphics clock (MHz) over the XCDs from amd-smi, or None."""
    try:
        r = subprocess.run(["amd-smi", "metric", "-p", "-c", "--json"], capture_output=True, text=True, timeout=30)
        d = json.loads(r.stdout)
        g = d["gpu_data"][0] if isinstance(d, dict) else d[0]
        clocks = [v["clk"]["value"] for k, v in g["clock"].items() if k.startswith("gfx_") and isinstance(v, dict)]
        return dict(power_w=float(g["power"]["socket_power"]["value"]), gfx_mhz=sum(clocks) / len(clocks))
    except Exception:  # no amd-smi, or a format it does not give here
        return None


def power_leg(step, stream, seconds: float = 1.2):
    """Board power and clock under the config's sustained back-to-back steps (after the timed and
    profiled steps, outside both): steps run in ~20 ms chunks for `seconds` while a thread samples
    amd-smi once, past the first half."""
    out = {}
    t0 = time.perf_counter()

    def sampler():
        time.sleep(seconds / 2)
        out["sample"] = board_sample()

    th = threading.Thread(target=sampler)
    th.start()
    while time.perf_counter() - t0 < seconds or th.is_alive():
        t = time.perf_counter()
        step()
        stream.synchronize()
        n = max(1, int(0.02 / max(time.perf_counter() - t, 1e-6)))
        for _ in range(n):
            step()
        stream.synchronize()
    th.join()
    return out.get("sample")


def measure(name: str, cfg: dict, steps: int, warmup: int, warmup_s: float, power: bool = False) -> dict:
    """Runs one config on the GPU: K timed steps over HBM-resident inputs, then K profiled steps for
    the per-kernel durations. Returns the step time, the throughput and the dominant kernel's
    roofline entry."""
    prog, ins = cfg["make"]()
    # Inputs are copied into HBM before the timed region; outputs stay on the device.
    dins = [hip.DeviceBuffer.from_array(x) for x in ins]
    douts = [hip.DeviceBuffer(t.byte_count()) for t in prog.output_types()]
    del ins
    stream = hip.Stream()
    ex = hip.Hip(prog)
    iptr = [b.ptr for b in dins]
    optr = [b.ptr for b in douts]

    def step():
        ex.launch_device(iptr, optr, stream.handle)

    # Warmup in chunks of about 20 ms of device work, one synchronisation per chunk (a gap between
    # launches would let the clock recover and the timed steps would not see the sustained state).
    t_w = time.perf_counter()
    step()
    stream.synchronize()
    done = 1
    chunk = max(1, int(0.02 / max(time.perf_counter() - t_w, 1e-6)))
    while done < warmup or time.perf_counter() - t_w < warmup_s:
        for _ in range(chunk):
            step()
        done += chunk
        stream.synchronize()
    start, end = hip.Event(), hip.Event()
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        step()
    end.record(stream)
    stream.synchronize()
    elapsed = time.perf_counter() - t0
    event_ms = start.elapsed_ms(end) / steps
    ms_per_step = max(elapsed * 1e3 / steps, event_ms)

    # Per-kernel durations: HIP events recorded on the launch stream around each kernel, over the
    # same number of back-to-back steps (no synchronisation between them).
    ex.set_profiling(True)
    for _ in range(steps):
        step()
    per_kernel = {k.label: k for k in ex.kernels()}
    ex.set_profiling(False)
    dominant = max(per_kernel.items(), key=lambda kv: kv[1].mean_ms)
    dom_stats = dominant[1]
    # A one-kernel program's kernel duration is the events around the timed region over the steps
    # (events around each launch add a few microseconds each); several kernels need their own events.
    single = len(per_kernel) == 1
    dom_ms = event_ms if single else float(dom_stats.mean_ms)
    scale = 1e9 if cfg["unit"] in ("GB/s", "GFLOP/s") else 1e12
    value = cfg["work"] / (ms_per_step * 1e-3) / scale
    # The roofline is the dominant kernel's: a one-kernel program's work is the config's; in a
    # program of several kernels it is that kernel's own algorithmic bytes or flops.
    if cfg["bound"] == "hbm":
        work = cfg["work"] if single else dom_stats.algorithmic_bytes
        achieved = work / (dom_ms * 1e-3) / 1e9
        roof = dict(bound="hbm", achieved=achieved, peak=cfg["peak"], unit="GB/s", frac=achieved / cfg["peak"],
                    traffic=measured_traffic(name, dominant[0]), kernel=dominant[0], kernel_ms=dom_ms)
    else:
        work = cfg["work"] if single else dom_stats.algorithmic_flops
        achieved = work / (dom_ms * 1e-3) / 1e12
        peak = cfg["peak"] / 1000.0 if cfg["unit"] == "GFLOP/s" else cfg["peak"]
        roof = dict(bound=cfg["bound"], achieved=achieved, peak=peak, unit="TFLOP/s", frac=achieved / peak,
                    traffic=measured_traffic(name, dominant[0]), kernel=dominant[0], kernel_ms=dom_ms)
    board = power_leg(step, stream) if power else None
    insts = measured_valu(name, dominant[0])
    if insts is not None:
        # VALU issue fraction (instructions x 64 lanes per second against 256 CUs x 2.4 GHz x 64)
        roof["valu_issue"] = dict(insts_per_launch=insts, frac=insts / (dom_ms * 1e-3) / VALU_ISSUE_PEAK)
    ex.deinit()
    for b in dins + douts:
        b.free()
    stream.destroy()
    r = dict(value=value, unit=cfg["unit"], ms_per_step=ms_per_step, dtype=cfg["dtype"], warmup_run=done,
             workload=dict(workload=name, **cfg["workload"]), roofline=roof,
             kernels={lbl: float(k.mean_ms) for lbl, k in per_kernel.items()})
    if power:
        r["board"] = board
    return r


HEADLINE = "c2-lse"
ALL = ["c2-lse", "c1-tone", "c3-gemm-f32", "c3-gemm-bf16", "c4-attention", "c5-decoder"]


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # Under sustained back-to-back launches the power controller first lowers the clock (a bf16 8192^3
    # contraction goes from about 0.82 to 1.08 ms per launch within four launches, the C2 row kernel
    # from 0.156 to 0.213 ms within 20) and then settles over some milliseconds. Warmup runs at least
    # --warmup steps and at least --warmup-seconds of them, so the timed steps measure the sustained
    # steady state. The line reports the requested --warmup as `warmup` and the steps actually run as
    # `warmup_steps_run`.
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--warmup-seconds", type=float, default=0.2)
    ap.add_argument("--config", default="all",
                    help="'all' (the headline C2 line plus every config under 'configs') or one config")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    ap.add_argument("--power", action="store_true",
                    help="after each config's timed steps, sample board power and clock (amd-smi) under sustained steps")
    ap.add_argument("--cpu-budget", type=float, default=6.0,
                    help="seconds per CPU leg for the headline config (the other configs get a third)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for {args.gpus}); the target runs on a single MI355X "
              "and has no multi-GPU path.", file=sys.stderr)
        return 2
    cfgs = config_table()
    names = ALL if args.config == "all" else [args.config]
    head = HEADLINE if args.config == "all" else args.config
    results = {}
    for name in names:
        print(f"bench: {name}", file=sys.stderr, flush=True)
        r = measure(name, cfgs[name], args.steps, args.warmup, args.warmup_seconds, args.power)
        budget = args.cpu_budget if name == head else args.cpu_budget / 3
        r["cpu_baseline"] = None if args.no_cpu else oracle_time(name, cfgs[name], budget)
        results[name] = r
    h = results[head]
    line = {
        "metric": METRIC, "value": h["value"], "unit": h["unit"], "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "warmup_steps_run": h["warmup_run"], "warmup_seconds": args.warmup_seconds,
        "ms_per_step": h["ms_per_step"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": h["dtype"], "data": "synthetic (seeded SplitMix64)",
        "config": h["workload"], "roofline": h["roofline"], "cpu_baseline": h["cpu_baseline"],
        "kernels": h["kernels"],
    }
    if args.power:
        line["board"] = h["board"]
    if len(names) > 1:
        line["configs"] = {
            n: dict(ms=r["ms_per_step"], value=r["value"], unit=r["unit"], dtype=r["dtype"], warmup_steps_run=r["warmup_run"],
                    bound=r["roofline"]["bound"],
                    kernel=r["roofline"]["kernel"], kernel_ms=r["roofline"]["kernel_ms"],
                    achieved=r["roofline"]["achieved"], peak=r["roofline"]["peak"],
                    roofline_unit=r["roofline"]["unit"], frac=r["roofline"]["frac"],
                    traffic=r["roofline"]["traffic"], valu_issue=r["roofline"].get("valu_issue"),
                    cpu_baseline=r["cpu_baseline"], kernels=r["kernels"], **({"board": r["board"]} if args.power else {}))
            for n, r in results.items()}
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
