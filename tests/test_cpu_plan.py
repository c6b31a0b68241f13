"""Pins the CPU baseline's fused loops (oracle/runcpu_plan.cpp: runCpu's kernel plan for C1-C4 without
materialised intermediates) against the op-by-op oracle: every output bit for bit, on small inputs
of each benchmark program, including a causal mask, bf16 truncation and NaN / -inf in the rows."""
import ctypes
import math

import numpy as np
import pytest

from accy_amd import workloads as W
from conftest import oracle_lib, oracle_run

F = ctypes.c_void_p
I = ctypes.c_int64


def lib():
    l = oracle_lib()
    l.accy_cpu_plan_tone.argtypes = [F, I, F, F, I, F]
    l.accy_cpu_plan_logsumexp.argtypes = [F, I, I, F]
    l.accy_cpu_plan_mulsum.argtypes = [F, F, I, I, I, ctypes.c_int, F]
    l.accy_cpu_plan_attention_f16.argtypes = [F, F, F, I, I, I, ctypes.c_uint16, ctypes.c_int, F]
    return l


def p(x):
    return x.ctypes.data


def test_tone_plan_equals_oracle():
    f, t, s = W.tone_inputs(64, 2048, seed=7)
    out = np.zeros(64, np.float32)
    lib().accy_cpu_plan_tone(p(f), 64, p(t), p(s), 2048, p(out))
    ref = oracle_run(W.tone_program(64, 2048), [f, t, s])[0]
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


def test_logsumexp_plan_equals_oracle():
    x = W.logsumexp_inputs(96, 1000, seed=8)[0].copy()
    x[3, 17] = np.nan
    x[5, :] = -np.inf
    x[7, 9] = np.inf
    out = np.zeros(96, np.float32)
    lib().accy_cpu_plan_logsumexp(p(x), 96, 1000, p(out))
    ref = oracle_run(W.logsumexp_program(96, 1000), [x])[0]
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_mulsum_plan_equals_oracle(dtype):
    a, b = W.gemm_inputs(24, 300, 40, dtype, seed=9)
    out = np.zeros((24, 40), np.float32 if dtype == "f32" else np.uint16)
    lib().accy_cpu_plan_mulsum(p(a), p(b), 24, 300, 40, int(dtype == "bf16"), p(out))
    ref = oracle_run(W.gemm_program(24, 300, 40, dtype, "mulsum"), [a, b])[0]
    assert np.array_equal(out.view(np.uint8), ref.view(np.uint8))


@pytest.mark.parametrize("causal", [False, True])
def test_attention_plan_equals_oracle(causal):
    q, k, v = W.attention_inputs(2, 96, 32, "f16", seed=10)
    out = np.zeros_like(q)
    scale = np.array([1.0 / math.sqrt(32)], np.float16).view(np.uint16)[0]
    lib().accy_cpu_plan_attention_f16(p(q), p(k), p(v), 2, 96, 32, int(scale), int(causal), p(out))
    ref = oracle_run(W.attention_program(2, 96, 32, "f16", causal=causal), [q, k, v])[0]
    assert np.array_equal(out.view(np.uint16), ref.view(np.uint16))


def test_plans_give_the_same_bits_on_one_and_many_threads():
    l = lib()
    x = W.logsumexp_inputs(64, 512, seed=11)[0]
    one, many = np.zeros(64, np.float32), np.zeros(64, np.float32)
    l.accy_cpu_set_threads(1)
    l.accy_cpu_plan_logsumexp(p(x), 64, 512, p(one))
    l.accy_cpu_set_threads(8)
    l.accy_cpu_plan_logsumexp(p(x), 64, 512, p(many))
    assert np.array_equal(one, many)


@pytest.mark.parametrize("shape", [(2, 8, 16, 2, 8, 32), (1, 24, 64, 4, 16, 96)])
def test_decoder_plan_equals_oracle(shape):
    """The C5 block's plan (norm rows with the squared prologue fused, serial-k dots, per-row causal
    softmax, GELU, residuals) gives the op-by-op oracle's bits, with inputs of the benchmark's
    distribution and a row scaled so that the norms and softmax see large values."""
    B, S, M, H, D, FF = shape
    ins = W.decoder_inputs(B, S, M, H, D, FF, seed=12)
    x = W.bf16_to_f32(ins[0]).copy()
    x[0, 1] *= 40.0
    ins[0] = W.to_dtype(x, "bf16")
    out = np.zeros((B, S, M), np.uint16)
    l = lib()
    l.accy_cpu_plan_decoder_bf16.argtypes = [F] * 9 + [I] * 6 + [F]
    l.accy_cpu_plan_decoder_bf16(*[p(a) for a in ins], B, S, M, H, D, FF, p(out))
    ref = oracle_run(W.decoder_program(B, S, M, H, D, FF), ins)[0]
    assert np.array_equal(out, ref)
