"""The programs and seeded inputs of the five measured configurations.

Each program is recorded through the tracer exactly as a user of the reference would write it with
``tensor.define`` (the traced op sequences are those derived from builder.zig for each config), and
its inputs come from one SplitMix64 stream per config:

* uniform: ``(u >> 40) * 2^-24`` scaled to [a, b);
* normal: Box-Muller in f64 from two uniforms, then rounded to the target dtype (nearest even).

C1 tone     frequency f32[guess] ~ U(0.5, 5); time[i] = 0.25 i; sample = sin(3 time)
            output[guess] = sum over point of (sin(frequency*time) - sample)^2   (examples/consumer main.zig:20-27)
C2 lse      x f32[row, feature] ~ N(0,1); output[row] = max + log(sum(exp(x - max)))
C3 gemm     A[m,k], B[k,n] ~ U(-1,1); C = A.contract(B, k) or A.mul(B).sum(k)
C4 attn     Q,K,V f16[head, query|key, dim] ~ N(0,1); softmax(Q K^T * c) V, c = f16(1/sqrt(dim))
C5 decoder  pre-RMSNorm block: RMSNorm -> QKV -> causal attention -> out-proj -> residual ->
            RMSNorm -> W1 -> GELU(tanh) -> W2 -> residual, all bf16
"""
from __future__ import annotations

import math
from typing import Dict, List, Tuple

import numpy as np

from . import tensor as T

MASK64 = (1 << 64) - 1


def splitmix64(seed: int, n: int, start: int = 0) -> np.ndarray:
    """SplitMix64 outputs number start + 1 .. start + n (uint64) of the stream from ``seed``
    (vectorised; the stream is counter-based, so any window can be computed on its own)."""
    gamma = np.uint64(0x9E3779B97F4A7C15)
    idx = np.arange(start + 1, start + n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed & MASK64) + idx * gamma
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    return z


def uniform(seed: int, n: int, lo: float, hi: float) -> np.ndarray:
    """f64 uniforms in [lo, hi): 24 random bits per value."""
    u = (splitmix64(seed, n) >> np.uint64(40)).astype(np.float64) * (1.0 / (1 << 24))
    return lo + (hi - lo) * u


def _normal_pairs(seed: int, first_pair: int, pairs: int) -> np.ndarray:
    """Box-Muller values 2 first_pair .. 2 (first_pair + pairs) - 1 of the stream (f64)."""
    u = (splitmix64(seed, 2 * pairs, 2 * first_pair) >> np.uint64(40)).astype(np.float64)
    u1 = (u[0::2] + 1.0) * (1.0 / (1 << 24))
    u2 = u[1::2] * (1.0 / (1 << 24))
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * pairs)
    z[0::2] = r * np.cos(2 * math.pi * u2)
    z[1::2] = r * np.sin(2 * math.pi * u2)
    return z


def normal(seed: int, n: int) -> np.ndarray:
    """f64 standard normals, Box-Muller over pairs of uniforms in (0, 1]."""
    return _normal_pairs(seed, 0, (n + 1) // 2)[:n]


_CHUNK_PAIRS = 1 << 20


def normal_as(seed: int, n: int, dtype: str, scale: float = 1.0) -> np.ndarray:
    """``to_dtype(normal(seed, n) * scale, dtype)``, the same bytes, generated in chunks of 2^21 values
    so that the f64 temporaries stay in cache (a 2^28-value tensor takes seconds, not a minute)."""
    m = (n + 1) // 2
    out = np.empty(n, to_dtype(np.zeros(0), dtype).dtype)

    def fill(p0: int) -> None:
        pairs = min(_CHUNK_PAIRS, m - p0)
        z = _normal_pairs(seed, p0, pairs)
        if scale != 1.0:
            z = z * scale
        part = to_dtype(z[: min(2 * pairs, n - 2 * p0)], dtype)
        out[2 * p0: 2 * p0 + part.size] = part

    starts = range(0, m, _CHUNK_PAIRS)
    if len(starts) > 1:
        # numpy releases the interpreter lock inside its array operations, so chunks run in parallel
        from concurrent.futures import ThreadPoolExecutor
        with ThreadPoolExecutor(max_workers=min(8, len(starts))) as pool:
            list(pool.map(fill, starts))
    else:
        for p0 in starts:
            fill(p0)
    return out


def to_dtype(x: np.ndarray, dtype: str) -> np.ndarray:
    """Rounds f64 values to a storage dtype, nearest even (bf16 held as its 16 bits)."""
    if dtype == "f32":
        return x.astype(np.float32)
    if dtype == "f16":
        return x.astype(np.float16)
    if dtype == "bf16":
        f = x.astype(np.float32).view(np.uint32).astype(np.uint64)
        lsb = (f >> np.uint64(16)) & np.uint64(1)
        r = ((f + np.uint64(0x7FFF) + lsb) >> np.uint64(16)).astype(np.uint16)
        return r
    if dtype == "f64":
        return x.astype(np.float64)
    raise ValueError(dtype)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << np.uint32(16)).view(np.float32)


def as_f32(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return bf16_to_f32(x)
    return x.astype(np.float32)


# ---------------------------------------------------------------------------------------------
# C1: the README tone program, vectorised over guesses
# ---------------------------------------------------------------------------------------------

def mismatch(b: T.Builder, args: List[T.Value]) -> T.Value:
    """examples/consumer/src/main.zig:20-27."""
    frequency, time, sample = args
    predicted = frequency.mul(time).sin()
    difference = predicted.sub(sample)
    return difference.mul(difference).sum("point")


def tone_program(guesses: int = 8192, points: int = 16384, scalar: bool = False) -> T.Program:
    freq = T.spec("f32") if scalar else T.spec("f32", guess=guesses)
    return T.define("mismatch", [freq, T.spec("f32", point=points), T.spec("f32", point=points)], mismatch)


def mismatch_and_slope(b: T.Builder, args: List[T.Value]) -> List[T.Value]:
    """The README's `valueAndGrad(.wrt = frequency)` of the mismatch, vmapped over guesses
    (examples/consumer/src/main.zig:80-102; README.md:290-304): the mismatch and its derivative
    sum(2 (sin(f t) - s) cos(f t) t), written out as the two reductions the derivative program
    computes (the reference's autodiff is not available here, so its exact op order is not)."""
    frequency, time, sample = args
    phase = frequency.mul(time)
    difference = phase.sin().sub(sample)
    value = difference.mul(difference).sum("point")
    slope = difference.mul(b.full_float(T.Type("f32", ()), 2.0)).mul(phase.cos()).mul(time).sum("point")
    return [value, slope]


def tone_value_and_slope_program(guesses: int = 8, points: int = 16) -> T.Program:
    specs = [T.spec("f32", guess=guesses), T.spec("f32", point=points), T.spec("f32", point=points)]
    return T.define("mismatch_and_slope", specs, mismatch_and_slope)


def tone_inputs(guesses: int = 8192, points: int = 16384, seed: int = 1) -> List[np.ndarray]:
    frequency = uniform(seed, guesses, 0.5, 5.0).astype(np.float32)
    time = (np.arange(points, dtype=np.float32) * np.float32(0.25)).astype(np.float32)
    sample = np.sin(np.float32(3.0) * time).astype(np.float32)
    return [frequency, time, sample]


def readme_tone() -> Tuple[np.ndarray, np.ndarray]:
    """The README's 16-point tone: time[i] = 0.25 i (f32), sample = sinf(3 time) (main.zig:41-50)."""
    time = (np.arange(16, dtype=np.float32) * np.float32(0.25)).astype(np.float32)
    sample = np.sin(np.float32(3.0) * time).astype(np.float32)
    return time, sample


# ---------------------------------------------------------------------------------------------
# C2: row-wise logsumexp
# ---------------------------------------------------------------------------------------------

def logsumexp_body(b: T.Builder, args: List[T.Value]) -> T.Value:
    x = args[0]
    m = x.max("feature")
    s = x.sub(m).exp().sum("feature")
    return m.add(s.log())


def logsumexp_program(rows: int = 32768, features: int = 8192, dtype: str = "f32") -> T.Program:
    return T.define("logsumexp", [T.spec(dtype, row=rows, feature=features)], logsumexp_body)


def logsumexp_inputs(rows: int = 32768, features: int = 8192, seed: int = 2, dtype: str = "f32") -> List[np.ndarray]:
    return [normal_as(seed, rows * features, dtype).reshape(rows, features)]


# ---------------------------------------------------------------------------------------------
# C3: dense contraction
# ---------------------------------------------------------------------------------------------

def gemm_program(m: int = 8192, k: int = 8192, n: int = 8192, dtype: str = "f32", spelling: str = "contract") -> T.Program:
    def body(b, args):
        a, bb = args
        if spelling == "contract":
            return a.contract(bb, "k")
        return a.mul(bb).sum("k")
    return T.define("gemm", [T.spec(dtype, m=m, k=k), T.spec(dtype, k=k, n=n)], body)


def gemm_inputs(m: int = 8192, k: int = 8192, n: int = 8192, dtype: str = "f32", seed: int = 3) -> List[np.ndarray]:
    a = to_dtype(uniform(seed, m * k, -1.0, 1.0), dtype).reshape(m, k)
    b = to_dtype(uniform(seed + 1000, k * n, -1.0, 1.0), dtype).reshape(k, n)
    return [a, b]


# ---------------------------------------------------------------------------------------------
# C4: attention
# ---------------------------------------------------------------------------------------------

def attention_body(dtype: str, dim: int, causal: bool = False):
    def body(b: T.Builder, args: List[T.Value]) -> T.Value:
        q, k, v = args
        k = k.rename("query", "key") if k.ty.find("query") is not None else k
        v = v.rename("query", "key") if v.ty.find("query") is not None else v
        s = q.contract(k, "dim")
        c = b.full_float(T.Type(dtype, ()), 1.0 / math.sqrt(dim))
        s = s.mul(c)
        if causal:
            qi = b.iota("i32", "query", *[d for d in s.ty.dims if d[0] == "query"])
            ki = b.iota("i32", "key", *[d for d in s.ty.dims if d[0] == "key"])
            mask = qi.compare("ge", ki)
            ninf = b.full_float(T.Type(dtype, ()), -math.inf)
            s = mask.select(s, ninf)
        mx = s.max("key")
        e = s.sub(mx).exp()
        p = e.div(e.sum("key"))
        return p.contract(v, "key")
    return body


def attention_program(heads: int = 32, seq: int = 4096, dim: int = 128, dtype: str = "f16",
                      causal: bool = False) -> T.Program:
    specs = [T.spec(dtype, head=heads, query=seq, dim=dim), T.spec(dtype, head=heads, key=seq, dim=dim),
             T.spec(dtype, head=heads, key=seq, dim=dim)]
    return T.define("attention", specs, attention_body(dtype, dim, causal))


def attention_inputs(heads: int = 32, seq: int = 4096, dim: int = 128, dtype: str = "f16", seed: int = 4) -> List[np.ndarray]:
    n = heads * seq * dim
    return [normal_as(seed + 100 * i, n, dtype).reshape(heads, seq, dim) for i in range(3)]


# ---------------------------------------------------------------------------------------------
# C5: decoder block
# ---------------------------------------------------------------------------------------------

GELU_C = 0.7978845608028654  # sqrt(2/pi), src/kernel/library/fused.zig:471-478
GELU_A = 0.044715


def rms_norm(b: T.Builder, x: T.Value, g: T.Value, axis: str, dtype: str, eps: float = 1e-5) -> T.Value:
    ms = x.mul(x).mean(axis)
    denom = ms.add(b.full_float(T.Type(dtype, ()), eps)).sqrt()
    return x.div(denom).mul(g)


def gelu(b: T.Builder, x: T.Value, dtype: str) -> T.Value:
    """0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))."""
    s = lambda v: b.full_float(T.Type(dtype, ()), v)
    inner = x.add(x.mul(x).mul(x).mul(s(GELU_A))).mul(s(GELU_C))
    return x.mul(s(0.5)).mul(inner.tanh().add(s(1.0)))


def decoder_program(batch: int = 4, seq: int = 2048, model: int = 2048, heads: int = 16, hd: int = 128,
                    ffn: int = 8192, dtype: str = "bf16") -> T.Program:
    def body(b: T.Builder, args: List[T.Value]) -> T.Value:
        x, g1, wq, wk, wv, wo, g2, w1, w2 = args
        h = rms_norm(b, x, g1, "model", dtype)
        q = h.contract(wq, "model")                       # [batch, seq, head, hd]
        k = h.contract(wk, "model").rename("seq", "key")  # [batch, key, head, hd]
        v = h.contract(wv, "model").rename("seq", "key")
        s = q.contract(k, "hd")                           # [batch, seq, head, key]
        s = s.mul(b.full_float(T.Type(dtype, ()), 1.0 / math.sqrt(hd)))
        qi = b.iota("i32", "seq", ("seq", seq), ("key", seq))
        ki = b.iota("i32", "key", ("seq", seq), ("key", seq))
        s = qi.compare("ge", ki).select(s, b.full_float(T.Type(dtype, ()), -math.inf))
        mx = s.max("key")
        e = s.sub(mx).exp()
        p = e.div(e.sum("key"))
        o = p.contract(v, "key")                          # [batch, seq, head, hd]
        y = o.contract(wo, ("head", "hd"))                # [batch, seq, model]
        x1 = x.add(y)
        h2 = rms_norm(b, x1, g2, "model", dtype)
        f = gelu(b, h2.contract(w1, "model"), dtype)      # [batch, seq, ffn]
        return x1.add(f.contract(w2, "ffn"))
    specs = [T.spec(dtype, batch=batch, seq=seq, model=model), T.spec(dtype, model=model),
             T.spec(dtype, model=model, head=heads, hd=hd), T.spec(dtype, model=model, head=heads, hd=hd),
             T.spec(dtype, model=model, head=heads, hd=hd), T.spec(dtype, head=heads, hd=hd, model=model),
             T.spec(dtype, model=model), T.spec(dtype, model=model, ffn=ffn), T.spec(dtype, ffn=ffn, model=model)]
    return T.define("decoder_block", specs, body)


def decoder_inputs(batch: int = 4, seq: int = 2048, model: int = 2048, heads: int = 16, hd: int = 128,
                   ffn: int = 8192, dtype: str = "bf16", seed: int = 5) -> List[np.ndarray]:
    def w(i, *shape, std=0.02):
        return normal_as(seed + 100 * i, int(np.prod(shape)), dtype, std).reshape(shape)
    ones = lambda n: to_dtype(np.ones(n), dtype)
    return [w(0, batch, seq, model, std=1.0), ones(model), w(1, model, heads, hd), w(2, model, heads, hd),
            w(3, model, heads, hd), w(4, heads, hd, model), ones(model), w(5, model, ffn), w(6, ffn, model)]


CONFIGS: Dict[str, dict] = {
    "c1-tone": dict(program=tone_program, inputs=tone_inputs, kw=dict(guesses=8192, points=16384)),
    "c2-lse": dict(program=logsumexp_program, inputs=logsumexp_inputs, kw=dict(rows=32768, features=8192)),
    "c3-gemm-f32": dict(program=gemm_program, inputs=gemm_inputs, kw=dict(m=8192, k=8192, n=8192, dtype="f32")),
    "c3-gemm-bf16": dict(program=gemm_program, inputs=gemm_inputs, kw=dict(m=8192, k=8192, n=8192, dtype="bf16")),
    "c4-attention": dict(program=attention_program, inputs=attention_inputs, kw=dict(heads=32, seq=4096, dim=128)),
    "c5-decoder": dict(program=decoder_program, inputs=decoder_inputs, kw=dict()),
}
