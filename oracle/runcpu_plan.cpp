// ORACLE — test infrastructure only. runCpu's kernel plan for the benchmark configurations C1-C5 as
// fused CPU loops: the CPU baseline that bench.py times beside the GPU (never the thing measured as
// the product, never called by accy_amd). Each function computes, per output element, exactly the
// operations of the traced program in the reference's order and rounding (the op-by-op evaluator in
// runcpu.cpp is the definition; tests/test_cpu_plan.py checks every function against it bit for bit),
// but without materialising the intermediates, as runCpu's fusion does:
//  * C1 tone: one fused reduction with the prologue mul, sin, sub, mul
//    (src/preparation/fusion/pass.zig:1300-1388; lowering/reduction.zig:839-901);
//  * C2 logsumexp: a max reduction, a sum reduction with the prologue sub, exp, then log and add;
//  * C3 mul + sum: the rank-3 interior reduction, per output a serial fold over k of the products
//    rounded to the element type (reduction.zig:1157-1177);
//  * C4 attention (f16): per query row the scores (dot, f32 accumulator, f16 store;
//    lowering/dot.zig:2049-2115), the scale, the optional causal select, max, sub, exp, sum, div, and
//    the product with V, every elementwise result rounded to f16 (src/eval/root.zig:14-16);
//  * C5 decoder block (bf16): each RMS norm as one row pass (the sum of squares with its prologue
//    fused, then the row's mean, epsilon, sqrt, divide and scale), the contractions as serial-k dots,
//    the causal softmax per query row as C4's, the GELU once per element, the residual adds fused
//    after their contractions; every elementwise result truncated to bf16 (Bf16.fromF32).
// Built with -ffp-contract=off (multiply and add rounded separately) and OpenMP over independent
// outputs (the per-output order is unchanged, so every thread count gives the same bits).
#include <omp.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <vector>

#include "../accy_amd/csrc/ir.hpp"

using namespace accy;

namespace {

// maxss then a NaN result replaced by the first operand (x64/scalar.zig:675-720), as runcpu.cpp.
inline float fold_max(float a, float b) {
  const float r = a > b ? a : b;
  return r != r ? a : r;
}

// bf16 as the high half of an f32; a bf16 result keeps the high 16 bits (Bf16.fromF32,
// deps/lib/compiler/gpu/abi/src/dtype.zig:6-9). Written as bit masks so the loops vectorise.
inline float bf16_value(uint16_t h) {
  const uint32_t u = (uint32_t)h << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}
inline float round_bf16(float x) {
  uint32_t u;
  std::memcpy(&u, &x, 4);
  u &= 0xffff0000u;
  std::memcpy(&x, &u, 4);
  return x;
}
inline float f16_value(uint16_t h) { return f16_bits_to_f32(h); }
inline float round_f16(float x) { return f16_bits_to_f32(f32_to_f16_bits(x)); }

}  // namespace

extern "C" {

// out[g] = sum over p of (sin(f[g] * t[p]) - s[p])^2, left to right from +0.
void accy_cpu_plan_tone(const float* f, int64_t guesses, const float* t, const float* s, int64_t points, float* out) {
#pragma omp parallel for schedule(static)
  for (int64_t g = 0; g < guesses; ++g) {
    float acc = 0.0f;
    for (int64_t p = 0; p < points; ++p) {
      const float phase = f[g] * t[p];
      const float d = sinf(phase) - s[p];
      const float sq = d * d;
      acc = acc + sq;
    }
    out[g] = acc;
  }
}

// out[r] = m + log(sum over c of exp(x[r, c] - m)), m = max over c (from -inf).
void accy_cpu_plan_logsumexp(const float* x, int64_t rows, int64_t cols, float* out) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float* row = x + r * cols;
    float m = -std::numeric_limits<float>::infinity();
    for (int64_t c = 0; c < cols; ++c) m = fold_max(m, row[c]);
    float acc = 0.0f;
    for (int64_t c = 0; c < cols; ++c) {
      const float d = row[c] - m;
      acc = acc + expf(d);
    }
    out[r] = m + logf(acc);
  }
}

// C[i, j] = sum over k of round(A[i, k] * B[k, j]), serial in k from +0 with an f32 accumulator;
// f32 (bf16 = 0) or bf16 (bf16 = 1, elements as 16-bit words, results truncated).
void accy_cpu_plan_mulsum(const void* a, const void* b, int64_t m, int64_t k, int64_t n, int bf16, void* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < m; ++i) {
    std::vector<float> acc((size_t)n, 0.0f);
    for (int64_t kk = 0; kk < k; ++kk) {
      if (bf16) {
        const float av = bf16_value(((const uint16_t*)a)[i * k + kk]);
        const uint16_t* brow = (const uint16_t*)b + kk * n;
        for (int64_t j = 0; j < n; ++j) acc[(size_t)j] = acc[(size_t)j] + round_bf16(av * bf16_value(brow[j]));
      } else {
        const float av = ((const float*)a)[i * k + kk];
        const float* brow = (const float*)b + kk * n;
        for (int64_t j = 0; j < n; ++j) {
          const float prod = av * brow[j];
          acc[(size_t)j] = acc[(size_t)j] + prod;
        }
      }
    }
    for (int64_t j = 0; j < n; ++j) {
      if (bf16) ((uint16_t*)out)[i * n + j] = f32_to_bf16_trunc(acc[(size_t)j]);
      else ((float*)out)[i * n + j] = acc[(size_t)j];
    }
  }
}

// f16 attention over [heads, seq, dim] (Q, K, V and O as 16-bit words): softmax(scale * Q K^T
// [key <= query]) V with the program's per-op f16 rounding; `scale` is the traced f16 constant.
void accy_cpu_plan_attention_f16(const uint16_t* q, const uint16_t* k, const uint16_t* v, int64_t heads, int64_t seq,
                                 int64_t dim, uint16_t scale, int causal, uint16_t* out) {
  const float c = f16_value(scale);
  const float ninf = -std::numeric_limits<float>::infinity();
  // Q, K and V widened to f32 once (exact), as the contractions do before folding.
  const size_t total = (size_t)(heads * seq * dim);
  std::vector<float> q32(total), k32(total), v32(total);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < (int64_t)total; ++i) {
    q32[(size_t)i] = f16_value(q[i]);
    k32[(size_t)i] = f16_value(k[i]);
    v32[(size_t)i] = f16_value(v[i]);
  }
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t h = 0; h < heads; ++h)
    for (int64_t qi = 0; qi < seq; ++qi) {
      std::vector<float> e((size_t)seq), o((size_t)dim, 0.0f);
      const float* qrow = q32.data() + (h * seq + qi) * dim;
      float mx = ninf;
      for (int64_t kj = 0; kj < seq; ++kj) {
        const float* krow = k32.data() + (h * seq + kj) * dim;
        float acc = 0.0f;
        for (int64_t d = 0; d < dim; ++d) {
          const float prod = qrow[d] * krow[d];
          acc = acc + prod;
        }
        float sc = round_f16(round_f16(acc) * c);
        if (causal && kj > qi) sc = ninf;
        e[(size_t)kj] = sc;
        mx = fold_max(mx, sc);
      }
      float sum = 0.0f;
      for (int64_t kj = 0; kj < seq; ++kj) {
        const float x = round_f16(expf(round_f16(e[(size_t)kj] - mx)));
        e[(size_t)kj] = x;
        sum = sum + x;
      }
      const float sum16 = round_f16(sum);
      for (int64_t kj = 0; kj < seq; ++kj) {
        const float p = round_f16(e[(size_t)kj] / sum16);
        const float* vrow = v32.data() + (h * seq + kj) * dim;
        for (int64_t d = 0; d < dim; ++d) {
          const float prod = p * vrow[d];
          o[(size_t)d] = o[(size_t)d] + prod;
        }
      }
      uint16_t* orow = out + (h * seq + qi) * dim;
      for (int64_t d = 0; d < dim; ++d) orow[d] = f32_to_f16_bits(o[(size_t)d]);
    }
}

}  // extern "C"

namespace {

// A traced bf16 constant: the f32 value of the program's double, truncated (Bf16.fromF32).
inline float bf16_const(double v) { return round_bf16((float)v); }

// One RMS norm row over `m` elements (workloads.rms_norm: x * x, mean, + eps, sqrt, x / that, * g),
// bf16 results as f32 values.
void rms_row(const float* x, const float* g, int64_t m, float count, float eps, float* out) {
  float acc = 0.0f;
  for (int64_t i = 0; i < m; ++i) acc = acc + round_bf16(x[i] * x[i]);
  const float den = round_bf16(sqrtf(round_bf16(round_bf16(round_bf16(acc) / count) + eps)));
  for (int64_t i = 0; i < m; ++i) out[i] = round_bf16(round_bf16(x[i] / den) * g[i]);
}

// out[r, j] = bf16(sum over k of a[r, k] * w[k, j]) for r < rows, serial in k with an f32
// accumulator (the products not rounded: lowering/dot.zig's acc + a * b).
void dot_rows(const float* a, const float* w, int64_t rows, int64_t k, int64_t n, float* out) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    std::vector<float> acc((size_t)n, 0.0f);
    for (int64_t kk = 0; kk < k; ++kk) {
      const float av = a[r * k + kk];
      const float* wr = w + kk * n;
      for (int64_t j = 0; j < n; ++j) {
        const float prod = av * wr[j];
        acc[(size_t)j] = acc[(size_t)j] + prod;
      }
    }
    for (int64_t j = 0; j < n; ++j) out[r * n + j] = round_bf16(acc[(size_t)j]);
  }
}

std::vector<float> widen_bf16(const uint16_t* p, size_t n) {
  std::vector<float> v(n);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < (int64_t)n; ++i) v[(size_t)i] = bf16_value(p[i]);
  return v;
}

}  // namespace

extern "C" {

// The C5 decoder block (workloads.decoder_program) in bf16: x [b, s, m], g1 [m], wq / wk / wv
// [m, heads, hd], wo [heads, hd, m], g2 [m], w1 [m, f], w2 [f, m], all 16-bit words; out [b, s, m].
void accy_cpu_plan_decoder_bf16(const uint16_t* x16, const uint16_t* g1_16, const uint16_t* wq16,
                                const uint16_t* wk16, const uint16_t* wv16, const uint16_t* wo16,
                                const uint16_t* g2_16, const uint16_t* w1_16, const uint16_t* w2_16, int64_t batch,
                                int64_t seq, int64_t model, int64_t heads, int64_t hd, int64_t ffn, uint16_t* out) {
  const int64_t rows = batch * seq, hw = heads * hd;
  const float count = bf16_const((double)model), eps = bf16_const(1e-5), scale = bf16_const(1.0 / std::sqrt((double)hd));
  const float ga = bf16_const(0.044715), gc = bf16_const(0.7978845608028654), half = bf16_const(0.5),
              one = bf16_const(1.0);
  const float ninf = -std::numeric_limits<float>::infinity();
  const std::vector<float> x = widen_bf16(x16, (size_t)(rows * model)), g1 = widen_bf16(g1_16, (size_t)model),
                           g2 = widen_bf16(g2_16, (size_t)model), wq = widen_bf16(wq16, (size_t)(model * hw)),
                           wk = widen_bf16(wk16, (size_t)(model * hw)), wv = widen_bf16(wv16, (size_t)(model * hw)),
                           wo = widen_bf16(wo16, (size_t)(hw * model)), w1 = widen_bf16(w1_16, (size_t)(model * ffn)),
                           w2 = widen_bf16(w2_16, (size_t)(ffn * model));
  std::vector<float> h((size_t)(rows * model));
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) rms_row(&x[(size_t)(r * model)], g1.data(), model, count, eps, &h[(size_t)(r * model)]);
  std::vector<float> q((size_t)(rows * hw)), k((size_t)(rows * hw)), v((size_t)(rows * hw));
  dot_rows(h.data(), wq.data(), rows, model, hw, q.data());
  dot_rows(h.data(), wk.data(), rows, model, hw, k.data());
  dot_rows(h.data(), wv.data(), rows, model, hw, v.data());
  // Causal attention per (batch, head, query): q, k, v and o are [b, s, head, hd].
  std::vector<float> o((size_t)(rows * hw));
#pragma omp parallel for collapse(3) schedule(static)
  for (int64_t b = 0; b < batch; ++b)
    for (int64_t hh = 0; hh < heads; ++hh)
      for (int64_t qi = 0; qi < seq; ++qi) {
        std::vector<float> e((size_t)seq), acc((size_t)hd, 0.0f);
        const float* qrow = &q[(size_t)(((b * seq + qi) * heads + hh) * hd)];
        float mx = ninf;
        for (int64_t kj = 0; kj < seq; ++kj) {
          const float* krow = &k[(size_t)(((b * seq + kj) * heads + hh) * hd)];
          float dacc = 0.0f;
          for (int64_t d = 0; d < hd; ++d) {
            const float prod = qrow[d] * krow[d];
            dacc = dacc + prod;
          }
          float sc = round_bf16(round_bf16(dacc) * scale);
          if (kj > qi) sc = ninf;
          e[(size_t)kj] = sc;
          mx = fold_max(mx, sc);
        }
        float sum = 0.0f;
        for (int64_t kj = 0; kj < seq; ++kj) {
          const float t = round_bf16(expf(round_bf16(e[(size_t)kj] - mx)));
          e[(size_t)kj] = t;
          sum = sum + t;
        }
        const float den = round_bf16(sum);
        for (int64_t kj = 0; kj < seq; ++kj) {
          const float p = round_bf16(e[(size_t)kj] / den);
          const float* vrow = &v[(size_t)(((b * seq + kj) * heads + hh) * hd)];
          for (int64_t d = 0; d < hd; ++d) {
            const float prod = p * vrow[d];
            acc[(size_t)d] = acc[(size_t)d] + prod;
          }
        }
        float* orow = &o[(size_t)(((b * seq + qi) * heads + hh) * hd)];
        for (int64_t d = 0; d < hd; ++d) orow[d] = round_bf16(acc[(size_t)d]);
      }
  // Out-projection over (head, hd), then the residual x1 = x + y.
  std::vector<float> y((size_t)(rows * model)), x1((size_t)(rows * model));
  dot_rows(o.data(), wo.data(), rows, hw, model, y.data());
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < rows * model; ++i) x1[(size_t)i] = round_bf16(x[(size_t)i] + y[(size_t)i]);
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) rms_row(&x1[(size_t)(r * model)], g2.data(), model, count, eps, &h[(size_t)(r * model)]);
  // MLP-up, GELU (0.5 x (1 + tanh(c (x + a x^3))) in the traced order), MLP-down, residual.
  std::vector<float> f((size_t)(rows * ffn));
  dot_rows(h.data(), w1.data(), rows, model, ffn, f.data());
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < rows * ffn; ++i) {
    const float z = f[(size_t)i];
    const float cube = round_bf16(round_bf16(z * z) * z);
    const float inner = round_bf16(round_bf16(z + round_bf16(cube * ga)) * gc);
    f[(size_t)i] = round_bf16(round_bf16(z * half) * round_bf16(round_bf16(tanhf(inner)) + one));
  }
  dot_rows(f.data(), w2.data(), rows, ffn, model, y.data());
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < rows * model; ++i) out[i] = f32_to_bf16_trunc(x1[(size_t)i] + y[(size_t)i]);
}

}  // extern "C"
