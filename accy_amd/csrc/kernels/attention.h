// Fused attention O[b, q, :] = softmax_k(scale * Q[b, q, :] . K[b, k, :] [masked k > q]) V[b, k, :] on
// gfx950 matrix cores, for 16-bit Q, K, V with a head dimension of 128 (both for Q.K and for V).
//
// One workgroup of WAVES wavefronts owns 64 * WAVES queries of one batch index and streams the keys
// in blocks of 64. Each wave owns two 32-query tiles (queries q0 + 32 w and q0 + 32 (WAVES + w), so
// that under a causal mask every wave of the group has almost the same work).
//
// Orientation: the scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16. In the
// 32 x 32 accumulator layout lane l then holds one query (column l % 32) and 16 keys (rows
// 8 g + 4 (l / 32) + j at register 4 g + j), so a row maximum or sum over the keys is a register
// fold plus one exchange with lane l ^ 32. The Q^T operand (B) is the same for every key block and
// stays in registers. The probabilities P^T are packed to 16 bits in registers and fed back as the B
// operand of O^T = V^T P^T: registers 8 s .. 8 s + 7 of a score tile are the B operand of 16-key
// step s when both operands number the keys of that step in the same permuted order (slot
// 8 h + 4 r + t holds key 16 s + 8 r + 4 h + t), which the V^T fragment read (ds_read_b64_tr_b16
// with rows 16 s + 8 r + 4 h + t) follows. No data moves between lanes for the softmax output.
//
// Softmax: f32 throughout, online over key blocks in the log2 domain: e = exp2(s * scale * log2 e -
// m) with v_exp_f32. The subtracted maximum m only moves when the running maximum exceeds it by more
// than 8 (a factor 256), so the accumulators are rescaled rarely; e <= 256 stays well inside the
// 16-bit range of the P operand. Row sums accumulate the f32 e; the result is O / sum.
//
// K and V tiles go straight from global memory to LDS (global_load_lds_dwordx4) three blocks deep,
// in three distinct LDS arrays per operand so that the compiler's wait analysis can tell the
// in-flight loads from the reads. Layouts (256-byte rows of 128 elements, conflict-free reads):
//  * K: 16-byte chunk c of key row r at chunk c ^ (r & 15); A-operand reads are ds_read_b128.
//  * V: 32-byte unit u of key row r at unit u ^ (r & 7); A-operand reads are ds_read_b64_tr_b16.
//
// The configuration struct C supplies: DT (0 bf16, 1 f16), WAVES, SQ, SK, NB (batch count), the
// element strides Q_S, K_S, V_S of one query / key row (the head dimension has stride 1), the batch
// offset functions q_off(b), k_off(b), v_off(b), CAUSAL and SL (the score scale times log2 e, > 0).
// O is written row-major as [b][q][128].
#pragma once

namespace accy {
namespace attn {

using gemm::f32x16;
using gemm::i16x4;
using gemm::u32x4;
typedef u32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int HD = 128;  // head dimension of Q, K and V
constexpr int BK = 64;   // keys per block

// Issues this wave's share of the K tile of keys [k0, k0 + 64): 16 instructions of 4 rows each.
template <int WAVES, long KS>
__device__ __forceinline__ void load_k(const u16_t* __restrict__ kb, long k0, u16_t* lds, int wave, int lane) {
  constexpr int PER = 16 / WAVES;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int gi = wave * PER + i;
    const int row = 4 * gi + (lane >> 4);
    const int c = (lane & 15) ^ (row & 15);
    gemm::dma16(kb + (k0 + row) * KS + 8 * c, (ACCY_LDS void*)(lds + gi * 512));
  }
}

template <int WAVES, long VS>
__device__ __forceinline__ void load_v(const u16_t* __restrict__ vb, long k0, u16_t* lds, int wave, int lane) {
  constexpr int PER = 16 / WAVES;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int gi = wave * PER + i;
    const int row = 4 * gi + (lane >> 4);
    const int p = lane & 15;
    const int u = (p >> 1) ^ (row & 7);
    gemm::dma16(vb + (k0 + row) * VS + 16 * u + 8 * (p & 1), (ACCY_LDS void*)(lds + gi * 512));
  }
}

// A operand of S^T for key tile kt (32 keys) and head-dim step dd (16 elements).
__device__ __forceinline__ u32x4 k_frag(const u16_t* lds, int kt, int dd, int lane) {
  const int row = kt * 32 + (lane & 31);
  const int c = 2 * dd + (lane >> 5);
  return *(const u32x4*)(lds + row * HD + ((c ^ (row & 15)) << 3));
}

// A operand of O^T = V^T P^T for head-dim tile dt (32) and 16-key step s, keys in the permuted order.
__device__ __forceinline__ u32x4 v_frag(const u16_t* lds, int dt, int s, int lane) {
  const int g = lane >> 4, i = lane & 15;
  const int n0 = dt * 32 + ((g & 1) << 4);
  u32x4 out;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int k = 16 * s + 8 * r + 4 * (g >> 1) + (i >> 2);
    const int unit = (n0 >> 4) ^ (k & 7);
    const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((ACCY_LDS i16x4*)(lds + k * HD + unit * 16 + 4 * (i & 3)));
    out[2 * r] = (u32_t)(u16_t)v[0] | ((u32_t)(u16_t)v[1] << 16);
    out[2 * r + 1] = (u32_t)(u16_t)v[2] | ((u32_t)(u16_t)v[3] << 16);
  }
  return out;
}

template <int DT>
__device__ __forceinline__ u32_t pack2(float a, float b) {
  if constexpr (DT == 0) return (u32_t)f32_to_bf16(a) | ((u32_t)f32_to_bf16(b) << 16);
  else return (u32_t)f32_to_f16(a) | ((u32_t)f32_to_f16(b) << 16);
}

template <class C>
struct Flash {
  static constexpr int WAVES = C::WAVES, BQ = 64 * WAVES, QT = 2, KT = BK / 32, DS = HD / 16, DTN = HD / 32;
  static constexpr int PER = 2 * (16 / WAVES);  // load instructions per wave per key block
  static constexpr long NQB = C::SQ / BQ, NKB = C::SK / BK;
  static_assert(C::SQ % BQ == 0 && C::SK % BK == 0, "exact blocks only");

  const u16_t* __restrict__ kb;
  const u16_t* __restrict__ vb;
  u16_t* const* ks;
  u16_t* const* vs;
  u32x4 qf[QT][DS];
  f32x16 o[QT][DTN];
  float m[QT], l[QT];
  long q0;
  int wave, lane;

  __device__ __forceinline__ long query(int qt) const { return q0 + 32 * (qt * WAVES + wave) + (lane & 31); }

  template <int ST>
  __device__ __forceinline__ void issue(long j) {
    load_k<WAVES, C::K_S>(kb, j * BK, ks[ST], wave, lane);
    load_v<WAVES, C::V_S>(vb, j * BK, vs[ST], wave, lane);
  }

  // Key block j from stage ST; block j + 2 goes to stage NX once every wave is past block j - 1.
  template <int ST, int NX>
  __device__ __forceinline__ void step(long j, long nkb) {
    if (j + 1 < nkb) gemm::wait_vmcnt<PER>();
    else gemm::wait_vmcnt<0>();
    gemm::lds_reads_done_barrier();
    if (j + 2 < nkb) issue<NX>(j + 2);
    const u16_t* kl = ks[ST];
    const u16_t* vl = vs[ST];
    const long k0 = j * BK;

    f32x16 s[QT][KT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) s[qt][kt] = f32x16{};
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int dd = 0; dd < DS; ++dd) {
        const u32x4 a = k_frag(kl, kt, dd, lane);
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) s[qt][kt] = gemm::mfma32x32x16<C::DT>(a, qf[qt][dd], s[qt][kt]);
      }

    if constexpr (C::CAUSAL) {
      if (k0 + BK - 1 > q0) {
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          const long qi = query(qt);
#pragma unroll
          for (int kt = 0; kt < KT; ++kt)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const long ki = k0 + 32 * kt + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
              if (ki > qi) s[qt][kt][r] = -__builtin_inff();
            }
        }
      }
    }

    u32x4 p[QT][BK / 16];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      float mx = s[qt][0][0];
#pragma unroll
      for (int kt = 0; kt < KT; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[qt][kt][r]);
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float mn = mx * C::SL;
      const bool need = mn > m[qt] + 8.0f;
      if (__any(need)) {
        const float alpha = need ? __builtin_amdgcn_exp2f(m[qt] - mn) : 1.0f;
        m[qt] = need ? mn : m[qt];
        l[qt] *= alpha;
#pragma unroll
        for (int dt = 0; dt < DTN; ++dt) o[qt][dt] *= alpha;
      }
      const float msub = m[qt] == -__builtin_inff() ? 0.0f : m[qt];
      float sum = 0.0f;
#pragma unroll
      for (int kt = 0; kt < KT; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(s[qt][kt][r], C::SL, -msub));
          s[qt][kt][r] = e;
          sum += e;
        }
      l[qt] += sum;
#pragma unroll
      for (int st = 0; st < BK / 16; ++st) {
        const int kt = st >> 1, b = 8 * (st & 1);
#pragma unroll
        for (int w = 0; w < 4; ++w) p[qt][st][w] = pack2<C::DT>(s[qt][kt][b + 2 * w], s[qt][kt][b + 2 * w + 1]);
      }
    }

#pragma unroll
    for (int dt = 0; dt < DTN; ++dt)
#pragma unroll
      for (int st = 0; st < BK / 16; ++st) {
        const u32x4 a = v_frag(vl, dt, st, lane);
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) o[qt][dt] = gemm::mfma32x32x16<C::DT>(a, p[qt][st], o[qt][dt]);
      }
  }
};

template <class C>
__device__ __forceinline__ void flash(const u16_t* __restrict__ Q, const u16_t* __restrict__ K,
                                      const u16_t* __restrict__ V, u16_t* __restrict__ O) {
  using F = Flash<C>;
  __shared__ __attribute__((aligned(1024))) u16_t k0s[BK * HD], k1s[BK * HD], k2s[BK * HD];
  __shared__ __attribute__((aligned(1024))) u16_t v0s[BK * HD], v1s[BK * HD], v2s[BK * HD];
  u16_t* const ks[3] = {k0s, k1s, k2s};
  u16_t* const vs[3] = {v0s, v1s, v2s};

  // Tiles of one batch index go to one XCD (they share K and V in its L2); under a causal mask the
  // query blocks with the most keys start first.
  const long total = (long)gridDim.x;
  long t = (long)blockIdx.x;
  if (total % 8 == 0) t = (t % 8) * (total / 8) + t / 8;
  const long b = t / F::NQB;
  long qb = t % F::NQB;
  if constexpr (C::CAUSAL) qb = F::NQB - 1 - qb;

  F f;
  f.ks = ks;
  f.vs = vs;
  f.wave = (int)(threadIdx.x >> 6);
  f.lane = (int)(threadIdx.x & 63);
  f.q0 = qb * F::BQ;
  f.kb = K + C::k_off(b);
  f.vb = V + C::v_off(b);
  const u16_t* __restrict__ qb_ptr = Q + C::q_off(b);
#pragma unroll
  for (int qt = 0; qt < F::QT; ++qt)
#pragma unroll
    for (int dd = 0; dd < F::DS; ++dd)
      f.qf[qt][dd] = *(const u32x4*)(qb_ptr + f.query(qt) * C::Q_S + 16 * dd + 8 * (f.lane >> 5));
#pragma unroll
  for (int qt = 0; qt < F::QT; ++qt) {
    f.m[qt] = -__builtin_inff();
    f.l[qt] = 0.0f;
#pragma unroll
    for (int dt = 0; dt < F::DTN; ++dt) f.o[qt][dt] = f32x16{};
  }

  long nkb = F::NKB;
  if constexpr (C::CAUSAL) {
    const long last = (f.q0 + F::BQ - 1) / BK + 1;
    nkb = last < nkb ? last : nkb;
  }
  f.template issue<0>(0);
  if (nkb > 1) f.template issue<1>(1);
  for (long j = 0; j < nkb; j += 3) {
    f.template step<0, 2>(j, nkb);
    if (j + 1 < nkb) f.template step<1, 0>(j + 1, nkb);
    if (j + 2 < nkb) f.template step<2, 1>(j + 2, nkb);
  }

  const int h = f.lane >> 5;
#pragma unroll
  for (int qt = 0; qt < F::QT; ++qt) {
    const float lt = f.l[qt] + __shfl_xor(f.l[qt], 32);
    const float inv = 1.0f / lt;
    u16_t* __restrict__ orow = O + (b * C::SQ + f.query(qt)) * HD;
#pragma unroll
    for (int dt = 0; dt < F::DTN; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x16& acc = f.o[qt][dt];
        u32_t lo = pack2<C::DT>(acc[4 * g] * inv, acc[4 * g + 1] * inv);
        u32_t hi = pack2<C::DT>(acc[4 * g + 2] * inv, acc[4 * g + 3] * inv);
        *(u32x2*)(orow + dt * 32 + 8 * g + 4 * h) = u32x2{lo, hi};
      }
  }
}

}  // namespace attn
}  // namespace accy
