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

// Compile-time loop: For<B, E>::run(f) calls f(Int<i>{}) for i = B .. E - 1, so that every register
// array index in the body is a constant.
template <int N> struct Int { static constexpr int value = N; };
template <int B, int E> struct For {
  template <class F> __device__ __forceinline__ static void run(F&& f) {
    if constexpr (B < E) {
      f(Int<B>{});
      For<B + 1, E>::run(f);
    }
  }
};

constexpr int HD = 128;  // head dimension of Q, K and V
constexpr int BK = 32;   // keys per block

// Issues this wave's share of the K tile of keys [k0, k0 + 32): 8 instructions of 4 rows each.
template <int WAVES, long KS>
__device__ __forceinline__ void load_k(const u16_t* __restrict__ kb, long k0, u16_t* lds, int wave, int lane) {
  constexpr int PER = 8 / WAVES;
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
  constexpr int PER = 8 / WAVES;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int gi = wave * PER + i;
    const int row = 4 * gi + (lane >> 4);
    const int p = lane & 15;
    const int u = (p >> 1) ^ (row & 7);
    gemm::dma16(vb + (k0 + row) * VS + 16 * u + 8 * (p & 1), (ACCY_LDS void*)(lds + gi * 512));
  }
}

// A operand of S^T for the block's 32 keys and head-dim step dd (16 elements).
__device__ __forceinline__ u32x4 k_frag(const u16_t* lds, int dd, int lane) {
  const int row = lane & 31;
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
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  if constexpr (DT == 0) {
    typedef __bf16 b16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(u32_t, __builtin_convertvector(f32x2{a, b}, b16x2));  // v_cvt_pk_bf16_f32 (RNE)
  } else {
    typedef _Float16 h16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(u32_t, __builtin_convertvector(f32x2{a, b}, h16x2));  // v_cvt_pk_f16_f32 (RNE)
  }
}

// max(a, b, c) in one v_max3_f32. (fmaxf on MFMA results costs a canonicalising v_max per value
// on top of the comparison; the scores here are never signalling NaNs.)
__device__ __forceinline__ float max3(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// acc + p.lo + p.hi for a packed pair of 16-bit probabilities, in one v_dot2_f32_{f16,bf16}: the row
// sum accumulates in f32 exactly the rounded values that the P.V product uses.
template <int DT>
__device__ __forceinline__ float add_pair(u32_t p, float acc) {
  if constexpr (DT == 0) {
    typedef __bf16 b16x2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b16x2, p), b16x2{(__bf16)1.0f, (__bf16)1.0f}, acc, false);
  } else {
    typedef _Float16 h16x2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h16x2, p), h16x2{(_Float16)1.0f, (_Float16)1.0f}, acc, false);
  }
}

// x[l] and x[l ^ 32] for every lane l. v_permlane32_swap exchanges the upper 32 lanes of its first
// operand with the lower 32 lanes of its second, so swapping x with a copy of itself leaves lane l
// holding x[l] in one register and x[l ^ 32] in the other. It is written as inline assembly with
// two distinct read-write registers (the compiler's builtin for it, used on two copies of one
// value, kept only one of the results here), with wait states around it for the VALU writes and
// reads of its operands.
__device__ __forceinline__ void with_partner(float x, float& r0, float& r1) {
  u32_t a = __builtin_bit_cast(u32_t, x), b = a;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
  r0 = __builtin_bit_cast(float, a);
  r1 = __builtin_bit_cast(float, b);
}
__device__ __forceinline__ float max_with_partner(float x) {
  float a, b;
  with_partner(x, a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float sum_with_partner(float x) {
  float a, b;
  with_partner(x, a, b);
  return a + b;
}

// Software pipeline per wave, iteration j (key block j of 32 keys):
//   A: the 16 MFMAs of S(j) = K(j) Q^T, with the softmax of block j - 1 slotted between them
//      (slots 0-3 row maxima, slot 4 the exchange with the partner lane and the rare rescale,
//      slots 5-15 exp2, partial sums and packing of P(j - 1));
//   B: the 16 MFMAs of O^T += V(j - 1)^T P(j - 1)^T.
// The softmax VALU work of one block thus issues under the MFMAs of the next. S alternates between
// two register sets by block parity (no copies); K and V stages are four deep, because V(j - 1) is
// still read while block j + 2 is loading.
template <class C>
struct Flash {
  static constexpr int WAVES = C::WAVES, BQ = 64 * WAVES, QT = 2, DS = HD / 16, DTN = HD / 32;
  static constexpr int PER = 2 * (8 / WAVES);  // load instructions per wave per key block
  static constexpr long NQB = C::SQ / BQ, NKB = C::SK / BK;
  static_assert(C::SQ % BQ == 0 && C::SK % BK == 0, "exact blocks only");

  const u16_t* __restrict__ kb;
  const u16_t* __restrict__ vb;
  u16_t* const* ks;
  u16_t* const* vs;
  u32x4 qf[QT][DS];
  f32x16 o[QT][DTN];
  f32x16 s[2][QT];  // scores of the blocks of even / odd index
  float m[QT], l[QT];
  long q0;
  int wave, lane;

  __device__ __forceinline__ long query(int qt) const { return q0 + 32 * (qt * WAVES + wave) + (lane & 31); }

  template <int ST>
  __device__ __forceinline__ void issue(long j) {
    load_k<WAVES, C::K_S>(kb, j * BK, ks[ST], wave, lane);
    load_v<WAVES, C::V_S>(vb, j * BK, vs[ST], wave, lane);
  }

  // Scores of keys above the query are -inf (blocks that cross the diagonal only).
  template <int PB>
  __device__ __forceinline__ void mask(long k0) {
    if (k0 + BK - 1 <= q0) return;
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const long qi = query(qt);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const long ki = k0 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (ki > qi) s[PB][qt][r] = -__builtin_inff();
      }
    }
  }

  // Softmax work of slot T (see above) on the scores in set PB; p receives P as MFMA B operands.
  template <int PB, int T>
  __device__ __forceinline__ void softmax_slot(float (&mx)[QT], float (&msub)[QT], float (&ls)[QT][4], u32x4 (&p)[QT][2]) {
    f32x16 (&sp)[QT] = s[PB];
    if constexpr (T < 4) {
      constexpr int qt = T >> 1, r0 = 8 * (T & 1);
#pragma unroll
      for (int r = 0; r < 8; r += 2) mx[qt] = max3(mx[qt], sp[qt][r0 + r], sp[qt][r0 + r + 1]);
    } else if constexpr (T == 4) {
      bool need[QT];
      float mn[QT];
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        mn[qt] = max_with_partner(mx[qt]) * C::SL;
        need[qt] = mn[qt] > m[qt] + 8.0f;
      }
      if (__any(need[0] || need[1])) {
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          const float alpha = need[qt] ? __builtin_amdgcn_exp2f(m[qt] - mn[qt]) : 1.0f;
          m[qt] = need[qt] ? mn[qt] : m[qt];
          l[qt] *= alpha;
#pragma unroll
          for (int dt = 0; dt < DTN; ++dt) o[qt][dt] *= alpha;
        }
      }
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) msub[qt] = m[qt] == -__builtin_inff() ? 0.0f : m[qt];
    } else {
      // 32 elements over slots 5..15; element e: qt = e / 16, r = e % 16.
      For<(T - 5) * 32 / 11, (T - 4) * 32 / 11>::run([&](auto ei) {
        constexpr int e = decltype(ei)::value, qt = e >> 4, r = e & 15;
        const float x = __builtin_amdgcn_exp2f(__builtin_fmaf(sp[qt][r], C::SL, -msub[qt]));
        sp[qt][r] = x;
        if constexpr (r & 1) {
          const u32_t pair = pack2<C::DT>(sp[qt][r - 1], x);
          p[qt][r >> 3][(r & 7) >> 1] = pair;
          ls[qt][(r >> 1) & 3] = add_pair<C::DT>(pair, ls[qt][(r >> 1) & 3]);
        }
      });
    }
  }

  // Phase A of block j (scores into set SB from stage ST) with the softmax of set PB when PREV.
  template <int ST, int SB, int PB, bool PREV>
  __device__ __forceinline__ void scores(long kprev0, u32x4 (&p)[QT][2]) {
    const u16_t* kl = ks[ST];
    float mx[QT], msub[QT], ls[QT][4];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      mx[qt] = -__builtin_inff();
      msub[qt] = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) ls[qt][i] = 0.0f;
      s[SB][qt] = f32x16{};
    }
    if constexpr (PREV && C::CAUSAL) mask<PB>(kprev0);
    u32x4 a = k_frag(kl, 0, lane), an = a;
    For<0, 16>::run([&](auto ti) {
      constexpr int t = decltype(ti)::value, dd = t >> 1, qt = t & 1;
      if constexpr (qt == 0 && t + 2 < 16) an = k_frag(kl, (t + 2) >> 1, lane);
      s[SB][qt] = gemm::mfma32x32x16<C::DT>(a, qf[qt][dd], s[SB][qt]);
      if constexpr (qt == 1) a = an;
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (PREV) softmax_slot<PB, t>(mx, msub, ls, p);
      __builtin_amdgcn_sched_barrier(0);
    });
    if constexpr (PREV) {
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) l[qt] += (ls[qt][0] + ls[qt][1]) + (ls[qt][2] + ls[qt][3]);
    }
  }

  // Phase B: O^T += V^T P^T for the block whose V tile is in stage VST.
  template <int VST>
  __device__ __forceinline__ void pv(const u32x4 (&p)[QT][2]) {
    const u16_t* vl = vs[VST];
    u32x4 a = v_frag(vl, 0, 0, lane), an = a;
    For<0, 16>::run([&](auto ti) {
      constexpr int t = decltype(ti)::value, dt = t >> 2, st = (t >> 1) & 1, qt = t & 1;
      if constexpr (qt == 0 && t + 2 < 16) an = v_frag(vl, (t + 2) >> 2, ((t + 2) >> 1) & 1, lane);
      o[qt][dt] = gemm::mfma32x32x16<C::DT>(a, p[qt][st], o[qt][dt]);
      if constexpr (qt == 1) a = an;
      __builtin_amdgcn_sched_barrier(0);
    });
  }

  // Iteration j >= 1 on stage ST = j % 4.
  template <int ST>
  __device__ __forceinline__ void iteration(long j, long nkb) {
    if (j + 1 < nkb) gemm::wait_vmcnt<PER>();
    else gemm::wait_vmcnt<0>();
    gemm::lds_reads_done_barrier();
    if (j + 2 < nkb) issue<(ST + 2) & 3>(j + 2);
    u32x4 p[QT][2];
    scores<ST, ST & 1, (ST + 1) & 1, true>((j - 1) * BK, p);
    pv<(ST + 3) & 3>(p);
  }

  // Softmax and P.V of the last block, in set PB and stage VST (no scores to overlap with).
  template <int PB, int VST>
  __device__ __forceinline__ void last(long k0) {
    if constexpr (C::CAUSAL) mask<PB>(k0);
    float mx[QT], msub[QT], ls[QT][4];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      mx[qt] = -__builtin_inff();
      msub[qt] = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) ls[qt][i] = 0.0f;
    }
    u32x4 p[QT][2];
    For<0, 16>::run([&](auto ti) { softmax_slot<PB, decltype(ti)::value>(mx, msub, ls, p); });
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) l[qt] += (ls[qt][0] + ls[qt][1]) + (ls[qt][2] + ls[qt][3]);
    pv<VST>(p);
  }
};

template <class C>
__device__ __forceinline__ void flash(const u16_t* __restrict__ Q, const u16_t* __restrict__ K,
                                      const u16_t* __restrict__ V, u16_t* __restrict__ O) {
  using F = Flash<C>;
  __shared__ __attribute__((aligned(1024))) u16_t k0s[BK * HD], k1s[BK * HD], k2s[BK * HD], k3s[BK * HD];
  __shared__ __attribute__((aligned(1024))) u16_t v0s[BK * HD], v1s[BK * HD], v2s[BK * HD], v3s[BK * HD];
  u16_t* const ks[4] = {k0s, k1s, k2s, k3s};
  u16_t* const vs[4] = {v0s, v1s, v2s, v3s};

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
  // Block 0: scores only.
  {
    if (nkb > 1) gemm::wait_vmcnt<F::PER>();
    else gemm::wait_vmcnt<0>();
    gemm::lds_reads_done_barrier();
    if (nkb > 2) f.template issue<2>(2);
    u32x4 unused[F::QT][2];
    f.template scores<0, 0, 1, false>(0, unused);
  }
  long j = 1;
  for (; j + 3 < nkb; j += 4) {
    f.template iteration<1>(j, nkb);
    f.template iteration<2>(j + 1, nkb);
    f.template iteration<3>(j + 2, nkb);
    f.template iteration<0>(j + 3, nkb);
  }
  if (j < nkb) f.template iteration<1>(j, nkb);
  if (j + 1 < nkb) f.template iteration<2>(j + 1, nkb);
  if (j + 2 < nkb) f.template iteration<3>(j + 2, nkb);
  // The last block (index nkb - 1) still needs its softmax and P.V.
  const long lb = nkb - 1;
  switch (lb & 3) {
    case 0: f.template last<0, 0>(lb * BK); break;
    case 1: f.template last<1, 1>(lb * BK); break;
    case 2: f.template last<0, 2>(lb * BK); break;
    default: f.template last<1, 3>(lb * BK); break;
  }

  const int h = f.lane >> 5;
#pragma unroll
  for (int qt = 0; qt < F::QT; ++qt) {
    const float inv = 1.0f / sum_with_partner(f.l[qt]);
    u16_t* __restrict__ orow = O + (b * C::SQ + f.query(qt)) * HD;
#pragma unroll
    for (int dt = 0; dt < F::DTN; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x16& acc = f.o[qt][dt];
        const u32_t lo = pack2<C::DT>(acc[4 * g] * inv, acc[4 * g + 1] * inv);
        const u32_t hi = pack2<C::DT>(acc[4 * g + 2] * inv, acc[4 * g + 3] * inv);
        *(u32x2*)(orow + dt * 32 + 8 * g + 4 * h) = u32x2{lo, hi};
      }
  }
}

}  // namespace attn
}  // namespace accy
