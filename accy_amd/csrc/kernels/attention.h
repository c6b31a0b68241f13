// Fused attention O[b, q, :] = softmax_k(scale * Q[b, q, :] . K[b, k, :] [masked k > q]) V[b, k, :] on
// gfx950 matrix cores, for 16-bit Q, K, V with a head dimension HD of 64 or 128 (both for Q.K and for
// V), and (flash_f32, at the end) for f32 Q, K, V with a head dimension of 64.
//
// A workgroup of 2 * WAVES wavefronts owns 64 * WAVES queries of one batch index and streams the
// keys in blocks of 32. Each group of 64 queries (two 32-query tiles, q0 + 32 w and
// q0 + 32 (WAVES + w), so that under a causal mask every group has almost the same work) is served
// by a scorer wave (S and softmax) and an accumulator wave (P.V and the output); see the work split
// below.
//
// Orientation: the scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16. In the
// 32 x 32 accumulator layout lane l then holds one query (column l % 32) and 16 keys (rows
// 8 g + 4 (l / 32) + j at register 4 g + j), so a row maximum or sum over the keys is a register
// fold plus one exchange with lane l ^ 32. The Q^T operand (B) is the same for every key block and
// stays in the scorer's registers. The probabilities P^T are packed to 16 bits and serve as the B
// operand of O^T = V^T P^T: registers 8 s .. 8 s + 7 of a score tile are the B operand of 16-key
// step s when both operands number the keys of that step in the same permuted order (slot
// 8 h + 4 r + t holds key 16 s + 8 r + 4 h + t), which the V^T fragment read (ds_read_b64_tr_b16
// with rows 16 s + 8 r + 4 h + t) follows. P crosses from scorer to accumulator through LDS in
// exactly this register layout (lane-linear 16-byte stores and loads).
//
// Softmax: f32 throughout, online over key blocks in the log2 domain: e = exp2(s * scale * log2 e -
// m) with v_exp_f32. The subtracted maximum m only moves when the running maximum exceeds it by more
// than 8 (a factor 256), so the accumulators are rescaled rarely; e <= 256 stays well inside the
// 16-bit range of the P operand. Row sums accumulate the f32 e; the result is O / sum.
//
// K and V tiles go straight from global memory to LDS (global_load_lds_dwordx4), four stages per
// operand in distinct LDS arrays so that the compiler's wait analysis can tell the in-flight loads
// from the reads. Layouts (256-byte rows of 128 elements, conflict-free reads):
//  * K: 16-byte chunk c of key row r at chunk c ^ (r & 15); A-operand reads are ds_read_b128.
//  * V: 32-byte unit u of key row r at unit u ^ gemm::tr_swizzle(r); A-operand reads are
//    ds_read_b64_tr_b16 (each 32-lane half covers 256 distinct bytes, the 64-bank LDS's width).
//
// The configuration struct C supplies: DT (0 bf16, 1 f16), HD, WAVES, SQ, SK, NB (batch count), the
// element strides Q_S, K_S, V_S of one query / key row (the head dimension has stride 1), the batch
// offset functions q_off(b), k_off(b), v_off(b), CAUSAL and SL (the score scale times log2 e, > 0).
// O is written row-major as [b][q][128]. The kernel is launched with 128 * WAVES threads.
#pragma once

namespace accy {
namespace attn {

using gemm::f32x16;
using gemm::i16x4;
using gemm::u32x4;
typedef u32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

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

constexpr int BK = 32;   // keys per block

// LDS layouts of a K / V tile (32 key rows of HD 16-bit elements), conflict-free on the 64-bank LDS:
//  * K: the 16-byte chunk c of key row r sits at chunk c ^ k_swizzle(r). A fragment's 16-lane group
//    reads one chunk of 16 consecutive rows: with 256-byte rows (HD 128) the XOR with r & 15 spreads
//    them over the 16 positions; with 128-byte rows (HD 64) two rows share 256 bytes, and the XOR
//    with (r / 2) & 7 spreads the 8 row pairs.
//  * V: the 32-byte unit u of key row r sits at unit u ^ v_swizzle(r). A 32-lane half of a transposed
//    read covers units (u, u ^ 1) of four consecutive rows: 256-byte rows use gemm::tr_swizzle
//    (2 (r & 3)); 128-byte rows (4 units, two rows per 256 bytes) XOR with 2 ((r / 2) & 1).
template <int HD> __device__ __forceinline__ int k_swizzle(int r) { return HD == 128 ? (r & 15) : ((r >> 1) & 7); }
template <int HD> __device__ __forceinline__ int v_swizzle(int r) { return HD == 128 ? gemm::tr_swizzle(r) : 2 * ((r >> 1) & 1); }

// Issues this wave's share of the K tile of keys [k0, k0 + 32): HD / 16 instructions of 1 KiB.
template <int WAVES, long KS, int HD>
__device__ __forceinline__ void load_k(const u16_t* __restrict__ kb, long k0, u16_t* lds, int wave, int lane) {
  constexpr int PER = HD / 16 / WAVES, LPR = HD / 8, RPI = 64 / LPR;  // lanes per row, rows per instruction
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int gi = wave * PER + i;
    const int row = RPI * gi + lane / LPR;
    const int c = (lane % LPR) ^ k_swizzle<HD>(row);
    gemm::dma16(kb + (k0 + row) * KS + 8 * c, (ACCY_LDS void*)(lds + gi * 512));
  }
}

template <int WAVES, long VS, int HD>
__device__ __forceinline__ void load_v(const u16_t* __restrict__ vb, long k0, u16_t* lds, int wave, int lane) {
  constexpr int PER = HD / 16 / WAVES, LPR = HD / 8, RPI = 64 / LPR;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int gi = wave * PER + i;
    const int row = RPI * gi + lane / LPR;
    const int p = lane % LPR;
    const int u = (p >> 1) ^ v_swizzle<HD>(row);
    gemm::dma16(vb + (k0 + row) * VS + 16 * u + 8 * (p & 1), (ACCY_LDS void*)(lds + gi * 512));
  }
}

// A operand of S^T for the block's 32 keys and head-dim step dd (16 elements).
template <int HD>
__device__ __forceinline__ u32x4 k_frag(const u16_t* lds, int dd, int lane) {
  const int row = lane & 31;
  const int c = 2 * dd + (lane >> 5);
  return *(const u32x4*)(lds + row * HD + ((c ^ k_swizzle<HD>(row)) << 3));
}

// A operand of O^T = V^T P^T for head-dim tile dt (32) and 16-key step s, keys in the permuted order.
template <int HD>
__device__ __forceinline__ u32x4 v_frag(const u16_t* lds, int dt, int s, int lane) {
  const int g = lane >> 4, i = lane & 15;
  const int n0 = dt * 32 + ((g & 1) << 4);
  u32x4 out;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int k = 16 * s + 8 * r + 4 * (g >> 1) + (i >> 2);
    const int unit = (n0 >> 4) ^ v_swizzle<HD>(k);
    const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((ACCY_LDS i16x4*)(lds + k * HD + unit * 16 + 4 * (i & 3)));
    out[2 * r] = (u32_t)(u16_t)v[0] | ((u32_t)(u16_t)v[1] << 16);
    out[2 * r + 1] = (u32_t)(u16_t)v[2] | ((u32_t)(u16_t)v[3] << 16);
  }
  return out;
}

// Probabilities P for the P.V product: an internal operand of the fused kernel (no traced value), packed
// with the hardware conversion, nearest even for both types.
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

// The output O, a traced result: f16 rounds to nearest even (@floatCast), bf16 keeps the high half of
// each f32 (Bf16.fromF32, deps/lib/compiler/gpu/abi/src/dtype.zig:6-9), as every bf16 result does.
template <int DT>
__device__ __forceinline__ u32_t pack2_out(float a, float b) {
  if constexpr (DT == 0) return pack_bf16x2(a, b);
  else return pack2<DT>(a, b);
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

// Work split. Each group of 64 queries is served by two waves, which the hardware places on one
// SIMD (waves w and w + WAVES of a workgroup of 2 * WAVES waves):
//  * the scorer computes S = K Q^T and the softmax and writes P (16-bit, already in the MFMA
//    B-operand layout) and the rescale factors to LDS;
//  * the accumulator reads them back and runs O^T += V^T P^T, then normalises and stores O.
// Each wave then fits in half the register file (the scorer holds Q^T and two score sets, the
// accumulator O), so the two share a SIMD, and the scorer's softmax VALU work issues while the
// accumulator's MFMAs run. Step t of the workgroup (one barrier each, nkb + 2 steps):
//  * scorer: S(t) for t < nkb, with the softmax of block t - 1 slotted between its 16 MFMAs (slots
//    0-3 row maxima, slot 4 the exchange with the partner lane and the rare rescale, slots 5-15
//    exp2, partial sums and packing); P(t - 1) and the factors go to buffer (t - 1) % 2;
//  * accumulator: for t >= 2, block t - 2 from buffer t % 2 and V stage (t - 2) % 4.
// K tiles are loaded by the scorers two steps ahead (K(t + 2) at step t), V tiles by the
// accumulators two steps before use (V(t) at step t); both have four LDS stages. A P buffer written
// at step t is read at step t + 1 and rewritten at step t + 2, after the barrier that follows the
// reads.
template <class C>
struct Lds {
  static constexpr int WAVES = C::WAVES;
  u16_t* const* ks;  // K stages [4][BK * HD]
  u16_t* const* vs;  // V stages [4][BK * HD]
  u32x4* pb;         // P: [2][WAVES][QT * 2][64] u32x4
  float* ab;         // rescale factors: [2][WAVES][64][QT]
  float* lb;         // row sums for the epilogue: [WAVES][64][QT]
};

template <class C>
struct Scorer {
  static constexpr int HD = C::HD, WAVES = C::WAVES, QT = 2, DS = HD / 16;
  static constexpr int NS = QT * DS;            // score MFMAs per key block (16 for HD 128, 8 for HD 64)
  static constexpr int PER = HD / 16 / WAVES;  // K load instructions per wave per key block
  static constexpr long NQB = C::SQ / (64 * WAVES), NKB = C::SK / BK;

  Lds<C> sh;
  const u16_t* __restrict__ kb;
  u32x4 qf[QT][DS];
  f32x16 s[2][QT];  // scores of the blocks of even / odd index
  float m[QT], l[QT];
  long q0;
  int wave, lane;

  __device__ __forceinline__ long query(int qt) const { return q0 + 32 * (qt * WAVES + wave) + (lane & 31); }

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

  // Softmax work of slot T on the scores in set PB; p receives P as MFMA B operands, alpha the
  // factor by which the accumulated O is to be scaled before P.V of this block (1 if unchanged).
  template <int PB, int T>
  __device__ __forceinline__ void softmax_slot(float (&mx)[QT], float (&msub)[QT], float (&ls)[QT][4], u32x4 (&p)[QT][2],
                                               float (&alpha)[QT]) {
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
        alpha[qt] = 1.0f;
      }
      if (__any(need[0] || need[1])) {
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          alpha[qt] = need[qt] ? __builtin_amdgcn_exp2f(m[qt] - mn[qt]) : 1.0f;
          m[qt] = need[qt] ? mn[qt] : m[qt];
          l[qt] *= alpha[qt];
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

  // Scores of one block into set SB from K stage ST, with the softmax of set PB when PREV.
  template <int ST, int SB, int PB, bool PREV>
  __device__ __forceinline__ void scores(long kprev0, u32x4 (&p)[QT][2], float (&alpha)[QT]) {
    const u16_t* kl = sh.ks[ST];
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
    u32x4 a = k_frag<HD>(kl, 0, lane), an = a;
    For<0, NS>::run([&](auto ti) {
      constexpr int t = decltype(ti)::value, dd = t >> 1, qt = t & 1;
      if constexpr (qt == 0 && t + 2 < NS) an = k_frag<HD>(kl, (t + 2) >> 1, lane);
      s[SB][qt] = gemm::mfma32x32x16<C::DT>(a, qf[qt][dd], s[SB][qt]);
      if constexpr (qt == 1) a = an;
      __builtin_amdgcn_sched_barrier(0);
      // the 16 softmax slots of the previous block, spread over this block's NS MFMAs
      if constexpr (PREV)
        For<t * 16 / NS, (t + 1) * 16 / NS>::run([&](auto si) { softmax_slot<PB, decltype(si)::value>(mx, msub, ls, p, alpha); });
      __builtin_amdgcn_sched_barrier(0);
    });
    if constexpr (PREV) {
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) l[qt] += (ls[qt][0] + ls[qt][1]) + (ls[qt][2] + ls[qt][3]);
    }
  }

  // Softmax of the last block (set PB), with no scores to overlap with.
  template <int PB>
  __device__ __forceinline__ void softmax_only(long k0, u32x4 (&p)[QT][2], float (&alpha)[QT]) {
    if constexpr (C::CAUSAL) mask<PB>(k0);
    float mx[QT], msub[QT], ls[QT][4];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      mx[qt] = -__builtin_inff();
      msub[qt] = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) ls[qt][i] = 0.0f;
    }
    For<0, 16>::run([&](auto ti) { softmax_slot<PB, decltype(ti)::value>(mx, msub, ls, p, alpha); });
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) l[qt] += (ls[qt][0] + ls[qt][1]) + (ls[qt][2] + ls[qt][3]);
  }

  // P and the rescale factors of one block into buffer PBUF (lane-linear, conflict-free).
  template <int PBUF>
  __device__ __forceinline__ void publish(const u32x4 (&p)[QT][2], const float (&alpha)[QT]) {
    u32x4* pw = sh.pb + (PBUF * WAVES + wave) * (QT * 2 * 64) + lane;
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
#pragma unroll
      for (int st = 0; st < 2; ++st) pw[(qt * 2 + st) * 64] = p[qt][st];
    float* aw = sh.ab + ((PBUF * WAVES + wave) * 64 + lane) * QT;
    *(f32x2*)aw = f32x2{alpha[0], alpha[1]};
  }

  // Step t (1 <= t < nkb) on K stage ST = t % 4.
  template <int ST>
  __device__ __forceinline__ void step(long t, long nkb) {
    if (t + 1 < nkb) gemm::wait_vmcnt<PER>();
    else gemm::wait_vmcnt<0>();
    gemm::lds_reads_done_barrier();
    if (t + 2 < nkb) load_k<WAVES, C::K_S, HD>(kb, (t + 2) * BK, sh.ks[(ST + 2) & 3], wave, lane);
    u32x4 p[QT][2];
    float alpha[QT];
    scores<ST, ST & 1, (ST + 1) & 1, true>((t - 1) * BK, p, alpha);
    publish<(ST + 1) & 1>(p, alpha);
  }

  // Step nkb: the softmax of the last block (index nkb - 1, score set and buffer PB).
  template <int PB>
  __device__ __forceinline__ void last_step(long nkb) {
    gemm::lds_reads_done_barrier();
    u32x4 p[QT][2];
    float alpha[QT];
    softmax_only<PB>((nkb - 1) * BK, p, alpha);
    publish<PB>(p, alpha);
  }

  __device__ __forceinline__ void run(const u16_t* __restrict__ qp, long nkb) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
#pragma unroll
      for (int dd = 0; dd < DS; ++dd) qf[qt][dd] = *(const u32x4*)(qp + query(qt) * C::Q_S + 16 * dd + 8 * (lane >> 5));
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      m[qt] = -__builtin_inff();
      l[qt] = 0.0f;
    }
    load_k<WAVES, C::K_S, HD>(kb, 0, sh.ks[0], wave, lane);
    if (nkb > 1) load_k<WAVES, C::K_S, HD>(kb, BK, sh.ks[1], wave, lane);
    // Step 0: scores of block 0 only.
    if (nkb > 1) gemm::wait_vmcnt<PER>();
    else gemm::wait_vmcnt<0>();
    gemm::lds_reads_done_barrier();
    if (nkb > 2) load_k<WAVES, C::K_S, HD>(kb, 2 * BK, sh.ks[2], wave, lane);
    {
      u32x4 unused_p[QT][2];
      float unused_a[QT];
      scores<0, 0, 1, false>(0, unused_p, unused_a);
    }
    long t = 1;
    for (; t + 3 < nkb; t += 4) {
      step<1>(t, nkb);
      step<2>(t + 1, nkb);
      step<3>(t + 2, nkb);
      step<0>(t + 3, nkb);
    }
    if (t < nkb) step<1>(t, nkb);
    if (t + 1 < nkb) step<2>(t + 1, nkb);
    if (t + 2 < nkb) step<3>(t + 2, nkb);
    if ((nkb - 1) & 1) last_step<1>(nkb);
    else last_step<0>(nkb);
    // Row sums (both lanes of a query) for the accumulator's epilogue, then step nkb + 1.
    float* lw = sh.lb + (wave * 64 + lane) * QT;
    *(f32x2*)lw = f32x2{sum_with_partner(l[0]), sum_with_partner(l[1])};
    gemm::lds_reads_done_barrier();
  }
};

template <class C>
struct Accumulator {
  static constexpr int HD = C::HD, WAVES = C::WAVES, QT = 2, DTN = HD / 32;
  static constexpr int NA = DTN * 2 * QT;      // P.V MFMAs per key block (16 for HD 128, 8 for HD 64)
  static constexpr int PER = HD / 16 / WAVES;  // V load instructions per wave per key block

  Lds<C> sh;
  const u16_t* __restrict__ vb;
  f32x16 o[QT][DTN];
  long q0;
  int wave, lane;

  __device__ __forceinline__ long query(int qt) const { return q0 + 32 * (qt * WAVES + wave) + (lane & 31); }

  // O^T = alpha O^T + V^T P^T for the block in P buffer PBUF and V stage VST.
  template <int PBUF, int VST>
  __device__ __forceinline__ void consume() {
    const u32x4* pr = sh.pb + (PBUF * WAVES + wave) * (QT * 2 * 64) + lane;
    const f32x2 al = *(const f32x2*)(sh.ab + ((PBUF * WAVES + wave) * 64 + lane) * QT);
    u32x4 p[QT][2];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
#pragma unroll
      for (int st = 0; st < 2; ++st) p[qt][st] = pr[(qt * 2 + st) * 64];
    const u16_t* vl = sh.vs[VST];
    u32x4 vf[DTN][2];
#pragma unroll
    for (int dt = 0; dt < DTN; ++dt)
#pragma unroll
      for (int st = 0; st < 2; ++st) vf[dt][st] = v_frag<HD>(vl, dt, st, lane);
    if (__any(al.x != 1.0f || al.y != 1.0f)) {
#pragma unroll
      for (int dt = 0; dt < DTN; ++dt) {
        o[0][dt] *= al.x;
        o[1][dt] *= al.y;
      }
    }
    For<0, NA>::run([&](auto ti) {
      constexpr int t = decltype(ti)::value, dt = t >> 2, st = (t >> 1) & 1, qt = t & 1;
      o[qt][dt] = gemm::mfma32x32x16<C::DT>(vf[dt][st], p[qt][st], o[qt][dt]);
    });
  }

  // Step t >= 2 on stage ST = t % 4: V(t) is issued, block t - 2 consumed.
  template <int ST>
  __device__ __forceinline__ void step(long t, long nkb) {
    if (t - 1 < nkb) gemm::wait_vmcnt<PER>();
    else gemm::wait_vmcnt<0>();
    gemm::lds_reads_done_barrier();
    if (t < nkb) load_v<WAVES, C::V_S, HD>(vb, t * BK, sh.vs[ST], wave, lane);
    consume<ST & 1, (ST + 2) & 3>();
  }

  __device__ __forceinline__ void run(u16_t* __restrict__ out, long b, long nkb) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
#pragma unroll
      for (int dt = 0; dt < DTN; ++dt) o[qt][dt] = f32x16{};
    // Steps 0 and 1: V(0) and V(1) are issued.
    gemm::lds_reads_done_barrier();
    load_v<WAVES, C::V_S, HD>(vb, 0, sh.vs[0], wave, lane);
    gemm::lds_reads_done_barrier();
    if (nkb > 1) load_v<WAVES, C::V_S, HD>(vb, BK, sh.vs[1], wave, lane);
    // Steps 2 .. nkb + 1.
    long t = 2;
    for (; t + 3 <= nkb + 1; t += 4) {
      step<2>(t, nkb);
      step<3>(t + 1, nkb);
      step<0>(t + 2, nkb);
      step<1>(t + 3, nkb);
    }
    if (t <= nkb + 1) step<2>(t, nkb);
    if (t + 1 <= nkb + 1) step<3>(t + 1, nkb);
    if (t + 2 <= nkb + 1) step<0>(t + 2, nkb);

    const f32x2 lsum = *(const f32x2*)(sh.lb + (wave * 64 + lane) * QT);
    const float inv[QT] = {1.0f / lsum.x, 1.0f / lsum.y};
    const int h = lane >> 5;
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      u16_t* __restrict__ orow = out + (b * C::SQ + query(qt)) * HD;
#pragma unroll
      for (int dt = 0; dt < DTN; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x16& acc = o[qt][dt];
          const u32_t lo = pack2_out<C::DT>(acc[4 * g] * inv[qt], acc[4 * g + 1] * inv[qt]);
          const u32_t hi = pack2_out<C::DT>(acc[4 * g + 2] * inv[qt], acc[4 * g + 3] * inv[qt]);
          *(u32x2*)(orow + dt * 32 + 8 * g + 4 * h) = u32x2{lo, hi};
        }
    }
  }
};

// Query blocks per workgroup: under a causal mask with an even number of query blocks, a workgroup
// takes block NQB - 1 - p and then block p, so that every workgroup streams the same number of key
// blocks (the heavy blocks start first); the grid is NB * NQB / blocks_per_group workgroups.
template <class C>
constexpr long blocks_per_group() {
  constexpr long NQB = C::SQ / (64 * C::WAVES);
  return C::CAUSAL && NQB % 2 == 0 ? 2 : 1;
}

// One query block (queries qb * 64 * WAVES ...) of batch index b, by the workgroup's scorer and
// accumulator waves. Both roles meet nkb + 2 barriers, so blocks can follow each other.
template <class C>
__device__ __forceinline__ void flash_block(const Lds<C>& sh, const u16_t* __restrict__ Q, const u16_t* __restrict__ K,
                                            const u16_t* __restrict__ V, u16_t* __restrict__ O, long b, long qb) {
  constexpr int WAVES = C::WAVES;
  constexpr long BQ = 64 * WAVES, NKB = C::SK / BK;
  const long q0 = qb * BQ;
  long nkb = NKB;
  if constexpr (C::CAUSAL) {
    const long last = (q0 + BQ - 1) / BK + 1;
    nkb = last < nkb ? last : nkb;
  }
  // The wave index is uniform across the wave; readfirstlane lets the compiler branch on the role.
  const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int lane = (int)(threadIdx.x & 63);
  if (w < WAVES) {
    Scorer<C> f;
    f.sh = sh;
    f.kb = K + C::k_off(b);
    f.q0 = q0;
    f.wave = w;
    f.lane = lane;
    f.run(Q + C::q_off(b), nkb);
  } else {
    Accumulator<C> f;
    f.sh = sh;
    f.vb = V + C::v_off(b);
    f.q0 = q0;
    f.wave = w - WAVES;
    f.lane = lane;
    f.run(O, b, nkb);
  }
}

// Workgroup of 2 * C::WAVES waves (128 * C::WAVES threads) over blocks_per_group<C>() query blocks
// of 64 * C::WAVES queries of one batch index.
template <class C>
__device__ __forceinline__ void flash(const u16_t* __restrict__ Q, const u16_t* __restrict__ K,
                                      const u16_t* __restrict__ V, u16_t* __restrict__ O) {
  constexpr int WAVES = C::WAVES, QT = 2, HD = C::HD;
  constexpr long BQ = 64 * WAVES, NQB = C::SQ / BQ, PAIR = blocks_per_group<C>(), PER_B = NQB / PAIR;
  static_assert(C::SQ % BQ == 0 && C::SK % BK == 0, "exact blocks only");
  static_assert((HD == 64 || HD == 128) && (HD / 16) % WAVES == 0, "head dimension 64 or 128");
  __shared__ __attribute__((aligned(1024))) u16_t k0s[BK * HD], k1s[BK * HD], k2s[BK * HD], k3s[BK * HD];
  __shared__ __attribute__((aligned(1024))) u16_t v0s[BK * HD], v1s[BK * HD], v2s[BK * HD], v3s[BK * HD];
  __shared__ __attribute__((aligned(16))) u32x4 pbuf[2 * WAVES * QT * 2 * 64];
  __shared__ __attribute__((aligned(16))) float abuf[2 * WAVES * 64 * QT];
  __shared__ __attribute__((aligned(16))) float lbuf[WAVES * 64 * QT];
  u16_t* const ks[4] = {k0s, k1s, k2s, k3s};
  u16_t* const vs[4] = {v0s, v1s, v2s, v3s};
  const Lds<C> sh{ks, vs, pbuf, abuf, lbuf};

  // Tiles of one batch index go to one XCD (they share K and V in its L2); under a causal mask the
  // query blocks with the most keys start first.
  const long total = (long)gridDim.x;
  long t = (long)blockIdx.x;
  if (total % 8 == 0) t = (t % 8) * (total / 8) + t / 8;
  const long b = t / PER_B, p = t % PER_B;
  if (b >= C::NB) return;  // a grid larger than the work
  if constexpr (PAIR == 2) {
    flash_block<C>(sh, Q, K, V, O, b, NQB - 1 - p);
    gemm::wait_vmcnt<0>();  // the first block's output stores, before the second block's waits
    flash_block<C>(sh, Q, K, V, O, b, p);
  } else {
    flash_block<C>(sh, Q, K, V, O, b, C::CAUSAL ? NQB - 1 - p : p);
  }
}

// ---------------------------------------------------------------------------------------------
// f32 attention with a head dimension of 64: the reference's own flash pattern (f32 Q, K, V of head
// dimension 64, src/preparation/kernelization/lowering/flash.zig:24-31), on v_mfma_f32_32x32x2_f32.
//
// A workgroup of WAVES waves owns 32 * WAVES queries of one batch index; each wave keeps its 32
// queries' Q^T in registers and streams the keys in blocks of 32 through two LDS buffers. Lane half
// h = lane / 32 supplies head dims 32 h .. 32 h + 31 to both MFMA operands (any split of the
// contracted dims is valid when A and B agree), so one ds_read_b128 of a K row feeds four MFMAs.
// Per block of 32 keys:
//  * S^T = K Q^T: 32 MFMAs into one 32 x 32 accumulator (lane l: query l % 32, keys 8 g + 4 h + j in
//    register 4 g + j);
//  * online softmax in f32 in the log2 domain: the scores are scaled by SL = scale * log2 e, the
//    block maximum joins the running maximum (exchange with lane l ^ 32, which holds the same query),
//    O and the row sum are rescaled by exp2(m_old - m_new) every block;
//  * O^T += V^T P^T: two head-dim tiles x 16 key steps; step (g, j) takes key 8 g + j from lanes
//    0-31 and key 8 g + 4 + j from lanes 32-63, exactly the keys those lanes' score registers 4 g + j
//    hold, so P is the B operand as it stands; V is stored transposed in LDS so that one
//    ds_read_b128 gives the A operands of four steps;
// then O = O / l. LDS layouts (conflict-free 16-lane b128 reads on the 64-bank LDS): K as [key][64]
// with the 16-byte chunk c of key row r at chunk c ^ (r & 15); V^T as [64][32 keys] with the chunk of
// keys 4 kc .. 4 kc + 3 of row d at chunk kc ^ ((d / 2) & 7).
// The configuration struct C supplies WAVES, SQ, SK, NB, Q_S, K_S, V_S (element strides of a query /
// key row; head dims have stride 1), CAUSAL, SL and q_off / k_off / v_off (batch offsets). O is
// written row-major as [b][q][64]. Launched with 64 * WAVES threads, NB * SQ / (32 * WAVES) workgroups.
template <class C>
__device__ __forceinline__ void flash_f32(const float* __restrict__ Q, const float* __restrict__ K,
                                          const float* __restrict__ V, float* __restrict__ O) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  constexpr int WAVES = C::WAVES, D = 64, THREADS = 64 * WAVES, LD = 512 / THREADS;
  constexpr long BQ = 32 * WAVES, NQB = C::SQ / BQ;
  static_assert(C::SQ % BQ == 0 && C::SK % 32 == 0 && 512 % THREADS == 0, "exact blocks only");
  __shared__ __attribute__((aligned(16))) float ks[2][32 * D];
  __shared__ __attribute__((aligned(16))) float vt[2][D * 32];

  // Workgroups of one batch index go to one XCD (they share its K and V); under a causal mask the
  // query blocks with the most keys start first.
  const long total = (long)gridDim.x;
  long t = (long)blockIdx.x;
  if (total % 8 == 0) t = (t % 8) * (total / 8) + t / 8;
  const long b = t / NQB, qb = C::CAUSAL ? NQB - 1 - t % NQB : t % NQB;
  if (b >= C::NB) return;  // a grid larger than the work
  const int tid = (int)threadIdx.x, wave = tid >> 6, lane = tid & 63, h = lane >> 5, l32 = lane & 31;
  const long q0 = qb * BQ, query = q0 + 32 * wave + l32;
  const float* __restrict__ qp = Q + C::q_off(b);
  const float* __restrict__ kp = K + C::k_off(b);
  const float* __restrict__ vp = V + C::v_off(b);

  float qf[32];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const f32x4 x = *(const f32x4*)(qp + query * C::Q_S + 32 * h + 4 * i);
#pragma unroll
    for (int e = 0; e < 4; ++e) qf[4 * i + e] = x[e];
  }
  long nkb = C::SK / 32;
  if constexpr (C::CAUSAL) {
    const long last = (q0 + BQ - 1) / 32 + 1;
    nkb = last < nkb ? last : nkb;
  }

  // A block's K and V tiles (32 x 64 f32 each, 512 16-byte chunks): LD chunks of each per thread.
  f32x4 kr[LD], vr[LD];
  auto fetch = [&](long k0) {
#pragma unroll
    for (int i = 0; i < LD; ++i) {
      const int idx = tid + i * THREADS, row = idx >> 4, c = idx & 15;
      kr[i] = *(const f32x4*)(kp + (k0 + row) * C::K_S + 4 * c);
      vr[i] = *(const f32x4*)(vp + (k0 + row) * C::V_S + 4 * c);
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int i = 0; i < LD; ++i) {
      const int idx = tid + i * THREADS, row = idx >> 4, c = idx & 15;
      *(f32x4*)(&ks[buf][row * D + 4 * (c ^ (row & 15))]) = kr[i];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int d = 4 * c + e;
        vt[buf][d * 32 + 4 * ((row >> 2) ^ ((d >> 1) & 7)) + (row & 3)] = vr[i][e];
      }
    }
  };

  float m = -__builtin_inff(), l = 0.0f;
  f32x16 o[2] = {f32x16{}, f32x16{}};
  fetch(0);
  stash(0);
  __syncthreads();
  for (long j = 0; j < nkb; ++j) {
    const int buf = (int)(j & 1);
    if (j + 1 < nkb) fetch((j + 1) * 32);
    const float* kl = ks[buf];
    const float* vl = vt[buf];
    f32x16 s = f32x16{};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const f32x4 a = *(const f32x4*)(kl + l32 * D + 4 * ((8 * h + i) ^ (l32 & 15)));
#pragma unroll
      for (int e = 0; e < 4; ++e) s = gemm::mfma32x32x2f32(a[e], qf[4 * i + e], s);
    }
    const long k0 = j * 32;
    float mx = -__builtin_inff();
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float x = s[r] * C::SL;
      if constexpr (C::CAUSAL) {
        if (k0 + 8 * (r >> 2) + 4 * h + (r & 3) > query) x = -__builtin_inff();
      }
      s[r] = x;
      mx = fmaxf(mx, x);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mn = fmaxf(m, mx);
    const float msub = mn == -__builtin_inff() ? 0.0f : mn;
    const float alpha = __builtin_amdgcn_exp2f(m - msub);
    float ps = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s[r] = __builtin_amdgcn_exp2f(s[r] - msub);
      ps += s[r];
    }
    l = l * alpha + ps;
    m = mn;
    o[0] *= alpha;
    o[1] *= alpha;
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = dt * 32 + l32;
        const f32x4 a = *(const f32x4*)(vl + d * 32 + 4 * ((2 * g + h) ^ ((d >> 1) & 7)));
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) o[dt] = gemm::mfma32x32x2f32(a[jj], s[4 * g + jj], o[dt]);
      }
    // Buffer (j + 1) % 2 was last read in block j - 1, before the barrier that ended it.
    if (j + 1 < nkb) stash((int)((j + 1) & 1));
    __syncthreads();
  }
  const float inv = 1.0f / (l + __shfl_xor(l, 32, 64));
  float* __restrict__ orow = O + (b * C::SQ + query) * D;
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int g = 0; g < 4; ++g)
      *(f32x4*)(orow + dt * 32 + 8 * g + 4 * h) =
          f32x4{o[dt][4 * g] * inv, o[dt][4 * g + 1] * inv, o[dt][4 * g + 2] * inv, o[dt][4 * g + 3] * inv};
}

}  // namespace attn
}  // namespace accy
