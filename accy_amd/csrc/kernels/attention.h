// Fused attention O[b, q, :] = softmax_k(scale * Q[b, q, :] . K[b, k, :] [masked k > q]) V[b, k, :] on
// gfx950 matrix cores, for 16-bit Q, K, V with a head dimension HD of 64 or 128 (both for Q.K and for
// V), and (flash_f32, at the end) for f32 Q, K, V with a head dimension of 64.
//
// A workgroup of WAVES wavefronts owns 32 * WAVES queries of one batch index (32 per wave) and
// streams the keys in blocks of 32; see the work split below.
//
// Orientation: the scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16. In the
// 32 x 32 accumulator layout lane l then holds one query (column l % 32) and 16 keys (rows
// 8 g + 4 (l / 32) + j at register 4 g + j), so a row maximum or sum over the keys is a register
// fold plus one exchange with lane l ^ 32. The Q^T operand (B) is the same for every key block and
// stays in registers. The probabilities P^T are packed to 16 bits and serve as the B
// operand of O^T = V^T P^T: registers 8 s .. 8 s + 7 of a score tile are the B operand of 16-key
// step s when both operands number the keys of that step in the same permuted order (slot
// 8 h + 4 r + t holds key 16 s + 8 r + 4 h + t), which the V^T fragment read (ds_read_b64_tr_b16
// with rows 16 s + 8 r + 4 h + t) follows, so P never leaves the registers.
//
// Softmax: f32 throughout, online over key blocks in the log2 domain: e = exp2(s * scale * log2 e -
// m) with v_exp_f32. The subtracted maximum m only moves when the running maximum exceeds it by more
// than 8 (a factor 256), so the accumulators are rescaled rarely; e <= 256 stays well inside the
// 16-bit range of the P operand. Row sums accumulate the 16-bit rounded e that the P.V product
// consumes (a dot product of each packed pair with ones), so numerator and denominator weight every
// key alike; the result is O / sum.
//
// A workgroup runs one or two query blocks (blocks_per_group); with two, the first issues the
// second's first loads after its last barrier.
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
// O is written row-major as [b][q][HD]. The kernel is launched with 64 * WAVES threads.
#pragma once

namespace accy {
namespace attn {

using gemm::f32x16;
using gemm::f32x4;
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
//    reads one chunk of 16 consecutive rows: with rows of 256 bytes (HD 128) the XOR with
//    r & 15 spreads them over the 16 positions of a 256-byte bank window; with 128-byte rows (HD 64)
//    two rows share 256 bytes, and the XOR with (r / 2) & 7 spreads the 8 row pairs.
//  * V: the 32-byte unit u of key row r sits at unit u ^ v_swizzle(r). A 32-lane half of a transposed
//    read covers units (u, u ^ 1) of four consecutive rows: 256-byte rows use
//    gemm::tr_swizzle (2 (r & 3)); 128-byte rows (4 units, two rows per 256 bytes) XOR with
//    2 ((r / 2) & 1).
template <int HD> __device__ __forceinline__ int k_swizzle(int r) { return HD == 128 ? (r & 15) : ((r >> 1) & 7); }
template <int HD> __device__ __forceinline__ int v_swizzle(int r) { return HD == 128 ? gemm::tr_swizzle(r) : 2 * ((r >> 1) & 1); }

// Byte offsets, within a tile, of one lane's pieces of the K / V tiles, computed once per query
// block. The per-step accesses then add only compile-time constants (LDS stage, key step) or a scalar
// base (the key block in global memory), so a step spends no VALU instructions on addresses; the
// offsets go through an empty asm statement so that the compiler keeps them in registers instead
// of recomputing them inside the loop.
template <int HD, int WAVES, long KS, long VS>
struct TileOffsets {
  static constexpr int DS = HD / 16, DTN = HD / 32, PER = HD / 16 / WAVES;
  static constexpr int LPR = HD / 8, RPI = 64 / LPR;  // lanes per 16-byte-chunked row, rows per load
  u32_t kf[DS];   // K fragment (A operand of S^T) of head-dim step dd: row lane % 32, chunk 2 dd + lane / 32
  u32_t vf[DTN];  // V^T fragment (ds_read_b64_tr_b16) of head-dim tile dt, for key step 0, half 0
  u32_t kg[PER];  // this lane's 16-byte chunk of K load i in global memory, and its LDS position
  u32_t vg[PER];

  __device__ __forceinline__ void init(int wave, int lane) {
    const int row = lane & 31;
#pragma unroll
    for (int dd = 0; dd < DS; ++dd) kf[dd] = 2u * (u32_t)(row * HD + (((2 * dd + (lane >> 5)) ^ k_swizzle<HD>(row)) << 3));
    // V^T fragment: lanes 16 g + i read key 4 (g / 2) + i / 4 (+ 16 s + 8 r for key step s, half r, which
    // the swizzle does not see) at column unit 2 dt + (g & 1), element 4 (i & 3)
    const int g = lane >> 4, i = lane & 15, k = 4 * (g >> 1) + (i >> 2);
#pragma unroll
    for (int dt = 0; dt < DTN; ++dt) {
      const int unit = (2 * dt + (g & 1)) ^ v_swizzle<HD>(k);
      vf[dt] = 2u * (u32_t)(k * HD + unit * 16 + 4 * (i & 3));
    }
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int r = RPI * (wave * PER + j) + lane / LPR, p = lane % LPR;
      kg[j] = 2u * (u32_t)(r * KS + 8 * ((p ^ k_swizzle<HD>(r))));
      vg[j] = 2u * (u32_t)(r * VS + 16 * ((p >> 1) ^ v_swizzle<HD>(r)) + 8 * (p & 1));
    }
#pragma unroll
    for (int dd = 0; dd < DS; ++dd) asm volatile("" : "+v"(kf[dd]));
#pragma unroll
    for (int dt = 0; dt < DTN; ++dt) asm volatile("" : "+v"(vf[dt]));
#pragma unroll
    for (int j = 0; j < PER; ++j) asm volatile("" : "+v"(kg[j]), "+v"(vg[j]));
  }
};

// Issues one wave's share (PER instructions of 1 KiB) of the tile whose first row starts at element
// `first` of g, into LDS tile `lds` (16-byte chunk positions as the offsets say).
template <int PER>
__device__ __forceinline__ void dma_share(const u16_t* __restrict__ g, long first, const u32_t (&go)[PER], u16_t* lds, int wave) {
  const char* base = (const char*)(g + first);
#pragma unroll
  for (int j = 0; j < PER; ++j) gemm::dma16(base + go[j], (ACCY_LDS void*)(lds + (wave * PER + j) * 512));
}

// A operand of S^T for head-dim step dd from K stage `lds`.
__device__ __forceinline__ u32x4 k_frag(const u16_t* lds, u32_t off) { return *(const u32x4*)((const char*)lds + off); }

// A operand of O^T = V^T P^T for one head-dim tile (offset off) and 16-key step s, keys in the
// permuted order: halves r = 0, 1 are rows 16 s + 8 r + ... of the tile.
template <int HD>
__device__ __forceinline__ u32x4 v_frag(const u16_t* lds, u32_t off, int s) {
  u32x4 out;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (ACCY_LDS i16x4*)((const char*)lds + off + 2 * (16 * s + 8 * r) * HD));
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
  float a, b, r;
  with_partner(x, a, b);
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));  // no canonicalising moves (no signalling NaNs here)
  return r;
}
__device__ __forceinline__ float sum_with_partner(float x) {
  float a, b;
  with_partner(x, a, b);
  return a + b;
}

// Work split. Every wave owns 32 queries and does all of their work: S^T = K Q^T, the online
// softmax and O^T += V^T P^T, with P kept in registers (the score registers of a block, packed in
// pairs, are the B operand of its P.V product as they stand). Two waves share each SIMD (one
// workgroup of eight waves per CU, or two of four): each wave interleaves its own MFMAs with its
// softmax VALU work, and the two waves take turns on the matrix core.
// Step t of a query block (nkb + 2 steps), on K stage t % 4:
//  * the MFMAs of S(t) (HD / 16, for t < nkb) alternate with those of P(t - 2).V(t - 2) (HD / 16,
//    for t >= 2, V stage (t - 2) % 4);
//  * the softmax of block t - 1 (for 1 <= t <= nkb) runs between them, one pair of scores (exp2,
//    packing, row sum) per slot, with the subtracted maximum of the earlier blocks; a check of the
//    block's row sum then sends the rare block that moves the maximum to the exact path;
//  * at the end of the step O is rescaled for block t - 1 when its maximum moved (rarely), between
//    the P.V of block t - 2 and that of block t - 1;
//  * even steps meet the workgroup at a barrier and then issue K(t + 2), K(t + 3), V(t) and
//    V(t + 1) to their stages: every tile is issued at least two steps before its use, and every
//    stage is rewritten only after the barrier that follows its last read.
// What bounds it (C4 on MI355X): the chip's power limit. The MFMAs, the softmax's ~90 VALU
// instructions per wave and step and the LDS reads add up to about the measured time, and the
// clock drops as the work per cycle rises; every instruction removed from the loop counts.
template <class C>
struct Lds {
  u16_t* const* ks;  // K stages [4][BK * HD]
  u16_t* const* vs;  // V stages [4][BK * HD]
};

template <class C>
struct Worker {
  static constexpr int HD = C::HD, WAVES = C::WAVES, DS = HD / 16, DTN = HD / 32;
  static constexpr int NPV = 2 * DTN;          // P.V MFMAs per key block (= DS score MFMAs)
  static constexpr int PER = HD / 16 / WAVES;  // K and V load instructions per wave per key block
  static_assert(NPV == DS, "score and P.V MFMAs alternate one for one");

  Lds<C> sh;
  const u16_t* __restrict__ kb;
  const u16_t* __restrict__ vb;
  TileOffsets<HD, WAVES, C::K_S, C::V_S> off;
  u32x4 qf[DS];    // Q^T, the B operand of S^T for head-dim step dd
  f32x16 s[2];     // scores of the blocks of even / odd index
  f32x16 o[DTN];   // O^T, head-dim tile dt
  u32x4 p[2][2];   // P of the blocks of even / odd index: the B operands of their two 16-key steps
  float alpha[2];  // factor for O and l of the block of even / odd index (1 if the maximum did not move)
  float m, l;      // subtracted maximum (log2 domain, finite) and this lane's half of the row sum
  long q0;
  int wave, lane;
  // The workgroup's next query block (blocks run back to back): once every wave has read the last
  // K stage of this block, its Q^T and its first two K tiles are issued (ready: this block's were).
  const u16_t* next_q = nullptr;  // Q of the batch index, or nullptr when no block follows
  long next_q0 = 0, next_nkb = 0;
  bool ready = false;

  __device__ __forceinline__ long query() const { return q0 + 32 * wave + (lane & 31); }

  // Q^T of the queries q0 + 32 wave + (lane & 31) (this wave's 32 queries) into registers.
  __device__ __forceinline__ void load_q(const u16_t* __restrict__ qp, long first) {
    const long q = first + 32 * wave + (lane & 31);
#pragma unroll
    for (int dd = 0; dd < DS; ++dd) qf[dd] = *(const u32x4*)(qp + q * C::Q_S + 16 * dd + 8 * (lane >> 5));
  }

  // Called after the workgroup's last meeting at or after step nkb: no wave reads K any more, so
  // the next block's Q^T (into qf, free since the last score MFMA) and K(0), K(1) can be issued.
  __device__ __forceinline__ void issue_next() {
    if (next_q == nullptr) return;
    load_q(next_q, next_q0);
    dma_share<PER>(kb, 0, off.kg, sh.ks[0], wave);
    if (next_nkb > 1) dma_share<PER>(kb, BK * C::K_S, off.kg, sh.ks[1], wave);
  }

  // Scores of keys above the query are -inf (blocks that cross the diagonal only). Register r holds
  // key k0 + 8 (r / 4) + 4 (lane / 32) + r % 4, so the test is one 32-bit compare of a constant
  // against the lane's threshold (query - k0 - 4 (lane / 32)).
  template <int PB>
  __device__ __forceinline__ void mask(long k0) {
    if (k0 + BK - 1 <= q0 + 32 * wave) return;
    const int th = (int)(query() - k0) - 4 * (lane >> 5);
#pragma unroll
    for (int r = 0; r < 16; ++r)
      if (8 * (r >> 2) + (r & 3) > th) s[PB][r] = -__builtin_inff();
  }

  // Softmax of the block in score set PB, for scores 2 j and 2 j + 1: P = exp2(s * SL - m) with the
  // subtracted maximum m of the earlier blocks, packed to 16 bits (the B operand of 16-key step
  // j / 4), and the packed pair's exact sum into ls, this lane's part of the block's row sum.
  template <int PB, int J>
  __device__ __forceinline__ void pair(float ml, float& ls) {
    const f32x16& sp = s[PB];
    const float e0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sp[2 * J], C::SL, ml));
    const float e1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sp[2 * J + 1], C::SL, ml));
    const u32_t pr = pack2<C::DT>(e0, e1);
    p[PB][J >> 2][J & 3] = pr;
    ls = add_pair<C::DT>(pr, ls);
  }

  // The lazy maximum. m moves only when a block's maximum exceeds it by more than 8 (a factor 256),
  // so P stays <= 256. The exponentials are computed first with the old m; a lane whose block sum
  // stays <= 256 has every P <= 256, and when every lane's does (the common case) nothing else is
  // needed. Otherwise this takes the row maximum (two max3 chains, then the partner lane's half),
  // moves m where it must, sets alpha (the factor for O and l) and recomputes the block. m starts
  // at -FLT_MAX, so the first block always comes here (its exponentials overflow), and
  // s * SL - m is -inf exactly for the masked scores.
  template <int PB>
  __device__ __forceinline__ void exact_block(float& ls) {
    const f32x16& sp = s[PB];
    float a = max3(sp[0], sp[1], sp[2]), b = max3(sp[3], sp[4], sp[5]);
    a = max3(a, sp[6], sp[7]);
    b = max3(b, sp[8], sp[9]);
    a = max3(a, sp[10], sp[11]);
    b = max3(b, sp[12], sp[13]);
    a = max3(a, sp[14], sp[15]);
    const float mn = max_with_partner(max3(a, b, b)) * C::SL;
    const bool need = mn > m + 8.0f;
    if (__any(need)) {
      alpha[PB] = need ? __builtin_amdgcn_exp2f(m - mn) : 1.0f;
      m = need ? mn : m;
      ls = 0.0f;
      For<0, 8>::run([&](auto ji) { pair<PB, decltype(ji)::value>(-m, ls); });
    }
  }

  // Even step t (K stage ST = t % 4) meets the workgroup: every load in flight (issued at step
  // t - 2: K(t), K(t + 1), V(t - 2), V(t - 1)) is complete and the stages read at steps t - 2 and
  // t - 1 are free; then this wave's share of K(t + 2), K(t + 3), V(t) and V(t + 1) is issued (tiles
  // up to the workgroup's key block count nkb).
  template <int ST>
  __device__ __forceinline__ void meet(long t, long nkb) {
    gemm::wait_vmcnt<0>();
    gemm::lds_reads_done_barrier();
    if (t + 2 < nkb) dma_share<PER>(kb, (t + 2) * BK * C::K_S, off.kg, sh.ks[(ST + 2) & 3], wave);
    if (t + 3 < nkb) dma_share<PER>(kb, (t + 3) * BK * C::K_S, off.kg, sh.ks[(ST + 3) & 3], wave);
    if (t < nkb) dma_share<PER>(vb, t * BK * C::V_S, off.vg, sh.vs[ST], wave);
    if (t + 1 < nkb) dma_share<PER>(vb, (t + 1) * BK * C::V_S, off.vg, sh.vs[(ST + 1) & 3], wave);
  }

  // Step t on K stage ST = t % 4: S(t) when HS, the softmax of block t - 1 when HM, P.V of block
  // t - 2 when HP. Score sets, P sets and factors of block j live at index j % 2.
  template <int ST, bool HS, bool HM, bool HP>
  __device__ __forceinline__ void step(long t, long nkb) {
    constexpr int SB = ST & 1, PB = SB ^ 1, NE = (HS ? DS : 0) + (HP ? NPV : 0);
    constexpr int VST = (ST + 2) & 3;
    if constexpr ((ST & 1) == 0) meet<ST>(t, nkb);
    if constexpr (HM)
      if constexpr (C::CAUSAL) mask<PB>((t - 1) * BK);

    const u16_t* kl = sh.ks[ST];
    const u16_t* vl = sh.vs[VST];
    constexpr int PF = 2;  // fragments read ahead of their MFMA
    u32x4 kf[PF + 1], vf[PF + 1];
    if constexpr (HS) {
      For<0, PF>::run([&](auto ii) { constexpr int i = decltype(ii)::value; if constexpr (i < DS) kf[i] = k_frag(kl, off.kf[i]); });
      s[SB] = f32x16{};
    }
    if constexpr (HP)
      For<0, PF>::run([&](auto ii) { constexpr int i = decltype(ii)::value; if constexpr (i < NPV) vf[i] = v_frag<HD>(vl, off.vf[i / 2], i % 2); });
    // The softmax of block t - 1: pair 0 while the first fragments arrive, pairs 1-7 between the
    // MFMAs, then the check of the lazy maximum.
    const float ml = -m;
    float ls = 0.0f;
    auto slot = [&](auto ji) { pair<PB, decltype(ji)::value>(ml, ls); };
    if constexpr (HM) slot(Int<0>{});
    __builtin_amdgcn_sched_barrier(0);
    For<0, NE>::run([&](auto ei) {
      constexpr int e = decltype(ei)::value;
      // event e: score MFMA e / 2 and P.V MFMA e / 2 alternate when both are present
      constexpr bool is_s = HS && (!HP || (e & 1) == 0);
      constexpr int i = HS && HP ? e / 2 : e;
      if constexpr (is_s) {
        if constexpr (i + PF < DS) kf[(i + PF) % (PF + 1)] = k_frag(kl, off.kf[i + PF]);
        s[SB] = gemm::mfma32x32x16<C::DT>(kf[i % (PF + 1)], qf[i], s[SB]);
      } else {
        // P.V MFMA i: head-dim tile i / 2, 16-key step i % 2
        if constexpr (i + PF < NPV) vf[(i + PF) % (PF + 1)] = v_frag<HD>(vl, off.vf[(i + PF) / 2], (i + PF) % 2);
        o[i / 2] = gemm::mfma32x32x16<C::DT>(vf[i % (PF + 1)], p[SB][i % 2], o[i / 2]);
      }
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (HM) For<1 + e * 7 / NE, 1 + (e + 1) * 7 / NE>::run(slot);
      __builtin_amdgcn_sched_barrier(0);
    });
    if constexpr (HM) {
      if constexpr (NE == 0) For<1, 8>::run(slot);
      alpha[PB] = 1.0f;
      if (__any(!(ls <= 256.0f))) exact_block<PB>(ls);
      l = l * alpha[PB] + ls;
      // The softmax results are consumed here, so that no pass sinks their VALU work past the next
      // barrier (out of the MFMA slots it was placed in).
      asm volatile("" : "+v"(p[PB][0]), "+v"(p[PB][1]), "+v"(l), "+v"(alpha[PB]));
      // O is rescaled for block t - 1 after this step's P.V of block t - 2 and before the next step's
      // P.V of block t - 1 (rarely: only when the maximum moved).
      if (__any(alpha[PB] != 1.0f)) {
#pragma unroll
        for (int dt = 0; dt < DTN; ++dt) o[dt] *= alpha[PB];
      }
    }
  }

  // One query block: prologue (Q^T into registers, K(0) and K(1) issued), nkc + 2 steps over this
  // wave's key blocks, epilogue, then the workgroup's remaining steps (nkb - nkc = 0 or 4; key
  // blocks that are masked for every query of this wave) only meet the workgroup and issue loads.
  __device__ __forceinline__ void run(const u16_t* __restrict__ qp, u16_t* __restrict__ out, long b, long nkb,
                                      long nkc) {
    if (!ready) {
      load_q(qp, q0);
      off.init(wave, lane);
      dma_share<PER>(kb, 0, off.kg, sh.ks[0], wave);
      if (nkb > 1) dma_share<PER>(kb, BK * C::K_S, off.kg, sh.ks[1], wave);
    }
#pragma unroll
    for (int dt = 0; dt < DTN; ++dt) o[dt] = f32x16{};
    m = -0x1.fffffep127f;
    l = 0.0f;
    alpha[0] = alpha[1] = 1.0f;
    step0(nkb);
    if (nkb == 1) {
      step<1, false, true, false>(1, nkb);
      step<2, false, false, true>(2, nkb);
      issue_next();
    } else {
      steps(nkb, nkc);
    }
    epilogue(out, b);
    if (nkc < nkb) {
      // nkc = 0 (mod 4): the remaining even steps are nkc + 2 and nkc + 4 (= nkb, the last meeting)
      meet<2>(nkc + 2, nkb);
      meet<0>(nkc + 4, nkb);
      issue_next();
    }
  }

  // Steps 1 .. nkc + 1 for nkc >= 2 (loads up to nkb). The steady-state loop leaves t = 2 (mod 4),
  // so the stage of every remaining step is known; r = nkc - t scored steps remain (0 .. 3).
  __device__ __forceinline__ void steps(long nkb, long nkc) {
    step<1, true, true, false>(1, nkb);
    long t = 2;
    for (; t + 3 < nkc; t += 4) {
      step<2, true, true, true>(t, nkb);
      step<3, true, true, true>(t + 1, nkb);
      step<0, true, true, true>(t + 2, nkb);
      step<1, true, true, true>(t + 3, nkb);
    }
    // nkb % 4 is known at compile time in the common shapes (non-causal, or causal with query blocks
    // and key counts that are multiples of 128); then only that tail is compiled.
    constexpr long BQ = 32 * WAVES, NKB = C::SK / BK;
    constexpr int MOD = !C::CAUSAL ? (int)((NKB - 2) % 4) : (BQ % 128 == 0 && C::SK % 128 == 0 ? 2 : -1);
    const long r = MOD >= 0 ? MOD : nkc - t;
    // The next block's loads follow the first meeting at or after step nkc (the last one of this
    // block when nkc == nkb).
    const bool last = nkc == nkb;
    if (r == 0) {
      step<2, false, true, true>(t, nkb);
      if (last) issue_next();
      step<3, false, false, true>(t + 1, nkb);
    } else if (r == 1) {
      step<2, true, true, true>(t, nkb);
      step<3, false, true, true>(t + 1, nkb);
      step<0, false, false, true>(t + 2, nkb);
      if (last) issue_next();
    } else if (r == 2) {
      step<2, true, true, true>(t, nkb);
      step<3, true, true, true>(t + 1, nkb);
      step<0, false, true, true>(t + 2, nkb);
      if (last) issue_next();
      step<1, false, false, true>(t + 3, nkb);
    } else {
      step<2, true, true, true>(t, nkb);
      step<3, true, true, true>(t + 1, nkb);
      step<0, true, true, true>(t + 2, nkb);
      step<1, false, true, true>(t + 3, nkb);
      step<2, false, false, true>(t + 4, nkb);
      if (last) issue_next();
    }
  }

  // O = O^T / l, rounded to the element type, row-major [b][q][HD].
  __device__ __forceinline__ void epilogue(u16_t* __restrict__ out, long b) {
    const float inv = 1.0f / sum_with_partner(l);
    const int h = lane >> 5;
    u16_t* __restrict__ orow = out + (b * C::SQ + query()) * HD;
#pragma unroll
    for (int dt = 0; dt < DTN; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x16& acc = o[dt];
        const u32_t lo = pack2_out<C::DT>(acc[4 * g] * inv, acc[4 * g + 1] * inv);
        const u32_t hi = pack2_out<C::DT>(acc[4 * g + 2] * inv, acc[4 * g + 3] * inv);
        *(u32x2*)(orow + dt * 32 + 8 * g + 4 * h) = u32x2{lo, hi};
      }
  }

  // Step 0: K(0) and K(1) complete, barrier, K(2), K(3), V(0) and V(1) issued, S(0).
  __device__ __forceinline__ void step0(long nkb) {
    gemm::wait_vmcnt<0>();
    gemm::lds_reads_done_barrier();
    if (2 < nkb) dma_share<PER>(kb, 2 * BK * C::K_S, off.kg, sh.ks[2], wave);
    if (3 < nkb) dma_share<PER>(kb, 3 * BK * C::K_S, off.kg, sh.ks[3], wave);
    dma_share<PER>(vb, 0, off.vg, sh.vs[0], wave);
    if (1 < nkb) dma_share<PER>(vb, BK * C::V_S, off.vg, sh.vs[1], wave);
    const u16_t* kl = sh.ks[0];
    u32x4 kf[3];
    kf[0] = k_frag(kl, off.kf[0]);
    kf[1] = k_frag(kl, off.kf[1]);
    s[0] = f32x16{};
    For<0, DS>::run([&](auto ii) {
      constexpr int i = decltype(ii)::value;
      if constexpr (i + 2 < DS) kf[(i + 2) % 3] = k_frag(kl, off.kf[i + 2]);
      s[0] = gemm::mfma32x32x16<C::DT>(kf[i % 3], qf[i], s[0]);
    });
  }
};

// Query blocks per workgroup. Under a causal mask with an even number of query blocks, a workgroup
// takes block NQB - 1 - p and then block p, so that every workgroup streams the same number of key
// blocks (the heavy blocks start first). Without a mask, pairs of blocks when that leaves a whole
// number of rounds of 256 workgroups (one per CU of an MI355X): the second block's Q^T and first K
// tiles load during the first block's last steps instead of after a workgroup launch. The grid is
// NB * NQB / blocks_per_group workgroups.
template <class C>
constexpr long blocks_per_group() {
  constexpr long NQB = C::SQ / (32 * C::WAVES);
  if constexpr (C::CAUSAL) return NQB % 2 == 0 ? 2 : 1;
  return NQB % 2 == 0 && (C::NB * NQB) % 512 == 0 ? 2 : 1;
}

// Key blocks a query block starting at q0 reads (under the causal mask, up to its last query).
template <class C>
__device__ __forceinline__ long key_blocks(long q0) {
  constexpr long BQ = 32 * C::WAVES, NKB = C::SK / BK;
  long nkb = NKB;
  if constexpr (C::CAUSAL) {
    const long last = (q0 + BQ - 1) / BK + 1;
    nkb = last < nkb ? last : nkb;
  }
  return nkb;
}

// One query block (queries qb * 32 * WAVES ...) of batch index b on worker f (Qb: the batch index's
// Q). Every wave meets the same barriers, so blocks can follow each other.
template <class C>
__device__ __forceinline__ void flash_block(Worker<C>& f, const u16_t* __restrict__ Qb, u16_t* __restrict__ O, long b,
                                            long qb) {
  constexpr long BQ = 32 * C::WAVES;
  const long q0 = qb * BQ, nkb = key_blocks<C>(q0);
  f.q0 = q0;
  // Under the causal mask the last four key blocks of a 256-query block lie above the diagonal for
  // every query of waves 0-3 (queries q0 .. q0 + 127) when the block's keys reach its last query:
  // those waves skip their work and only meet the workgroup there. With waves w and w + 4 on one
  // SIMD, each SIMD then carries 12 instead of 16 wave-steps over the diagonal. (Only where the
  // loop tail is fixed at compile time: nkb = 0 (mod 4).)
  long nkc = nkb;
  if constexpr (C::CAUSAL && C::WAVES == 8 && C::SK % 128 == 0)
    if (f.wave < 4 && nkb == (q0 + BQ - 1) / BK + 1) nkc = nkb - 4;
  f.run(Qb, O, b, nkb, nkc);
}

// Workgroup of C::WAVES waves (64 * C::WAVES threads) over blocks_per_group<C>() query blocks of
// 32 * C::WAVES queries of one batch index.
template <class C>
__device__ __forceinline__ void flash(const u16_t* __restrict__ Q, const u16_t* __restrict__ K,
                                      const u16_t* __restrict__ V, u16_t* __restrict__ O) {
  constexpr int WAVES = C::WAVES, HD = C::HD;
  constexpr long BQ = 32 * WAVES, NQB = C::SQ / BQ, PAIR = blocks_per_group<C>(), PER_B = NQB / PAIR;
  static_assert(C::SQ % BQ == 0 && C::SK % BK == 0, "exact blocks only");
  static_assert((HD == 64 || HD == 128) && (HD / 16) % WAVES == 0, "head dimension 64 or 128, whole load shares");
  __shared__ __attribute__((aligned(1024))) u16_t k0s[BK * HD], k1s[BK * HD], k2s[BK * HD], k3s[BK * HD];
  __shared__ __attribute__((aligned(1024))) u16_t v0s[BK * HD], v1s[BK * HD], v2s[BK * HD], v3s[BK * HD];
  u16_t* const ks[4] = {k0s, k1s, k2s, k3s};
  u16_t* const vs[4] = {v0s, v1s, v2s, v3s};

  // Tiles of one batch index go to one XCD (they share K and V in its L2); under a causal mask the
  // query blocks with the most keys start first.
  const long total = (long)gridDim.x;
  long t = (long)blockIdx.x;
  if (total % 8 == 0) t = (t % 8) * (total / 8) + t / 8;
  const long b = t / PER_B, p = t % PER_B;
  if (b >= C::NB) return;  // a grid larger than the work
  Worker<C> f;
  f.sh = Lds<C>{ks, vs};
  f.kb = K + C::k_off(b);
  f.vb = V + C::v_off(b);
  f.wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  f.lane = (int)(threadIdx.x & 63);
  const u16_t* __restrict__ Qb = Q + C::q_off(b);
  if constexpr (PAIR == 2) {
    // one copy of the block code, run twice; the first issues the second's first loads
#pragma unroll 1
    for (int i = 0; i < 2; ++i) {
      f.next_q = i == 0 ? Qb : nullptr;
      f.next_q0 = p * BQ;
      f.next_nkb = key_blocks<C>(p * BQ);
      f.ready = i == 1;
      flash_block<C>(f, Qb, O, b, i == 0 ? NQB - 1 - p : p);
    }
  } else {
    flash_block<C>(f, Qb, O, b, C::CAUSAL ? NQB - 1 - p : p);
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
