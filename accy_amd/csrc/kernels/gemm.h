// Dense contraction C[b, m, n] = sum_k A[b, m, k] * B[b, k, n] on gfx950 matrix cores.
//
// Hand-written for CDNA4: f32 accumulation in v_mfma_f32_32x32x16_{bf16,f16}; a 256 x 256 x 64
// block tile computed by 8 wavefronts (4 along M x 2 along N), each owning a 64 x 128 sub-tile of
// 2 x 4 MFMA 32x32 accumulators; both operands staged through LDS with K innermost (rows padded by
// 16 bytes so that the 16-byte fragment reads of 8 consecutive lanes hit distinct banks) and double
// buffered, so one barrier per K step separates the LDS writes of tile k+1 from the reads of tile k
// while the global loads of tile k+1 are in flight under the MFMAs of tile k.
//
// Operand layouts: an operand whose K stride is 1 is loaded as 16-byte vectors along K and written
// to LDS unchanged; an operand whose M (or N) stride is 1 is loaded as 8 x 8 blocks (8 vectors along
// M/N at 8 consecutive k) and transposed in registers before the LDS write. Blocks are renumbered so
// that the tiles dispatched to one XCD are neighbours (shared A rows / B columns in that XCD's L2).
//
// The configuration struct C supplies extents, strides (elements), tile shape and dtype; the
// epilogue functor receives (batch, m, n, f32 accumulator) for every in-range output element.
#pragma once

namespace accy {
namespace gemm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef u32_t u32x4 __attribute__((ext_vector_type(4)));

template <int DT>
__device__ __forceinline__ f32x16 mfma32x32x16(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (DT == 0) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  }
}

// 8 x 8 transpose of 16-bit elements: in[k] holds 8 consecutive rows at one k; out[r] holds 8
// consecutive k of one row.
__device__ __forceinline__ void transpose8x8(const u32x4 (&in)[8], u32x4 (&out)[8]) {
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const int w = r >> 1;
    const bool hi = r & 1;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const u32_t lo_src = in[2 * d][w], hi_src = in[2 * d + 1][w];
      out[r][d] = hi ? ((lo_src >> 16) | (hi_src & 0xffff0000u)) : ((lo_src & 0xffffu) | (hi_src << 16));
    }
  }
}

// Tile numbering: dispatch order round-robins workgroups over the 8 XCDs; give each XCD a
// contiguous range of tiles, then walk that range in groups of GROUP_M tile rows.
template <long TILES_M, long TILES_N, int GROUP_M>
__device__ __forceinline__ void tile_of(long bid, long& tm, long& tn) {
  constexpr long TILES = TILES_M * TILES_N;
  if constexpr (TILES % 8 == 0) bid = (bid % 8) * (TILES / 8) + bid / 8;
  const long per_group = (long)GROUP_M * TILES_N;
  const long group = bid / per_group;
  const long first_m = group * GROUP_M;
  const long gsize = (TILES_M - first_m) < GROUP_M ? (TILES_M - first_m) : GROUP_M;
  tm = first_m + (bid % per_group) % gsize;
  tn = (bid % per_group) / gsize;
}

// Loads one operand tile (ROWS rows of the operand's M or N, BK values of K) into registers.
// KC: K stride is 1 (vectors along K); otherwise the row stride is 1 (8 x 8 blocks, transposed).
template <int ROWS, int BK, int THREADS, bool KC, long RT, long KT, long SR, long SK>
struct TileLoader {
  static constexpr int VEC_PER_ROW = BK / 8;
  static constexpr int VECS = ROWS * BK / 8;
  static constexpr int PER_THREAD = VECS / THREADS;
  static_assert(VECS % THREADS == 0, "tile vectors must divide evenly among loader threads");
  static_assert(KC || PER_THREAD % 8 == 0, "transposing loader handles whole 8 x 8 blocks");
  u32x4 v[PER_THREAD];

  __device__ __forceinline__ void load(const u16_t* __restrict__ base, long r0, long k0, int t) {
    if constexpr (KC) {
#pragma unroll
      for (int i = 0; i < PER_THREAD; ++i) {
        const int idx = t + i * THREADS;
        const int row = idx / VEC_PER_ROW, kc = idx % VEC_PER_ROW;
        const long r = r0 + row, k = k0 + kc * 8;
        if ((RT % 256 == 0 || r < RT) && (KT % 64 == 0 || k < KT))
          v[i] = *(const u32x4*)(base + r * SR + k);
        else
          v[i] = u32x4{0, 0, 0, 0};
      }
    } else {
      constexpr int RG = ROWS / 8;
#pragma unroll
      for (int b = 0; b < PER_THREAD / 8; ++b) {
        const int bidx = t + b * THREADS;
        const int kg = bidx / RG, rg = bidx % RG;
        const long r = r0 + rg * 8;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const long k = k0 + kg * 8 + i;
          if ((RT % 256 == 0 || r < RT) && (KT % 64 == 0 || k < KT))
            v[b * 8 + i] = *(const u32x4*)(base + k * SK + r);
          else
            v[b * 8 + i] = u32x4{0, 0, 0, 0};
        }
      }
    }
  }

  // Writes the staged tile into LDS as [row][k] with row stride LDK.
  template <int LDK>
  __device__ __forceinline__ void store(u16_t* __restrict__ lds, int t) {
    if constexpr (KC) {
#pragma unroll
      for (int i = 0; i < PER_THREAD; ++i) {
        const int idx = t + i * THREADS;
        const int row = idx / VEC_PER_ROW, kc = idx % VEC_PER_ROW;
        *(u32x4*)(lds + row * LDK + kc * 8) = v[i];
      }
    } else {
      constexpr int RG = ROWS / 8;
#pragma unroll
      for (int b = 0; b < PER_THREAD / 8; ++b) {
        const int bidx = t + b * THREADS;
        const int kg = bidx / RG, rg = bidx % RG;
        u32x4 in[8], out[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) in[i] = v[b * 8 + i];
        transpose8x8(in, out);
#pragma unroll
        for (int j = 0; j < 8; ++j) *(u32x4*)(lds + (rg * 8 + j) * LDK + kg * 8) = out[j];
      }
    }
  }
};

// One workgroup computes one BM x BN tile of one batch element. Needs BM*BN... LDS of
// 2 * (BM + BN) * (BK + 8) 16-bit elements, passed as dynamic shared memory.
template <class C, class Epi>
__device__ __forceinline__ void mma16(const u16_t* __restrict__ A, const u16_t* __restrict__ B, const Epi& epi) {
  constexpr int BM = C::BM, BN = C::BN, BK = C::BK, LDK = BK + 8;
  constexpr int WAVES = C::WAVES_M * C::WAVES_N, THREADS = WAVES * 64, HALF = THREADS / 2;
  constexpr int WTM = BM / C::WAVES_M, WTN = BN / C::WAVES_N;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  constexpr long TILES_M = (C::M + BM - 1) / BM, TILES_N = (C::N + BN - 1) / BN;
  constexpr long KTILES = (C::K + BK - 1) / BK;
  constexpr int STAGE = (BM + BN) * LDK;
  extern __shared__ u16_t lds[];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / C::WAVES_N, wn = wave % C::WAVES_N;
  long tm, tn;
  tile_of<TILES_M, TILES_N, 8>((long)blockIdx.x, tm, tn);
  const long m0 = tm * BM, n0 = tn * BN, batch = blockIdx.y;
  const u16_t* __restrict__ Ab = A + batch * C::A_B;
  const u16_t* __restrict__ Bb = B + batch * C::B_B;

  // The first half of the workgroup stages A, the second half B (whole wavefronts each).
  const bool loads_a = tid < HALF;
  const int lt = loads_a ? tid : tid - HALF;
  TileLoader<BM, BK, HALF, C::A_KC, C::M, C::K, C::A_M, C::A_K> la;
  TileLoader<BN, BK, HALF, C::B_KC, C::N, C::K, C::B_N, C::B_K> lb;

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x16{};

  if (loads_a) {
    la.load(Ab, m0, 0, lt);
    la.template store<LDK>(lds, lt);
  } else {
    lb.load(Bb, n0, 0, lt);
    lb.template store<LDK>(lds + BM * LDK, lt);
  }
  __syncthreads();

  const int frag_row = lane & 31, frag_k = (lane >> 5) * 8;
  for (long kt = 0; kt < KTILES; ++kt) {
    const bool more = kt + 1 < KTILES;
    if (more) {
      if (loads_a) la.load(Ab, m0, (kt + 1) * BK, lt);
      else lb.load(Bb, n0, (kt + 1) * BK, lt);
    }
    const u16_t* __restrict__ sa = lds + (kt & 1) * STAGE + (wm * WTM + frag_row) * LDK + frag_k;
    const u16_t* __restrict__ sb = lds + (kt & 1) * STAGE + BM * LDK + (wn * WTN + frag_row) * LDK + frag_k;
#pragma unroll
    for (int s = 0; s < BK / 16; ++s) {
      u32x4 a[TM], b[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) a[i] = *(const u32x4*)(sa + i * 32 * LDK + s * 16);
#pragma unroll
      for (int j = 0; j < TN; ++j) b[j] = *(const u32x4*)(sb + j * 32 * LDK + s * 16);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma32x32x16<C::DT>(a[i], b[j], acc[i][j]);
    }
    if (more) {
      u16_t* dst = lds + ((kt + 1) & 1) * STAGE;
      if (loads_a) la.template store<LDK>(dst, lt);
      else lb.template store<LDK>(dst + BM * LDK, lt);
    }
    __syncthreads();
  }

  // Accumulator layout of a 32x32 MFMA: lane l holds column l % 32, rows 8g + 4(l / 32) + j in
  // register 4g + j.
  const long col_base = n0 + wn * WTN + (lane & 31);
  const long row_base = m0 + wm * WTM + (lane >> 5) * 4;
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const long m = row_base + i * 32 + g * 8 + r, n = col_base + j * 32;
          if ((C::M % BM == 0 || m < C::M) && (C::N % BN == 0 || n < C::N)) epi(batch, m, n, acc[i][j][g * 4 + r]);
        }
}

}  // namespace gemm
}  // namespace accy
