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
// M/N at 8 consecutive k) and transposed in registers before the LDS write. Neighbouring lanes take
// neighbouring k-groups of one row group, so the 8 lanes of one LDS store cycle write 8 different
// 16-byte columns of the padded rows (distinct banks) while each global load instruction still covers
// whole 128-byte lines (8 lanes x 16 bytes of one k row). Blocks are renumbered so
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

// Dispatch order round-robins workgroups over the 8 XCDs: the index of workgroup `bid` when each
// XCD instead takes a contiguous range of the TOTAL indices.
template <long TOTAL>
__device__ __forceinline__ long xcd_contiguous(long bid) {
  if constexpr (TOTAL % 8 == 0) bid = (bid % 8) * (TOTAL / 8) + bid / 8;
  return bid;
}

// Tile of index `bid` when the tiles are walked in groups of GROUP_M tile rows.
template <long TILES_M, long TILES_N, int GROUP_M>
__device__ __forceinline__ void tile_in_groups(long bid, long& tm, long& tn) {
  const long per_group = (long)GROUP_M * TILES_N;
  const long group = bid / per_group;
  const long first_m = group * GROUP_M;
  const long gsize = (TILES_M - first_m) < GROUP_M ? (TILES_M - first_m) : GROUP_M;
  tm = first_m + (bid % per_group) % gsize;
  tn = (bid % per_group) / gsize;
}

// Tile numbering: each XCD works on a contiguous range of tiles, walked in groups of GROUP_M rows.
template <long TILES_M, long TILES_N, int GROUP_M>
__device__ __forceinline__ void tile_of(long bid, long& tm, long& tn) {
  tile_in_groups<TILES_M, TILES_N, GROUP_M>(xcd_contiguous<TILES_M * TILES_N>(bid), tm, tn);
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
      (void)RG;
#pragma unroll
      for (int b = 0; b < PER_THREAD / 8; ++b) {
        const int bidx = t + b * THREADS;
        const int kg = bidx % (BK / 8), rg = bidx / (BK / 8);
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
      (void)RG;
#pragma unroll
      for (int b = 0; b < PER_THREAD / 8; ++b) {
        const int bidx = t + b * THREADS;
        const int kg = bidx % (BK / 8), rg = bidx / (BK / 8);
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

// ---------------------------------------------------------------------------------------------
// Direct-to-LDS pipeline (tiles that divide the problem exactly).
//
// Each K step (BK = 32) stages a BM x 32 tile of A and a 32 x BN tile of B straight from global
// memory into LDS with global_load_lds_dwordx4 (lane l of an instruction writes bytes [16 l, 16 l + 16)
// after the wave's LDS base), four stages deep in four distinct LDS arrays, so that 3 K steps of loads
// are in flight under the MFMAs. Each wave waits only for its own loads of the step it consumes
// (s_waitcnt vmcnt), then one s_barrier (no memory fence) publishes every wave's part.
//
// LDS layouts. The gfx950 LDS has 64 banks of 4 bytes: a ds_read_b128 is served 16 lanes (256 bytes)
// per clock and a 64-bit read 32 lanes per clock, so a read is conflict-free when each such lane group
// covers 256 distinct bytes modulo 256 (measured with SQ_LDS_BANK_CONFLICT: groups that only cover 128
// distinct bytes take twice the cycles).
//  * K-contiguous operand (rows = M or N, 64 bytes of K per row): 256-byte lines of four rows; the
//    16-byte chunk at position p of line L holds logical slot p ^ (L & 3) (slot = 4 (row & 3) + chunk).
//    A fragment's 16-lane group reads one chunk of 16 consecutive rows: 4 lines x 4 rows, 16 distinct
//    positions. Fragments: ds_read_b128.
//  * M/N-contiguous operand (rows = K, BN x 2 bytes per row): the 32-byte unit at position p of row k
//    holds logical unit p ^ tr_swizzle(k), tr_swizzle(k) = 2 (k & 3). A fragment's 32-lane half reads
//    two adjacent units (u, u ^ 1) of four consecutive rows: eight distinct units modulo 256 bytes.
//    Fragments: ds_read_b64_tr_b16, which hands lane i of each
//    16-lane group element (i mod 4) of the 8 bytes addressed by lane 4t + i / 4 as its element t;
//    pointing lane j of the group at row k0 + j / 4, columns n0 + 4 (j mod 4) .. + 3 gives lane i the
//    4 values B[k0 .. k0 + 3][n0 + i], the MFMA B-operand layout (and likewise for A).
// ---------------------------------------------------------------------------------------------

#define ACCY_LDS __attribute__((address_space(3)))
typedef short i16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void dma16(const void* g, ACCY_LDS void* l) { __builtin_amdgcn_global_load_lds(g, l, 16, 0, 0); }

// Unit swizzle of an M/N-contiguous (transposed-read) tile row k: see the layouts above.
__device__ __forceinline__ int tr_swizzle(int k) { return 2 * (k & 3); }

template <int N> __device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Waits for this wave's LDS reads, then meets the other waves. The empty asm statements keep the
// optimiser from moving LDS accesses across the barrier (s_barrier alone is no memory fence, and a
// real fence would also wait for every outstanding global load).
__device__ __forceinline__ void lds_reads_done_barrier() {
  __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4) | (0 << 8));  // lgkmcnt(0)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// out[e] = the 16-bit LDS word at byte address addr[e], zero-extended: 16 reads and one wait in a
// single assembly statement, so no result is visible to the compiler before its data has arrived
// (split into one statement per read and one for the wait, a register copy or spill placed between
// them would read the register early). Written as assembly because the lookups address LDS as a
// whole: indexing the stage arrays makes the compiler branch on which array an index falls in, and
// plain loads through an LDS pointer are each waited for before the next, since the epilogue's
// stores go through generic pointers the compiler cannot separate from LDS.
__device__ __forceinline__ void lds_gather16(const u32_t (&addr)[16], u32_t (&out)[16]) {
  asm volatile(
      "ds_read_u16 %0, %16\n ds_read_u16 %1, %17\n ds_read_u16 %2, %18\n ds_read_u16 %3, %19\n"
      "ds_read_u16 %4, %20\n ds_read_u16 %5, %21\n ds_read_u16 %6, %22\n ds_read_u16 %7, %23\n"
      "ds_read_u16 %8, %24\n ds_read_u16 %9, %25\n ds_read_u16 %10, %26\n ds_read_u16 %11, %27\n"
      "ds_read_u16 %12, %28\n ds_read_u16 %13, %29\n ds_read_u16 %14, %30\n ds_read_u16 %15, %31\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(out[0]), "=&v"(out[1]), "=&v"(out[2]), "=&v"(out[3]), "=&v"(out[4]), "=&v"(out[5]),
        "=&v"(out[6]), "=&v"(out[7]), "=&v"(out[8]), "=&v"(out[9]), "=&v"(out[10]), "=&v"(out[11]),
        "=&v"(out[12]), "=&v"(out[13]), "=&v"(out[14]), "=&v"(out[15])
      : "v"(addr[0]), "v"(addr[1]), "v"(addr[2]), "v"(addr[3]), "v"(addr[4]), "v"(addr[5]), "v"(addr[6]),
        "v"(addr[7]), "v"(addr[8]), "v"(addr[9]), "v"(addr[10]), "v"(addr[11]), "v"(addr[12]), "v"(addr[13]),
        "v"(addr[14]), "v"(addr[15])
      : "memory");
}

// Element offsets of an operand tile: O::row(i) of row (M or N) index i, O::k(i) of contraction
// index i. The configuration struct supplies them as a_m / a_k / b_n / b_k (and a_b / b_b for the
// batch index): plain products for strided operands, or sums over several axes when a named group
// does not collapse to one stride. Within one tile the contiguous group is affine (the planner
// checks that its innermost axis has stride 1 and a multiple of the tile as extent).
template <class C> struct AOff {
  static __device__ __forceinline__ long row(long i) { return C::a_m(i); }
  static __device__ __forceinline__ long k(long i) { return C::a_k(i); }
};
template <class C> struct BOff {
  static __device__ __forceinline__ long row(long i) { return C::b_n(i); }
  static __device__ __forceinline__ long k(long i) { return C::b_k(i); }
};

// Offset functions of single-stride operands, for configurations written by hand.
template <long AB, long AM, long AK, long BB, long BK, long BN>
struct Strided {
  static __device__ __forceinline__ long a_b(long i) { return i * AB; }
  static __device__ __forceinline__ long a_m(long i) { return i * AM; }
  static __device__ __forceinline__ long a_k(long i) { return i * AK; }
  static __device__ __forceinline__ long b_b(long i) { return i * BB; }
  static __device__ __forceinline__ long b_k(long i) { return i * BK; }
  static __device__ __forceinline__ long b_n(long i) { return i * BN; }
};

// Issues load instruction i of this wave's share of one operand tile (ROWS * 64 bytes, 1 KiB per
// wave instruction, INSTRS / 4 instructions per wave). KC: rows of 32 k (64 bytes); else rows of k.
// RMAX is the operand's row extent (M or N). When it is not a multiple of the tile the last tile
// reaches past it: a row past the end reads the last row (KC), a 16-byte chunk past the end of a k
// row reads the last chunk (RMAX a multiple of 8), so every load stays inside the operand; those
// rows and columns only feed outputs that the epilogue does not store.
template <int ROWS, bool KC, class O, long RMAX>
__device__ __forceinline__ void dma_part(const u16_t* __restrict__ base, long r0, long k0, u16_t* lds, int wave,
                                         int lane, int i) {
  constexpr int INSTRS = ROWS * 64 / 1024;
  static_assert(INSTRS % 4 == 0, "four waves share the tile");
  constexpr bool RAGGED = RMAX % ROWS != 0;
  const int gi = wave * (INSTRS / 4) + i;
  const u16_t* src;
  if constexpr (KC) {
    // instruction gi fills lines 4 gi .. 4 gi + 3: lane l writes position l & 15 of line 4 gi + l / 16
    const int q = (lane & 15) ^ (lane >> 4);  // logical slot of this lane's physical chunk
    const int row = 16 * gi + 4 * (lane >> 4) + (q >> 2);
    long r = r0 + row;
    if constexpr (RAGGED) r = r < RMAX ? r : RMAX - 1;
    src = base + O::row(r) + O::k(k0) + 8 * (q & 3);
  } else {
    static_assert(!RAGGED || RMAX % 8 == 0, "whole 16-byte chunks");
    constexpr int ROWB = ROWS * 2;    // bytes per k row
    constexpr int LPR = ROWB / 16;    // lanes per k row
    constexpr int RPI = 1024 / ROWB;  // k rows per instruction
    const int row = RPI * gi + lane / LPR;
    const int p = lane % LPR;
    const int u = (p >> 1) ^ tr_swizzle(row);
    if constexpr (RAGGED) {
      long col = r0 + 16 * u + 8 * (p & 1);
      col = col <= RMAX - 8 ? col : RMAX - 8;
      src = base + O::k(k0 + row) + O::row(col);
    } else {
      // whole tiles lie inside one contiguous run of the row group: affine there
      src = base + O::k(k0 + row) + O::row(r0) + 16 * u + 8 * (p & 1);
    }
  }
  dma16(src, (ACCY_LDS void*)(lds + gi * 512));
}

template <int ROWS, bool KC, class O, long RMAX>
__device__ __forceinline__ void dma_tile(const u16_t* __restrict__ base, long r0, long k0, u16_t* lds, int wave, int lane) {
#pragma unroll
  for (int i = 0; i < ROWS * 64 / 1024 / 4; ++i) dma_part<ROWS, KC, O, RMAX>(base, r0, k0, lds, wave, lane, i);
}

// Fragment of 32 rows (M or N) x 16 k for one MFMA, read from a stage.
template <int ROWS, bool KC>
__device__ __forceinline__ u32x4 frag(const u16_t* lds, int row0, int s, int lane) {
  if constexpr (KC) {
    const int r = row0 + (lane & 31), c = 2 * s + (lane >> 5);
    const int line = r >> 2, slot = ((r & 3) << 2) | c;
    return *(const u32x4*)(lds + line * 128 + ((slot ^ (line & 3)) << 3));
  } else {
    constexpr int ROWE = ROWS;  // elements per k row
    const int g = lane >> 4, i = lane & 15;
    const int n0 = row0 + ((g & 1) << 4);
    u32x4 out;
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      const int k = 16 * s + 8 * (g >> 1) + 4 * rr + (i >> 2);
      const int unit = (n0 >> 4) ^ tr_swizzle(k);
      const u16_t* p = lds + k * ROWE + unit * 16 + 4 * (i & 3);
      const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((ACCY_LDS i16x4*)p);
      const u32_t lo = (u32_t)(u16_t)v[0] | ((u32_t)(u16_t)v[1] << 16);
      const u32_t hi = (u32_t)(u16_t)v[2] | ((u32_t)(u16_t)v[3] << 16);
      out[2 * rr] = lo;
      out[2 * rr + 1] = hi;
    }
    return out;
  }
}

// The fragments of one 16-deep sub-step for this wave's (BM / 2) x (BN / 2) sub-tile: TM A
// fragments, then TN B fragments (fragment q of the set is loaded by load_one(q)).
template <class C>
struct Frags {
  static constexpr int TM = C::BM / 64, TN = C::BN / 64, COUNT = TM + TN;
  u32x4 a[TM], b[TN];
  __device__ __forceinline__ void load_one(int q, const u16_t* as, const u16_t* bs, int s, int lane, int wm, int wn) {
    if (q < TM)
      a[q] = frag<C::BM, C::A_KC>(as, wm * (C::BM / 2) + q * 32, s, lane);
    else
      b[q - TM] = frag<C::BN, C::B_KC>(bs, wn * (C::BN / 2) + (q - TM) * 32, s, lane);
  }
  template <class Acc>
  __device__ __forceinline__ void mma_one(int t, Acc& acc) const {
    acc[t / TN][t % TN] = mfma32x32x16<C::DT>(a[t / TN], b[t % TN], acc[t / TN][t % TN]);
  }
};

// One K step on stage STAGE of S = C::STAGES. On entry f0 holds this step's first sub-step fragments
// and every wave has finished reading the previous stage (NEXT). The first half runs the MFMAs of f0
// with the loads of tile kt + S - 1 into NEXT and the reads of this stage's second sub-step (f1)
// slotted between them; then the wave waits for its own loads of tile kt + 1 (WAIT = the load
// instructions it may leave in flight) and its LDS reads and meets the other waves at the step's
// single barrier (after which tile kt + 1 is complete and nobody reads this stage any more); the
// second half runs the MFMAs of f1 with the reads of tile kt + 1's first sub-step (the next f0)
// between them. The explicit interleave keeps at most one sub-step of LDS reads in flight, so the
// compiler's lgkmcnt waits stay exact instead of draining the counter.
template <class C, int STAGE, int WAIT, bool ISSUE, bool HAS_NEXT>
struct DmaStep {
  static constexpr int S = C::STAGES, NEXT = (STAGE + S - 1) % S;
  template <class Acc>
  __device__ __forceinline__ static void run(const u16_t* __restrict__ Ab, const u16_t* __restrict__ Bb, long m0,
                                             long n0, long kt, u16_t* const (&as)[C::STAGES],
                                             u16_t* const (&bs)[C::STAGES], Frags<C>& f0, Acc& acc, int wave, int lane,
                                             int wm, int wn) {
    constexpr int NM = Frags<C>::TM * Frags<C>::TN, NF = Frags<C>::COUNT;
    constexpr int DA = C::BM * 64 / 1024 / 4, DB = C::BN * 64 / 1024 / 4;
    constexpr int ND = ISSUE ? DA + DB : 0, NI = NF + ND;
    Frags<C> f1;
#pragma unroll
    for (int t = 0; t < NM; ++t) {
      f0.mma_one(t, acc);
      __builtin_amdgcn_sched_barrier(0);
      // Items: the f1 fragment reads first (they must land before the barrier), then the tile loads.
#pragma unroll
      for (int k = t * NI / NM; k < (t + 1) * NI / NM; ++k) {
        if (k < NF) {
          f1.load_one(k, as[STAGE], bs[STAGE], 1, lane, wm, wn);
        } else if (k - NF < DA) {
          dma_part<C::BM, C::A_KC, AOff<C>, C::M>(Ab, m0, (kt + S - 1) * 32, as[NEXT], wave, lane, k - NF);
        } else {
          dma_part<C::BN, C::B_KC, BOff<C>, C::N>(Bb, n0, (kt + S - 1) * 32, bs[NEXT], wave, lane, k - NF - DA);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (HAS_NEXT) {
      wait_vmcnt<WAIT>();
      lds_reads_done_barrier();
    }
#pragma unroll
    for (int t = 0; t < NM; ++t) {
      f1.mma_one(t, acc);
      __builtin_amdgcn_sched_barrier(0);
      // One next-f0 fragment read per MFMA from the start (NF <= NM), so the last one lands well
      // before the next step's first MFMA.
      if constexpr (HAS_NEXT) {
        static_assert(NF <= NM, "fragment reads fit one per MFMA");
        if (t < NF) f0.load_one(t, as[(STAGE + 1) % S], bs[(STAGE + 1) % S], 0, lane, wm, wn);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
};

// Steps after the last full group of S: R more steps that issue a load (the last of them issues tile
// KT - 1), then S - 1 steps that only drain the pipeline (step j of those may leave S - 2 - j tiles in
// flight; the last has no next tile). Step I of this tail runs on stage I % S.
template <class C, int I, int R, int PER>
struct DmaTail {
  static constexpr int S = C::STAGES;
  template <class Acc>
  __device__ __forceinline__ static void run(const u16_t* __restrict__ Ab, const u16_t* __restrict__ Bb, long m0,
                                             long n0, long kt, u16_t* const (&as)[S], u16_t* const (&bs)[S],
                                             Frags<C>& f0, Acc& acc, int wave, int lane, int wm, int wn) {
    constexpr bool ISSUE = I < R;
    constexpr int J = ISSUE ? 0 : I - R + 1;  // 1 .. S - 1 for the draining steps
    constexpr int LEFT = S - 2 - J;
    constexpr int WAIT = LEFT > 0 ? LEFT * PER : 0;
    constexpr bool HAS_NEXT = J < S - 1;
    DmaStep<C, I % S, WAIT, ISSUE, HAS_NEXT>::run(Ab, Bb, m0, n0, kt, as, bs, f0, acc, wave, lane, wm, wn);
    if constexpr (HAS_NEXT) DmaTail<C, I + 1, R, PER>::run(Ab, Bb, m0, n0, kt + 1, as, bs, f0, acc, wave, lane, wm, wn);
  }
};

// One full group of S steps (stages 0 .. S - 1), each issuing a load.
template <class C, int I, int PER>
struct DmaGroup {
  template <class Acc>
  __device__ __forceinline__ static void run(const u16_t* __restrict__ Ab, const u16_t* __restrict__ Bb, long m0,
                                             long n0, long kt, u16_t* const (&as)[C::STAGES],
                                             u16_t* const (&bs)[C::STAGES], Frags<C>& f0, Acc& acc, int wave, int lane,
                                             int wm, int wn) {
    DmaStep<C, I, (C::STAGES - 2) * PER, true, true>::run(Ab, Bb, m0, n0, kt + I, as, bs, f0, acc, wave, lane, wm, wn);
    if constexpr (I + 1 < C::STAGES) DmaGroup<C, I + 1, PER>::run(Ab, Bb, m0, n0, kt, as, bs, f0, acc, wave, lane, wm, wn);
  }
};

// Epilogue functors with a lookup table declare `static constexpr bool kTable = true`, a member
// table() (65536 16-bit results in global memory), index(v) (the bit pattern of the rounded
// contraction value) and put(batch, m, n, bits); others are called as epi(batch, m, n, v).
template <class E, class = void> struct HasTable { static constexpr bool value = false; };
template <class E> struct HasTable<E, decltype((void)E::kTable)> { static constexpr bool value = E::kTable; };
// An epilogue with kStaged set reads other operands at the output's own row-major index and depends
// on the contraction value only through its rounding to the 16-bit element type (every 16-bit
// contraction result is rounded before any use). Its tile goes through LDS (staged_epilogue).
template <class E, class = void> struct IsStaged { static constexpr bool value = false; };
template <class E> struct IsStaged<E, decltype((void)E::kStaged)> { static constexpr bool value = E::kStaged; };

// The 16-bit result of one output of a contraction of element type DT (0 bf16: the high half,
// as every bf16 result; 1 f16: nearest even) and its value as f32.
template <int DT> __device__ __forceinline__ u16_t result_bits(float v) { return DT == 0 ? f32_to_bf16(v) : f32_to_f16(v); }
template <int DT> __device__ __forceinline__ float result_value(u16_t h) { return DT == 0 ? bf16_to_f32(h) : f16_to_f32(h); }

// Epilogue of a 256 x 256 tile through LDS: the rounded 16-bit results are written to the eight
// 16 KiB stage arrays (32 tile rows each, rows of 512 bytes whose 16-byte chunk c sits at
// c ^ (row & 7), so that the two 32-lane halves of a write, four rows apart, and the 16-lane groups
// of a row read hit distinct banks), then every thread takes 16-byte chunks of 8 consecutive
// outputs of one row and calls the epilogue for them in column order. The operands the epilogue
// reads and the output it writes are then accessed in whole row segments (512 bytes per 32 lanes)
// instead of 2-byte pieces of 32 rows. acc[i][j][4 g + r] is output (row_base + 32 i + 8 g + r,
// col_base + 32 j) of the wave; lo holds tile rows 0-127 (wm = 0), hi rows 128-255.
template <class C, class Epi, int TM, int TN>
__device__ __forceinline__ void staged_epilogue(const f32x16 (&acc)[TM][TN], u16_t* const (&lo)[4], u16_t* const (&hi)[4],
                                                const Epi& epi, long batch, long m0, long n0, int tid, int lane, int wm,
                                                int wn) {
  static_assert(TM == 4 && TN == 4, "256 x 256 tiles of four waves");
  wait_vmcnt<0>();
  lds_reads_done_barrier();
  const int hr = (lane >> 5) * 4, col = wn * 128 + (lane & 31);
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    u16_t* const arr = wm ? hi[i] : lo[i];
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int rr = g * 8 + hr + r, c = col + j * 32;
          arr[rr * 256 + (((c >> 3) ^ (rr & 7)) << 3) + (c & 7)] = result_bits<C::DT>(acc[i][j][g * 4 + r]);
        }
  }
  lds_reads_done_barrier();
  const int chunk = tid & 31;
#pragma unroll
  for (int it = 0; it < 32; ++it) {
    const int row = it * 8 + (tid >> 5), rr = row & 31;
    const u16_t* arr = it < 16 ? lo[it / 4] : hi[(it - 16) / 4];
    const u32x4 w = *(const u32x4*)(arr + rr * 256 + ((chunk ^ (rr & 7)) << 3));
#pragma unroll
    for (int e = 0; e < 8; ++e)
      epi(batch, m0 + row, n0 + chunk * 8 + e, result_value<C::DT>((u16_t)(w[e >> 1] >> (16 * (e & 1)))));
  }
}

// Requires K % 32 == 0 with at least STAGES K steps and 16-byte aligned rows (M or N not a multiple
// of the tile: see dma_part);
// 256 threads (2 x 2 waves). LDS: STAGES x (BM + BN) x 64 bytes (STAGES = 4 with a 256 x 256 tile:
// 128 KiB, one workgroup per CU; 3 with 256 x 128: 72 KiB, two per CU when the kernel is compiled for
// two waves per SIMD, so that one workgroup's epilogue runs beside the other's matrix work).
template <class C, class Epi>
__device__ __forceinline__ void mma16_dma_tile(const u16_t* __restrict__ A, const u16_t* __restrict__ B, const Epi& epi,
                                               long tm, long tn) {
  constexpr int BM = C::BM, BN = C::BN, S = C::STAGES;
  constexpr int TM = BM / 64, TN = BN / 64;
  constexpr long TILES_M = (C::M + BM - 1) / BM, TILES_N = (C::N + BN - 1) / BN, KT = C::K / 32;
  static_assert(C::K % 32 == 0, "whole K steps");
  static_assert(S >= 2 && S <= 4 && KT >= S, "two to four stages, at least one K step per stage");
  constexpr int PER = (BM * 64 / 1024) / 4 + (BN * 64 / 1024) / 4;  // DMA instructions per wave per step
  static_assert((S - 2) * PER < 64, "vmcnt range");
  // One LDS array per stage: with distinct objects the compiler can tell that the fragment reads of
  // one stage do not overlap the direct-to-LDS writes still in flight into another (stages of one
  // array would make it drain every load, s_waitcnt vmcnt(0), before each read). Stages past S get
  // one element.
  constexpr int A_ST = BM * 32, B_ST = BN * 32;
  __shared__ __attribute__((aligned(1024))) u16_t a0[A_ST], a1[A_ST], a2[S > 2 ? A_ST : 1], a3[S > 3 ? A_ST : 1];
  __shared__ __attribute__((aligned(1024))) u16_t b0[B_ST], b1[B_ST], b2[S > 2 ? B_ST : 1], b3[S > 3 ? B_ST : 1];
  u16_t* const a_all[4] = {a0, a1, a2, a3};
  u16_t* const b_all[4] = {b0, b1, b2, b3};
  u16_t* const (&asc)[S] = *reinterpret_cast<u16_t* const(*)[S]>(&a_all);
  u16_t* const (&bsc)[S] = *reinterpret_cast<u16_t* const(*)[S]>(&b_all);
  u16_t* const (&as)[S] = asc;
  u16_t* const (&bs)[S] = bsc;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  (void)TILES_M;
  (void)TILES_N;
  const long m0 = tm * BM, n0 = tn * BN, batch = blockIdx.y;
  const u16_t* __restrict__ Ab = A + C::a_b(batch);
  const u16_t* __restrict__ Bb = B + C::b_b(batch);

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x16{};

#pragma unroll
  for (int s = 0; s < S - 1; ++s) {
    dma_tile<BM, C::A_KC, AOff<C>, C::M>(Ab, m0, s * 32, as[s], wave, lane);
    dma_tile<BN, C::B_KC, BOff<C>, C::N>(Bb, n0, s * 32, bs[s], wave, lane);
  }
  // Tile 0 complete everywhere (tiles 1 .. S - 2 may still be in flight), then its first sub-step.
  Frags<C> f0;
  wait_vmcnt<(S - 2) * PER>();
  lds_reads_done_barrier();
#pragma unroll
  for (int q = 0; q < Frags<C>::COUNT; ++q) f0.load_one(q, as[0], bs[0], 0, lane, wm, wn);
  // Step kt issues tile kt + S - 1 and then waits for tile kt + 1. Steps 0 .. KT - S issue a load:
  // G full groups of S, then the tail.
  constexpr long ISSUING = KT - S + 1, G = ISSUING / S;
  constexpr int R = (int)(ISSUING % S);
  long kt = 0;
  for (long g = 0; g < G; ++g, kt += S) DmaGroup<C, 0, PER>::run(Ab, Bb, m0, n0, kt, asc, bsc, f0, acc, wave, lane, wm, wn);
  DmaTail<C, 0, R, PER>::run(Ab, Bb, m0, n0, kt, asc, bsc, f0, acc, wave, lane, wm, wn);

  const long col_base = n0 + wn * (BN / 2) + (lane & 31);
  const long row_base = m0 + wm * (BM / 2) + (lane >> 5) * 4;
  auto each = [&](auto f) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const long m = row_base + i * 32 + g * 8 + r, n = col_base + j * 32;
            if ((C::M % BM == 0 || m < C::M) && (C::N % BN == 0 || n < C::N)) f(m, n, acc[i][j][g * 4 + r]);
          }
  };
  if constexpr (IsStaged<Epi>::value && !HasTable<Epi>::value && S == 4 && BM == 256 && BN == 256 &&
                C::M % BM == 0 && C::N % BN == 0) {
    u16_t* const lo[4] = {a0, a1, a2, a3};
    u16_t* const hi[4] = {b0, b1, b2, b3};
    staged_epilogue<C>(acc, lo, hi, epi, batch, m0, n0, tid, lane, wm, wn);
  } else if constexpr (HasTable<Epi>::value) {
    // A table epilogue (65536 16-bit results indexed by the rounded contraction value): with four
    // stages of 256 x 256 tiles the eight 16 KiB stage arrays are the kernel's whole 128 KiB of LDS,
    // i.e. they tile LDS addresses [0, 128 KiB) in some order. After the last K step each array
    // receives the table entries of its own addresses, and the lookups read LDS address 2 x index,
    // 16 per wait (lds_gather16). Otherwise the table is read from global memory (L2).
    const u16_t* __restrict__ table = epi.table();
    bool in_lds = false;
    auto at = [](const u16_t* p) { return (u32_t)(unsigned long)(const ACCY_LDS u16_t*)p; };
    if constexpr (S == 4 && A_ST == 8192 && B_ST == 8192) {
      constexpr u32_t LAST = 131072 - 16384;
      in_lds = at(a0) <= LAST && at(a1) <= LAST && at(a2) <= LAST && at(a3) <= LAST && at(b0) <= LAST &&
               at(b1) <= LAST && at(b2) <= LAST && at(b3) <= LAST;
    }
    if (in_lds) {
      lds_reads_done_barrier();
      // each wave fills two arrays (16 KiB each, 16 instructions of 1 KiB)
      auto fill = [&](u16_t* dst) {
        const u16_t* const src = table + at(dst) / 2;
#pragma unroll
        for (int i = 0; i < 16; ++i) dma16(src + i * 512 + lane * 8, (ACCY_LDS void*)(dst + i * 512));
      };
      switch (__builtin_amdgcn_readfirstlane(wave)) {
        case 0: fill(a0); fill(a1); break;
        case 1: fill(a2); fill(a3); break;
        case 2: fill(b0); fill(b1); break;
        default: fill(b2); fill(b3); break;
      }
      wait_vmcnt<0>();
      lds_reads_done_barrier();
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          u32_t addr[16], bits[16];
#pragma unroll
          for (int e = 0; e < 16; ++e) addr[e] = 2u * (u32_t)Epi::index(acc[i][j][e]);
          lds_gather16(addr, bits);
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const long m = row_base + i * 32 + (e >> 2) * 8 + (e & 3), n = col_base + j * 32;
            if ((C::M % BM == 0 || m < C::M) && (C::N % BN == 0 || n < C::N)) epi.put(batch, m, n, (u16_t)bits[e]);
          }
        }
    } else {
      each([&](long m, long n, float v) { epi.put(batch, m, n, table[Epi::index(v)]); });
    }
  } else {
    each([&](long m, long n, float v) { epi(batch, m, n, v); });
  }
}

// Tile rows per group of the tile walk (C::GROUP_M when the configuration sets it, else 8). With 32
// workgroups per XCD at a time, 8 gives each XCD 8 A row panels x 4 B column panels and 4 gives 4 x 8:
// the same panel count, but with 4 each A panel of an 8-panel-wide B is read by one XCD only, which
// the planner prefers when A is the larger operand (its repeated reads would come from HBM).
template <class C, class = void> struct GroupM { static constexpr int value = 8; };
template <class C> struct GroupM<C, decltype((void)C::GROUP_M)> { static constexpr int value = C::GROUP_M; };

template <class C, class Epi>
__device__ __forceinline__ void mma16_dma(const u16_t* __restrict__ A, const u16_t* __restrict__ B, const Epi& epi) {
  constexpr long TILES_M = (C::M + C::BM - 1) / C::BM, TILES_N = (C::N + C::BN - 1) / C::BN;
  long tm, tn;
  tile_of<TILES_M, TILES_N, GroupM<C>::value>((long)blockIdx.x, tm, tn);
  mma16_dma_tile<C>(A, B, epi, tm, tn);
}

// G contractions that share the A operand, every extent and both layouts, each with its own B
// operand and output, in one launch of G x tiles workgroups (the projections of one activation:
// one fill and drain of the machine instead of G). Consecutive indices of an XCD's range take the G
// contractions of one tile, so the workgroups that read an A row panel run on the same XCD (its L2)
// at about the same time. The epilogue functor gives contraction g's output (epi.out(g), chosen once
// per workgroup) and stores into it: epi(out, b, m, n, v).
template <class C, int G, class Epi>
__device__ __forceinline__ void mma16_dma_group(const u16_t* __restrict__ A, const u16_t* const (&B)[G], const Epi& epi) {
  constexpr long TILES_M = (C::M + C::BM - 1) / C::BM, TILES_N = (C::N + C::BN - 1) / C::BN;
  const long bid = xcd_contiguous<G * TILES_M * TILES_N>((long)blockIdx.x);
  const int g = (int)(bid % G);
  long tm, tn;
  tile_in_groups<TILES_M, TILES_N, GroupM<C>::value>(bid / G, tm, tn);
  const u16_t* __restrict__ Bg = B[0];
#pragma unroll
  for (int i = 1; i < G; ++i)
    if (g == i) Bg = B[i];
  u16_t* __restrict__ const out = epi.out(g);
  mma16_dma_tile<C>(A, Bg, [&](long b, long m, long n, float v) { epi(out, b, m, n, v); }, tm, tn);
}

// ---------------------------------------------------------------------------------------------
// f32 contraction on v_mfma_f32_32x32x2_f32 (exact f32 products, f32 accumulation).
//
// 256 x 256 block tile, 4 wavefronts of 128 x 128 (4 x 4 accumulators of 32 x 32), K steps of 32
// staged straight from global memory into LDS (global_load_lds_dwordx4), two stages: one K step
// is 256 MFMAs per wave, long enough to cover the next step's loads.
//
// Within a K step the MFMA sub-step s (0..15) takes k = 16 h + s from lane half h = lane / 32 in
// both operands (any k order is valid when A and B agree), so a lane's A values for 4 sub-steps
// are 4 consecutive k of one row: one ds_read_b128. The wave's 128 output columns are assigned
// col = 4 (lane % 32) + j to accumulator tile j, so one ds_read_b128 of a B row serves the four
// column tiles, and the epilogue writes 4 consecutive columns per lane.
//
// LDS layouts: A rows of 32 f32 (128 bytes), 16-byte chunk c of row r at chunk c ^ ((r / 2) % 8)
// (16 consecutive rows of one read hit 16 distinct bank groups); B rows of 256 f32, unswizzled
// (32 consecutive lanes read 512 contiguous bytes).
//
// C supplies M, N, K (multiples of 256, 256, 32) and the offset functions a_b, a_m, a_k (A is
// K-contiguous within each 32-wide k tile), b_b, b_k, b_n (B is N-contiguous within each 256-wide
// n tile); the epilogue functor receives (batch, m, n, value).
// ---------------------------------------------------------------------------------------------

typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x16 mfma32x32x2f32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

template <class C>
__device__ __forceinline__ void f32_issue(const float* __restrict__ Ab, const float* __restrict__ Bb, long m0, long n0,
                                          long k0, float* as, float* bs, int wave, int lane) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int gi = wave * 8 + i;  // 1 KiB per instruction: 8 A rows, or 1 B row
    const int row = 8 * gi + (lane >> 3);
    const int c = (lane & 7) ^ ((row >> 1) & 7);
    // Past the end of M (N) the last tile reads the last row (last 4-float chunk): every load stays
    // inside the operand, and those rows and columns only feed outputs that are not stored.
    long r = m0 + row, col = n0 + 4 * lane;
    if constexpr (C::M % 256 != 0) r = r < C::M ? r : C::M - 1;
    if constexpr (C::N % 256 != 0) col = col <= C::N - 4 ? col : C::N - 4;
    dma16(Ab + C::a_m(r) + C::a_k(k0) + 4 * c, (ACCY_LDS void*)(as + gi * 256));
    dma16(Bb + C::b_k(k0 + gi) + C::b_n(col), (ACCY_LDS void*)(bs + gi * 256));
  }
}

template <class C, class Epi>
__device__ __forceinline__ void mma32f(const float* __restrict__ A, const float* __restrict__ B, const Epi& epi) {
  constexpr int BM = 256, BN = 256, BKF = 32;
  constexpr long TILES_M = (C::M + BM - 1) / BM, TILES_N = (C::N + BN - 1) / BN, KT = C::K / BKF;
  static_assert(C::K % BKF == 0 && C::N % 4 == 0, "whole K steps, 16-byte chunks of B rows");
  __shared__ __attribute__((aligned(1024))) float a0[BM * BKF], a1[BM * BKF];
  __shared__ __attribute__((aligned(1024))) float b0[BKF * BN], b1[BKF * BN];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1, h = lane >> 5, l32 = lane & 31;
  long tm, tn;
  tile_of<TILES_M, TILES_N, 8>((long)blockIdx.x, tm, tn);
  const long m0 = tm * BM, n0 = tn * BN, batch = blockIdx.y;
  const float* __restrict__ Ab = A + C::a_b(batch);
  const float* __restrict__ Bb = B + C::b_b(batch);

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};

  auto step = [&](const float* as, const float* bs) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      f32x4 av[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = wm * 128 + i * 32 + l32;
        const int pc = (4 * h + c) ^ ((row >> 1) & 7);
        av[i] = *(const f32x4*)(as + row * BKF + pc * 4);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) bv[u] = *(const f32x4*)(bs + (16 * h + 4 * c + u) * BN + wn * 128 + 4 * l32);
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][j] = mfma32x32x2f32(av[i][u], bv[u][j], acc[i][j]);
    }
  };

  f32_issue<C>(Ab, Bb, m0, n0, 0, a0, b0, wave, lane);
  long kt = 0;
  for (; kt + 2 <= KT; kt += 2) {
    wait_vmcnt<0>();
    lds_reads_done_barrier();
    if (kt + 1 < KT) f32_issue<C>(Ab, Bb, m0, n0, (kt + 1) * BKF, a1, b1, wave, lane);
    step(a0, b0);
    wait_vmcnt<0>();
    lds_reads_done_barrier();
    if (kt + 2 < KT) f32_issue<C>(Ab, Bb, m0, n0, (kt + 2) * BKF, a0, b0, wave, lane);
    step(a1, b1);
  }
  if (kt < KT) {
    wait_vmcnt<0>();
    lds_reads_done_barrier();
    step(a0, b0);
  }
  // The accumulators stay in AGPRs through the K loop. (With an epilogue that computes on the values,
  // the register allocator otherwise gave the loop's per-lane offsets to scratch memory and reloaded
  // them every K step; a plain store takes its data from the AGPRs.)
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) asm volatile("" : "+a"(acc[i][j]));

  const long col_base = n0 + wn * 128 + 4 * l32;
  const long row_base = m0 + wm * 128 + 4 * h;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const long m = row_base + i * 32 + g * 8 + r, n = col_base + j;
          if ((C::M % BM == 0 || m < C::M) && (C::N % BN == 0 || n < C::N)) epi(batch, m, n, acc[i][j][g * 4 + r]);
        }
}

}  // namespace gemm
}  // namespace accy
