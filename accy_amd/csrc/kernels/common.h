// Device helpers shared by every kernel the HIP target generates for gfx950: storage loads and stores
// for each element type, per-operation 16-bit rounding, integer wrap-around arithmetic, and wave64 /
// workgroup reductions. Generated kernels compute 16-bit floats in f32 and round back after every
// operation, and keep multiplies and adds separately rounded, as the reference's arithmetic contract
// requires (src/eval/root.zig:10-16).
#pragma once
#pragma clang fp contract(off)
#ifndef __HIPCC_RTC__
// hiprtc provides the HIP device environment itself; an offline hipcc build (the build-time check of
// these sources) needs the header.
#include <hip/hip_runtime.h>
#endif

typedef signed char i8_t;
typedef short i16_t;
typedef int i32_t;
typedef long long i64_t;
typedef unsigned char u8_t;
typedef unsigned short u16_t;
typedef unsigned int u32_t;
typedef unsigned long long u64_t;

namespace accy {

// ---- 16-bit floats: f16 is IEEE binary16 and rounds to nearest even (Zig @floatCast); bf16 is the
// top half of an f32 and every bf16 result keeps the high 16 bits of its f32 value, the reference's
// Bf16.fromF32 (deps/lib/compiler/gpu/abi/src/dtype.zig:6-9), which its evaluator applies to every
// bf16 operation result (src/eval/evaluator.zig:2242-2244, 2338, 2384-2386, 2860).
__device__ __forceinline__ float f16_to_f32(u16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ u16_t f32_to_f16(float x) { return __builtin_bit_cast(u16_t, (_Float16)x); }
__device__ __forceinline__ float bf16_to_f32(u16_t h) { return __builtin_bit_cast(float, ((u32_t)h) << 16); }
__device__ __forceinline__ u16_t f32_to_bf16(float x) { return (u16_t)(__builtin_bit_cast(u32_t, x) >> 16); }
__device__ __forceinline__ float round_f16(float x) { return (float)(_Float16)x; }
// The f32 value of bf16(x): one v_and_b32 of the low mantissa half.
__device__ __forceinline__ float round_bf16(float x) {
  return __builtin_bit_cast(float, __builtin_bit_cast(u32_t, x) & 0xffff0000u);
}
// Two bf16 results packed into one word, lo in the low half (the compiler makes it one v_perm_b32).
__device__ __forceinline__ u32_t pack_bf16x2(float lo, float hi) {
  return (__builtin_bit_cast(u32_t, lo) >> 16) | (__builtin_bit_cast(u32_t, hi) & 0xffff0000u);
}

// ---- loads and stores in the compute domain (f32 for 16-bit floats) ----
template <typename I> __device__ __forceinline__ float ld_f16(const u16_t* __restrict__ p, I i) { return f16_to_f32(p[i]); }
template <typename I> __device__ __forceinline__ float ld_bf16(const u16_t* __restrict__ p, I i) { return bf16_to_f32(p[i]); }
template <typename I> __device__ __forceinline__ void st_f16(u16_t* __restrict__ p, I i, float v) { p[i] = f32_to_f16(v); }
template <typename I> __device__ __forceinline__ void st_bf16(u16_t* __restrict__ p, I i, float v) { p[i] = f32_to_bf16(v); }
template <typename T, typename I> __device__ __forceinline__ T ld(const T* __restrict__ p, I i) { return p[i]; }
template <typename T, typename I> __device__ __forceinline__ void st(T* __restrict__ p, I i, T v) { p[i] = v; }
template <typename I> __device__ __forceinline__ bool ld_i1(const u8_t* __restrict__ p, I i) { return p[i] != 0; }
// Four consecutive elements read as one vector load (the row kernels load each input's four elements
// of a thread this way at the top of an iteration); alignment capped at the 16 bytes every buffer
// base guarantees.
template <typename T> struct alignas(4 * sizeof(T) < 16 ? 4 * sizeof(T) : 16) Quad { T v[4]; };
// The same four elements with the non-temporal hint, for data that a kernel reads exactly once (each
// element by one workgroup, in one pass): the lines stream through the caches without displacing
// lines that are reused, and a streaming read of HBM sustains about 7.0 TB/s instead of about 6.3.
typedef u32_t u32x2_nt __attribute__((ext_vector_type(2)));
typedef u32_t u32x4_nt __attribute__((ext_vector_type(4)));
struct alignas(16) U32x8_nt { u32x4_nt lo, hi; };
template <typename T> __device__ __forceinline__ Quad<T> ld_quad_stream(const T* __restrict__ p) {
  constexpr int BYTES = 4 * (int)sizeof(T);
  if constexpr (BYTES == 4) {
    return __builtin_bit_cast(Quad<T>, __builtin_nontemporal_load((const u32_t*)p));
  } else if constexpr (BYTES == 8) {
    return __builtin_bit_cast(Quad<T>, __builtin_nontemporal_load((const u32x2_nt*)p));
  } else if constexpr (BYTES == 16) {
    return __builtin_bit_cast(Quad<T>, __builtin_nontemporal_load((const u32x4_nt*)p));
  } else {
    static_assert(BYTES == 32, "element sizes 1, 2, 4 and 8");
    U32x8_nt w;
    w.lo = __builtin_nontemporal_load((const u32x4_nt*)p);
    w.hi = __builtin_nontemporal_load((const u32x4_nt*)p + 1);
    return __builtin_bit_cast(Quad<T>, w);
  }
}
template <typename I> __device__ __forceinline__ void st_i1(u8_t* __restrict__ p, I i, bool v) { p[i] = v ? 1 : 0; }

// ---- f32 transcendentals used by generated kernels ----
// exp: e^x = 2^(x log2 e). The product x * log2(e) is carried as eh + el, with el the exact rounding
// error of the f32 product (one FMA) plus x times the tail of log2(e); n = rint(eh) is clamped to
// [-160, 160] so that +-inf and NaN propagate through the same instructions; 2^f for |f| <= 0.5 comes
// from the hardware exp2 (v_exp_f32, 1 ulp) and 2^n from ldexp. About 1.5 ulp over the f32 range,
// with no compares (so no VCC hazard wait states). el is clamped to [-1, 1]: it is NaN only for
// infinite x, where the clamp turns it into a finite value and eh alone gives 0 or inf.
__device__ __forceinline__ float exp_f32(float x) {
  const float L2E = 0x1.715476p+0f, L2E_LO = 0x1.4ae0cp-26f;
  const float eh = x * L2E;
  const float el = __builtin_fminf(__builtin_fmaxf(__builtin_fmaf(x, L2E_LO, __builtin_fmaf(x, L2E, -eh)), -1.0f), 1.0f);
  const float n = __builtin_rintf(__builtin_fminf(__builtin_fmaxf(eh, -160.0f), 160.0f));
  const float f = (eh - n) + el;
  return __builtin_ldexpf(__builtin_amdgcn_exp2f(f), (int)n);
}

// tanh: for |x| >= 1/8, 1 - 2 / (e^(2|x|) + 1) with e^(2|x|) from the hardware exp2 (v_exp_f32) and
// the hardware reciprocal (v_rcp_f32), both about 1 ulp, so the result is within about 1e-6 relative
// (the exp2 argument's rounding dominates near |x| = 1/8); below 1/8 the odd Taylor polynomial to
// x^7 (truncation under 2e-9 relative), which avoids the cancellation of the first form. e = inf
// gives 1; NaN propagates through the first form; the sign is copied back (tanh(-0) = -0). No
// branches.
__device__ __forceinline__ float tanh_f32(float x) {
  const float ax = __builtin_fabsf(x);
  const float e = __builtin_amdgcn_exp2f(ax * 0x1.715476p+1f);  // e^(2|x|)
  const float big = __builtin_fmaf(-2.0f, __builtin_amdgcn_rcpf(e + 1.0f), 1.0f);
  const float x2 = ax * ax;
  float p = __builtin_fmaf(x2, -0x1.ba1ba2p-5f, 0x1.111112p-3f);  // -17/315, 2/15
  p = __builtin_fmaf(x2, p, -0x1.555556p-2f);                      // -1/3
  p = __builtin_fmaf(ax * x2, p, ax);
  return __builtin_copysignf(ax < 0.125f ? p : big, x);
}

// sin / cos: Cody-Waite reduction by pi/2 with a three-part constant (P1 + P2 + P3 = pi/2 to ~2^-75;
// the first FMA is exact for the quadrants below 2^17), then Taylor polynomials for sin and cos on
// [-pi/4, pi/4] (truncation below 2^-28). Arguments of magnitude 2^17 and beyond take the library's
// sinf / cosf (Payne-Hanek reduction).
__device__ __forceinline__ float sincos_core(float r, int q) {
  const float r2 = r * r;
  float s = __builtin_fmaf(r2, 0x1.71de3ap-19f, -0x1.a01a02p-13f);  // 1/9!, -1/7!
  s = __builtin_fmaf(r2, s, 0x1.111112p-7f);                          // 1/5!
  s = __builtin_fmaf(r2, s, -0x1.555556p-3f);                         // -1/3!
  s = __builtin_fmaf(r * r2, s, r);
  float c = __builtin_fmaf(r2, -0x1.27e4fcp-22f, 0x1.a01a02p-16f);  // -1/10!, 1/8!
  c = __builtin_fmaf(r2, c, -0x1.6c16c2p-10f);                        // -1/6!
  c = __builtin_fmaf(r2, c, 0x1.555556p-5f);                          // 1/4!
  c = __builtin_fmaf(r2, c, -0.5f);
  c = __builtin_fmaf(r2, c, 1.0f);
  const float v = (q & 1) ? c : s;
  return __builtin_bit_cast(float, __builtin_bit_cast(u32_t, v) ^ ((u32_t)(q & 2) << 30));
}

// sin with one polynomial: x = k pi + r, k = rint(x / pi) read off the low mantissa bits of
// x / pi + 1.5 * 2^23 (so the sign (-1)^k needs no integer conversion, and k = +0 for x = -0),
// r = x - k pi by the three-part reduction with FMAs, then an odd polynomial through r^9 and the
// sign. The polynomial r + r^3 P(r^2), P of degree 3, minimises the largest relative error against
// sin on [-pi/2, pi/2] (Remez exchange on (sin r - r) / r^3 weighted by r^3 / sin r; 6.1e-9 before
// the coefficients are rounded to f32), two FMAs fewer than the Taylor polynomial through r^13 with
// the same accuracy in f32 (1.74 against 1.80 ulp worst case over 4.6 million arguments).
// The library's reductions for |x| >= 2^17, out of line so that their code does not sit between the
// loads and arithmetic of every element that takes the fast path (`const`: no memory effects, so
// loads still move and merge across the calls).
__device__ __attribute__((noinline, const)) float sin_large(float x) { return sinf(x); }
__device__ __attribute__((noinline, const)) float cos_large(float x) { return cosf(x); }

__device__ __forceinline__ float sin_f32(float x) {
  const float M = 0x1.8p+23f;
  // pi = P1 + P2 + P3 + O(2^-74 pi), every part positive (P1, P2 rounded down), so that x = -0 keeps
  // r = -0 through all three FMAs.
  const float P1 = 0x1.921fb4p+1f, P2 = 0x1.4442d0p-23f, P3 = 0x1.84698ap-47f;
  const float t = __builtin_fmaf(x, 0x1.45f306p-2f, M);
  const float k = t - M;
  float r = __builtin_fmaf(-k, P1, x);
  r = __builtin_fmaf(-k, P2, r);
  r = __builtin_fmaf(-k, P3, r);
  const float r2 = r * r;
  float p = __builtin_fmaf(r2, 0x1.5dbdf0p-19f, -0x1.9f6ffep-13f);
  p = __builtin_fmaf(r2, p, 0x1.110ed4p-7f);
  p = __builtin_fmaf(r2, p, -0x1.55554cp-3f);
  // sin r has the sign of r on [-pi/2, pi/2]; or-ing r's sign bit in only matters for r = -0 (the
  // FMA turns it into +0).
  const float s = __builtin_fmaf(r * r2, p, r);
  const u32_t sb = __builtin_bit_cast(u32_t, s) | (__builtin_bit_cast(u32_t, r) & 0x80000000u);
  float v = __builtin_bit_cast(float, sb ^ (__builtin_bit_cast(u32_t, t) << 31));
  if (__builtin_fabsf(x) >= 0x1p+17f) v = sin_large(x);
  return v;
}

__device__ __forceinline__ float cos_f32(float x) {
  const float P1 = 0x1.921fb6p+0f, P2 = -0x1.777a5cp-25f, P3 = -0x1.ee59dap-50f;
  const float k = __builtin_rintf(x * 0x1.45f306p-1f);
  float r = __builtin_fmaf(-k, P1, x);
  r = __builtin_fmaf(-k, P2, r);
  r = __builtin_fmaf(-k, P3, r);
  float v = sincos_core(r, (int)k + 1);
  if (__builtin_fabsf(x) >= 0x1p+17f) v = cos_large(x);
  return v;
}

// ---- integer arithmetic wraps at the declared width; division by zero yields zero ----
template <typename T, typename U> __device__ __forceinline__ T wadd(T a, T b) { return (T)((U)a + (U)b); }
template <typename T, typename U> __device__ __forceinline__ T wsub(T a, T b) { return (T)((U)a - (U)b); }
template <typename T, typename U> __device__ __forceinline__ T wmul(T a, T b) { return (T)((U)a * (U)b); }
// Truncating division. A signed division by -1 is a negation that wraps (the most negative value stays
// itself), computed in 64-bit unsigned arithmetic so no step overflows; unsigned types divide plainly
// (their all-ones value is a large divisor, not -1).
template <typename T> __device__ __forceinline__ T idiv(T a, T b) {
  if (b == 0) return (T)0;
  if constexpr ((T)-1 < (T)0) {
    if (b == (T)-1) return (T)(0ull - (u64_t)(i64_t)a);
  }
  return (T)(a / b);
}
template <typename T> __device__ __forceinline__ T imax(T a, T b) { return a > b ? a : b; }
template <typename T> __device__ __forceinline__ T imin(T a, T b) { return a < b ? a : b; }
// A serial fold's float max / min step, as runCpu's x86 code computes it (maxss / minss, then a NaN
// result replaced by the first operand): the first operand when it is strictly greater (smaller) or
// the second is NaN, otherwise the second, so a tie (+0 / -0 included) keeps the later element and
// NaN elements are skipped. (v_max_f32 orders -0 below +0 and would keep +0 on such a tie.)
template <typename T> __device__ __forceinline__ T fold_max(T a, T b) { return (a > b || b != b) ? a : b; }
template <typename T> __device__ __forceinline__ T fold_min(T a, T b) { return (a < b || b != b) ? a : b; }

// ---- reduction operators ----
struct SumOp {
  template <typename T> __device__ __forceinline__ T operator()(T a, T b) const { return a + b; }
};
struct MaxOp {
  __device__ __forceinline__ float operator()(float a, float b) const { return fmaxf(a, b); }
  __device__ __forceinline__ double operator()(double a, double b) const { return fmax(a, b); }
  template <typename T> __device__ __forceinline__ T operator()(T a, T b) const { return a > b ? a : b; }
};
struct MinOp {
  __device__ __forceinline__ float operator()(float a, float b) const { return fminf(a, b); }
  __device__ __forceinline__ double operator()(double a, double b) const { return fmin(a, b); }
  template <typename T> __device__ __forceinline__ T operator()(T a, T b) const { return a < b ? a : b; }
};

// Butterfly reduction over the 64 lanes of a wavefront; every lane ends with the same value.
template <typename T, typename Op> __device__ __forceinline__ T wave_reduce(T v, Op op) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) v = op(v, __shfl_xor(v, offset, 64));
  return v;
}

// Workgroup reduction: wave partials go through LDS and every thread combines them in wave order,
// so all threads hold the same, deterministic result. `lds` holds at least BLOCK/64 elements.
template <int BLOCK, typename T, typename Op> __device__ __forceinline__ T block_reduce(T v, Op op, T* lds) {
  v = wave_reduce(v, op);
  if constexpr (BLOCK > 64) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) lds[wave] = v;
    __syncthreads();
    v = lds[0];
#pragma unroll
    for (int w = 1; w < BLOCK / 64; ++w) v = op(v, lds[w]);
    __syncthreads();
  }
  return v;
}

}  // namespace accy
