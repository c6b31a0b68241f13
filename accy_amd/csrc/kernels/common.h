// Device helpers shared by every kernel the HIP target generates for gfx950: storage loads and stores
// for each element type, per-operation 16-bit rounding, integer wrap-around arithmetic, and wave64 /
// workgroup reductions. Generated kernels compute 16-bit floats in f32 and round back after every
// operation, and keep multiplies and adds separately rounded, as the reference's arithmetic contract
// requires (src/eval/root.zig:10-16).
#pragma once
#pragma clang fp contract(off)

typedef signed char i8_t;
typedef short i16_t;
typedef int i32_t;
typedef long long i64_t;
typedef unsigned char u8_t;
typedef unsigned short u16_t;
typedef unsigned int u32_t;
typedef unsigned long long u64_t;

namespace accy {

// ---- 16-bit floats: f16 is IEEE binary16, bf16 is the top half of an f32; both round to nearest even.
__device__ __forceinline__ float f16_to_f32(u16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ u16_t f32_to_f16(float x) { return __builtin_bit_cast(u16_t, (_Float16)x); }
__device__ __forceinline__ float bf16_to_f32(u16_t h) { return __builtin_bit_cast(float, ((u32_t)h) << 16); }
__device__ __forceinline__ u16_t f32_to_bf16(float x) { return __builtin_bit_cast(u16_t, (__bf16)x); }
__device__ __forceinline__ float round_f16(float x) { return (float)(_Float16)x; }
__device__ __forceinline__ float round_bf16(float x) { return (float)(__bf16)x; }

// ---- loads and stores in the compute domain (f32 for 16-bit floats) ----
template <typename I> __device__ __forceinline__ float ld_f16(const u16_t* __restrict__ p, I i) { return f16_to_f32(p[i]); }
template <typename I> __device__ __forceinline__ float ld_bf16(const u16_t* __restrict__ p, I i) { return bf16_to_f32(p[i]); }
template <typename I> __device__ __forceinline__ void st_f16(u16_t* __restrict__ p, I i, float v) { p[i] = f32_to_f16(v); }
template <typename I> __device__ __forceinline__ void st_bf16(u16_t* __restrict__ p, I i, float v) { p[i] = f32_to_bf16(v); }
template <typename T, typename I> __device__ __forceinline__ T ld(const T* __restrict__ p, I i) { return p[i]; }
template <typename T, typename I> __device__ __forceinline__ void st(T* __restrict__ p, I i, T v) { p[i] = v; }
template <typename I> __device__ __forceinline__ bool ld_i1(const u8_t* __restrict__ p, I i) { return p[i] != 0; }
template <typename I> __device__ __forceinline__ void st_i1(u8_t* __restrict__ p, I i, bool v) { p[i] = v ? 1 : 0; }

// ---- integer arithmetic wraps at the declared width; division by zero yields zero ----
template <typename T, typename U> __device__ __forceinline__ T wadd(T a, T b) { return (T)((U)a + (U)b); }
template <typename T, typename U> __device__ __forceinline__ T wsub(T a, T b) { return (T)((U)a - (U)b); }
template <typename T, typename U> __device__ __forceinline__ T wmul(T a, T b) { return (T)((U)a * (U)b); }
template <typename T> __device__ __forceinline__ T idiv(T a, T b) { return b == 0 ? (T)0 : ((b == (T)-1) ? (T)(0 - a) : (T)(a / b)); }
template <typename T> __device__ __forceinline__ T imax(T a, T b) { return a > b ? a : b; }
template <typename T> __device__ __forceinline__ T imin(T a, T b) { return a < b ? a : b; }

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
