// Build-time check (compiled by accy_amd/build.py with hipcc --offload-arch=gfx950): instantiates the
// hand-written device templates with representative configurations so that a host without a GPU
// still verifies that they compile for CDNA4. Nothing calls these kernels.
#include "common.h"
#include "gemm.h"

struct CheckNN {
  static constexpr int DT = 0;
  static constexpr long M = 8192, N = 8192, K = 8192;
  static constexpr long A_B = 0, A_M = 8192, A_K = 1, B_B = 0, B_K = 8192, B_N = 1;
  static constexpr bool A_KC = true, B_KC = false;
  static constexpr int BM = 256, BN = 256, BK = 64, WAVES_M = 4, WAVES_N = 2;
};

struct CheckNT {
  static constexpr int DT = 1;
  static constexpr long M = 4100, N = 1000, K = 136;
  static constexpr long A_B = 4100 * 136, A_M = 136, A_K = 1, B_B = 1000 * 136, B_K = 1, B_N = 136;
  static constexpr bool A_KC = true, B_KC = true;
  static constexpr int BM = 256, BN = 256, BK = 64, WAVES_M = 4, WAVES_N = 2;
};

struct CheckEpi {
  u16_t* c;
  long ld;
  __device__ __forceinline__ void operator()(long b, long m, long n, float v) const { c[m * ld + n] = accy::f32_to_bf16(v); }
};

extern "C" __global__ void __launch_bounds__(512) accy_check_gemm_nn(const u16_t* a, const u16_t* b, u16_t* c) {
  accy::gemm::mma16<CheckNN>(a, b, CheckEpi{c, 8192});
}

extern "C" __global__ void __launch_bounds__(512) accy_check_gemm_nt(const u16_t* a, const u16_t* b, u16_t* c) {
  accy::gemm::mma16<CheckNT>(a, b, CheckEpi{c, 1000});
}

extern "C" __global__ void __launch_bounds__(256) accy_check_common(const float* x, float* y) {
  __shared__ float lds[4];
  float v = accy::exp_f32(x[threadIdx.x]) + accy::sin_f32(x[threadIdx.x]) + accy::cos_f32(x[threadIdx.x]);
  v = accy::block_reduce<256>(v, accy::SumOp(), lds);
  if (threadIdx.x == 0) y[blockIdx.x] = accy::round_bf16(v);
}

struct CheckDmaNN : accy::gemm::Strided<0, 8192, 1, 0, 8192, 1> {
  static constexpr int DT = 0;
  static constexpr long M = 8192, N = 8192, K = 8192;
  static constexpr long A_B = 0, A_M = 8192, A_K = 1, B_B = 0, B_K = 8192, B_N = 1;
  static constexpr bool A_KC = true, B_KC = false;
  static constexpr int BM = 256, BN = 256, STAGES = 4;
};

// Two workgroups per CU: a 256 x 128 tile, three stages (72 KiB of LDS each), K steps not a multiple
// of three (the tail schedule's remainder).
struct CheckDmaNN2 : CheckDmaNN {
  static constexpr long K = 2048;
  static constexpr int BM = 256, BN = 128, STAGES = 3;
};

struct CheckDmaTN : accy::gemm::Strided<0, 1, 384, 0, 1, 256> {
  static constexpr int DT = 1;
  static constexpr long M = 384, N = 128, K = 256;
  static constexpr long A_B = 0, A_M = 1, A_K = 384, B_B = 0, B_K = 1, B_N = 256;
  static constexpr bool A_KC = false, B_KC = true;
  static constexpr int BM = 128, BN = 128, STAGES = 4;
};

extern "C" __global__ void __launch_bounds__(256) accy_check_gemm_dma_nn(const u16_t* a, const u16_t* b, u16_t* c) {
  accy::gemm::mma16_dma<CheckDmaNN>(a, b, CheckEpi{c, 8192});
}

extern "C" __global__ void __launch_bounds__(256, 2) accy_check_gemm_dma_nn2(const u16_t* a, const u16_t* b, u16_t* c) {
  accy::gemm::mma16_dma<CheckDmaNN2>(a, b, CheckEpi{c, 8192});
}

extern "C" __global__ void __launch_bounds__(256) accy_check_gemm_dma_tn(const u16_t* a, const u16_t* b, u16_t* c) {
  accy::gemm::mma16_dma<CheckDmaTN>(a, b, CheckEpi{c, 128});
}

struct CheckF32NN : accy::gemm::Strided<0, 8192, 1, 0, 8192, 1> {
  static constexpr long M = 8192, N = 8192, K = 8192;
  static constexpr long A_B = 0, A_M = 8192, B_B = 0, B_K = 8192;
};

struct CheckEpiF32 {
  float* c;
  long ld;
  __device__ __forceinline__ void operator()(long b, long m, long n, float v) const { c[m * ld + n] = v; }
};

extern "C" __global__ void __launch_bounds__(256) accy_check_gemm_f32_nn(const float* a, const float* b, float* c) {
  accy::gemm::mma32f<CheckF32NN>(a, b, CheckEpiF32{c, 8192});
}

// A contraction over two named axes of a [batch, head, seq, hd] operand: rows (batch, seq), k (head, hd).
struct CheckDmaMultiAxis {
  static constexpr int DT = 0;
  static constexpr long M = 8192, N = 2048, K = 2048;
  static constexpr bool A_KC = true, B_KC = false;
  static constexpr int BM = 256, BN = 256, STAGES = 4;
  static __device__ __forceinline__ long a_b(long) { return 0; }
  static __device__ __forceinline__ long a_m(long i) { return (i / 2048) * 4194304L + (i % 2048) * 128L; }
  static __device__ __forceinline__ long a_k(long i) { return (i / 128) * 262144L + (i % 128); }
  static __device__ __forceinline__ long b_b(long) { return 0; }
  static __device__ __forceinline__ long b_k(long i) { return i * 2048L; }
  static __device__ __forceinline__ long b_n(long i) { return i; }
};

extern "C" __global__ void __launch_bounds__(256) accy_check_gemm_dma_multi(const u16_t* a, const u16_t* b, u16_t* c) {
  accy::gemm::mma16_dma<CheckDmaMultiAxis>(a, b, CheckEpi{c, 2048});
}
