// Build-time check (compiled by accy_amd/build.py with hipcc --offload-arch=gfx950): instantiates the
// fused attention template for the shapes the planner emits, so that a host without a GPU still
// verifies that it compiles for CDNA4. Nothing calls these kernels.
#include "common.h"
#include "gemm.h"
#include "attention.h"

struct CheckAttnF16 {
  static constexpr int DT = 1, HD = 128, WAVES = 8;
  static constexpr long SQ = 4096, SK = 4096, NB = 32;
  static constexpr long Q_S = 128, K_S = 128, V_S = 128;
  static constexpr bool CAUSAL = false;
  static constexpr float SL = 0x1.fe0000p-4f;
  static __device__ __forceinline__ long q_off(long b) { return b * 524288L; }
  static __device__ __forceinline__ long k_off(long b) { return b * 524288L; }
  static __device__ __forceinline__ long v_off(long b) { return b * 524288L; }
};

struct CheckAttnCausalBf16 {
  static constexpr int DT = 0, HD = 128, WAVES = 4;
  static constexpr long SQ = 2048, SK = 2048, NB = 64;
  static constexpr long Q_S = 2048, K_S = 2048, V_S = 2048;
  static constexpr bool CAUSAL = true;
  static constexpr float SL = 0x1.fe0000p-4f;
  static __device__ __forceinline__ long q_off(long b) { return (b / 16) * 4194304L + (b % 16) * 128L; }
  static __device__ __forceinline__ long k_off(long b) { return (b / 16) * 4194304L + (b % 16) * 128L; }
  static __device__ __forceinline__ long v_off(long b) { return (b / 16) * 4194304L + (b % 16) * 128L; }
};

struct CheckAttnHd64Bf16 {
  static constexpr int DT = 0, HD = 64, WAVES = 4;
  static constexpr long SQ = 1024, SK = 1024, NB = 8;
  static constexpr long Q_S = 64, K_S = 64, V_S = 64;
  static constexpr bool CAUSAL = true;
  static constexpr float SL = 0x1.6a09e6p-2f;
  static __device__ __forceinline__ long q_off(long b) { return b * 65536L; }
  static __device__ __forceinline__ long k_off(long b) { return b * 65536L; }
  static __device__ __forceinline__ long v_off(long b) { return b * 65536L; }
};

extern "C" __global__ void __launch_bounds__(256) accy_check_attention_hd64_bf16(const u16_t* q, const u16_t* k, const u16_t* v, u16_t* o) {
  accy::attn::flash<CheckAttnHd64Bf16>(q, k, v, o);
}

extern "C" __global__ void __launch_bounds__(512) accy_check_attention_f16(const u16_t* q, const u16_t* k, const u16_t* v, u16_t* o) {
  accy::attn::flash<CheckAttnF16>(q, k, v, o);
}

extern "C" __global__ void __launch_bounds__(256) accy_check_attention_causal_bf16(const u16_t* q, const u16_t* k, const u16_t* v, u16_t* o) {
  accy::attn::flash<CheckAttnCausalBf16>(q, k, v, o);
}

struct CheckAttnF32Causal {
  static constexpr int WAVES = 4;
  static constexpr long SQ = 1024, SK = 1024, NB = 4;
  static constexpr long Q_S = 64, K_S = 64, V_S = 64;
  static constexpr bool CAUSAL = true;
  static constexpr float SL = 0x1.6a09e6p-2f;
  static __device__ __forceinline__ long q_off(long b) { return b * 65536L; }
  static __device__ __forceinline__ long k_off(long b) { return b * 65536L; }
  static __device__ __forceinline__ long v_off(long b) { return b * 65536L; }
};

extern "C" __global__ void __launch_bounds__(256) accy_check_attention_f32(const float* q, const float* k, const float* v, float* o) {
  accy::attn::flash_f32<CheckAttnF32Causal>(q, k, v, o);
}
