// Kernel plan: what the HIP target runs for one program. The planner (lower.cpp) decides which values
// live in device buffers (slots) and which kernels compute them; the runtime (runtime.cpp) allocates
// the slots, compiles each kernel source with hiprtc for gfx950 and launches the steps in order.
//
// This plays the role of the reference's artifact plan (slots: inputs / outputs / intermediates,
// planned kernels, launch geometry; src/artifact/plan.zig:840-874, 2650-2688) and launch plan
// (src/executable/plan.zig:410), restated for one HIP device.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "ir.hpp"

namespace accy {

struct SlotInfo {
  enum Role : uint8_t { Input, Output, Temp, Const } role = Temp;
  int io_index = -1;  // parameter / output position for Input and Output slots
  uint64_t bytes = 0;
  DType dtype = DType::f32;
  std::string data;  // Const payload, uploaded once at compile time
};

// A generated source containing this line is compiled with MFMA results in VGPRs.
constexpr const char* kMfmaVgprForm = "// accy: mfma-vgpr-form\n";

struct KernelStep {
  std::string source;        // complete HIP source, compiled with hiprtc
  std::string name;          // extern "C" symbol in `source`
  std::vector<int> args;     // slot ids passed as device pointers, in parameter order
  uint32_t grid[3] = {1, 1, 1};
  uint32_t block[3] = {64, 1, 1};
  uint32_t shared_bytes = 0;
  std::string label;         // class and root value, e.g. "row:%11"
  std::string klass;         // "map", "row", "fold", "dot", "gemm", "attention", ...
  double algorithmic_bytes = 0;  // HBM bytes the kernel must move (inputs read once, outputs written)
  double algorithmic_flops = 0;  // useful floating-point work
  // Launch tuning: kernels with more than one launch candidate (results bit-identical across them)
  // carry a key (device family, class, fingerprint of the default source, shape) and the candidate
  // this source was generated for (0 = the planner's default).
  std::string tuning_key;
  uint32_t candidate_count = 1;
  uint32_t candidate = 0;
  // The kernel's output depends on constants only (a lookup table): an executor runs it once, when it
  // is built, into its own temporaries (which persist); a scratch-bound invocation runs it every time.
  bool once = false;
};

struct CopyStep {
  int src = -1, dst = -1;
  uint64_t bytes = 0;
};

struct Plan;

// A scan run as a host loop (src/tensor/lower.zig:119-167 lowers scans unrolled or host-looped): the
// body's plan runs `length` times, its parameters the current carries and its outputs the next ones.
struct LoopStep {
  std::shared_ptr<const Graph> body;
  std::shared_ptr<const Plan> plan;  // the body's plan (input / output slots = carries in / out)
  int64_t length = 0;
  std::vector<int> init_slots;       // per carry: the slot of its initial value
  std::vector<int> result_slots;     // per carry: the slot that receives its final value, or -1
};

struct Step {
  enum Type : uint8_t { Kernel, Copy, Loop } type = Kernel;
  KernelStep kernel;
  CopyStep copy;
  LoopStep loop;
};

struct Plan {
  std::vector<SlotInfo> slots;
  std::vector<Step> steps;
  std::vector<int> input_slots;   // per parameter
  std::vector<int> output_slots;  // per program output
};

class TuningTable;

struct LowerOptions {
  bool allow_gemm = true;       // MFMA contraction kernels for f32 / f16 / bf16
  bool allow_attention = true;  // fused QK^T -> softmax -> V
  bool allow_row = true;        // fused row pipelines (else serial folds)
  // Launch candidate per kernel index (the order of the plan's kernel steps), for measuring; a
  // kernel not listed takes the table's selection for its key, else candidate 0.
  std::map<size_t, uint32_t> force_candidate;
  const TuningTable* tuning = nullptr;
};

// Lowers a decoded program. Throws accy::Error(Unsupported) for operations the target cannot run.
Plan lower(const Program& program, const LowerOptions& options = {});

// Device source shared by every generated kernel (kernels/common.h), embedded at build time.
extern const char* const kCommonDeviceSource;
extern const char* const kGemmDeviceSource;
extern const char* const kAttentionDeviceSource;

}  // namespace accy
