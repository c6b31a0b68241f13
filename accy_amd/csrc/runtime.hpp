// HIP runtime for the gfx950 target: kernel compilation (hiprtc), module cache, device buffers and
// execution of a kernel plan on one stream. This is the device layer the reference reaches through
// its backend vtable (deps/lib/compiler/gpu/src/contract.zig:2048-2084): load_artifact,
// allocate_buffer, write_buffer / read_buffer, launch, synchronize, destroy_object.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "ir.hpp"
#include "plan.hpp"

namespace accy {

// A failure with the status number it maps to (src/tensor/session/session.zig:33-43).
struct HipFailure : std::runtime_error {
  int status;
  HipFailure(int s, const std::string& m) : std::runtime_error(m), status(s) {}
};

constexpr int kStatusOk = 0, kStatusInvalidProgram = 1, kStatusUnsupportedVersion = 2, kStatusInvalidHandle = 3,
              kStatusInvalidBuffer = 4, kStatusTooManyPrograms = 5, kStatusOutOfMemory = 6,
              kStatusCompileFailed = 7, kStatusLaunchFailed = 8;
// Device buffers passed in place must be aligned to this many bytes (hipMalloc's are).
constexpr uintptr_t kMinBufferAlignment = 16;

// True when the byte ranges [a, a + an) and [b, b + bn) share a byte (empty ranges share none).
inline bool ranges_overlap(const void* a, size_t an, const void* b, size_t bn) {
  if (!an || !bn) return false;
  auto x = (const uint8_t*)a, y = (const uint8_t*)b;
  return x < y + bn && y < x + an;
}

// Compiles one generated kernel source for gfx950 with hiprtc; returns the code object.
std::vector<char> compile_kernel_source(const std::string& source, const std::string& name);

// The complete text hiprtc receives for a generated kernel: device helpers + kernel body.
std::string full_kernel_source(const std::string& body);

struct KernelTiming {
  std::string label, klass;
  double algorithmic_bytes = 0, algorithmic_flops = 0;
  float last_ms = 0;   // the latest recorded invocation
  float mean_ms = 0;   // mean over the recorded invocations
  uint32_t calls = 0;  // recorded invocations (at most kProfiledCalls)
};

// A compiled program bound to device memory: the HIP counterpart of the reference's loaded fragment.
class Executor {
 public:
  Executor(Program program, Plan plan);
  ~Executor();
  Executor(const Executor&) = delete;
  Executor& operator=(const Executor&) = delete;

  const Program& program() const { return program_; }
  const Plan& plan() const { return plan_; }

  // Host slices in, host slices out; sizes must equal the descriptors' byte sizes.
  void invoke_host(const void* const* inputs, const size_t* input_lens, size_t n_inputs, void* const* outputs,
                   const size_t* output_lens, size_t n_outputs);
  // Device pointers in and out, enqueued on `stream`, no synchronisation. With `scratch` set, every
  // intermediate buffer of the run (temporaries, scan carries, the scan bodies' temporaries) is taken
  // from [scratch, scratch + scratch_bytes()) instead of the executor's own allocations, and no
  // profiling events are recorded: the call then allocates no device memory and creates no object.
  void invoke_device(const void* const* inputs, size_t n_inputs, void* const* outputs, size_t n_outputs,
                     hipStream_t stream, uint8_t* scratch = nullptr);
  // Bytes of device scratch an invocation with `scratch` uses: every intermediate buffer at its own
  // 256-byte aligned offset (no reuse between buffers).
  uint64_t scratch_bytes() const { return scratch_total_; }

  // While profiling is on, every invocation records a HIP event pair around each kernel on the
  // launch stream (no synchronisation, so back-to-back invocations keep their steady state);
  // timings() waits for the recorded work and reports the last and the mean duration. Turning
  // profiling on starts a new measurement.
  static constexpr size_t kProfiledCalls = 256;
  void set_profiling(bool on);
  const std::vector<KernelTiming>& timings();

 private:
  void run_steps(hipStream_t stream, uint8_t* scratch);
  void launch(size_t step, hipStream_t stream);  // one kernel step with the slots bound now
  Program program_;
  Plan plan_;
  std::vector<void*> owned_;     // device allocation per slot (Temp / Const; staging for Input / Output)
  std::vector<void*> bound_;     // pointer used for each slot during a run
  std::vector<hipFunction_t> fn_;
  std::vector<uint8_t> skipped_;   // per profiled call and kernel: a run-once kernel was skipped
  hipStream_t stream_ = nullptr;
  bool profiling_ = false;
  bool pending_ = false;           // recorded events not yet read back
  size_t recorded_ = 0;            // invocations recorded since profiling was turned on
  std::vector<hipEvent_t> events_;  // kProfiledCalls slots of 2 events per kernel
  std::vector<KernelTiming> timings_;
  // Loop steps: the body's executor and two sets of carry buffers (carries in / out), per step.
  std::vector<std::unique_ptr<Executor>> loops_;
  std::vector<std::vector<void*>> loop_bufs_;
  void run_loop(size_t step, hipStream_t stream, uint8_t* scratch);
  // Scratch layout: offset of each temporary slot, and per loop step the offsets of its 2 x carries
  // buffers followed by the offset of its body's own scratch.
  std::vector<uint64_t> scratch_off_;
  std::vector<std::vector<uint64_t>> loop_scratch_off_;
  uint64_t scratch_total_ = 0;
};

int device_count();
std::string device_arch();

}  // namespace accy
