// Launch tuning on the device: every candidate plan of a program is compiled, checked against the
// default plan's outputs byte for byte, and timed; the fastest candidate per tunable kernel goes
// into the tuning table (src/executable/tuning.zig:233-268, recordMeasurements).
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <type_traits>
#include <vector>

#include "plan.hpp"
#include "runtime.hpp"
#include "tuning.hpp"

namespace accy {

namespace {

void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) throw HipFailure(kStatusLaunchFailed, std::string(what) + ": " + hipGetErrorString(e));
}

struct Tunable {
  size_t kernel;  // index among the plan's kernel steps
  std::string key;
  uint32_t count;
};

}  // namespace

size_t tune_program(const Program& program, const void* const* inputs, size_t n_inputs, void* const* outputs,
                    size_t n_outputs, uint32_t repeats, TuningTable& table) {
  if (repeats == 0) repeats = 1;
  LowerOptions base;  // no table: the default candidates
  const Plan plan0 = lower(program, base);
  std::vector<Tunable> tun;
  size_t ki = 0;
  for (const Step& st : plan0.steps) {
    if (st.type != Step::Kernel) continue;
    if (st.kernel.candidate_count > 1) tun.push_back({ki, st.kernel.tuning_key, st.kernel.candidate_count});
    ++ki;
  }
  if (tun.empty()) return 0;
  uint32_t ncand = 0;
  for (const Tunable& t : tun) ncand = std::max(ncand, t.count);

  // One executor per candidate index: kernels with fewer candidates keep candidate 0.
  std::vector<std::unique_ptr<Executor>> ex;
  for (uint32_t c = 0; c < ncand; ++c) {
    LowerOptions o;
    for (const Tunable& t : tun) o.force_candidate[t.kernel] = c < t.count ? c : 0;
    ex.push_back(std::make_unique<Executor>(program, lower(program, o)));
  }
  if (n_outputs != plan0.output_slots.size() || n_inputs != plan0.input_slots.size())
    throw HipFailure(kStatusInvalidBuffer, "buffer count mismatch");

  hipStream_t stream = nullptr;
  hip_check(hipStreamCreate(&stream), "hipStreamCreate");
  std::unique_ptr<std::remove_pointer_t<hipStream_t>, decltype(&hipStreamDestroy)> guard(stream, &hipStreamDestroy);

  // Outputs of every candidate equal candidate 0's.
  std::vector<std::vector<uint8_t>> want(n_outputs), got(n_outputs);
  auto read_outputs = [&](std::vector<std::vector<uint8_t>>& into) {
    for (size_t i = 0; i < n_outputs; ++i) {
      into[i].resize(plan0.slots[(size_t)plan0.output_slots[i]].bytes);
      if (!into[i].empty())
        hip_check(hipMemcpyAsync(into[i].data(), outputs[i], into[i].size(), hipMemcpyDeviceToHost, stream),
                  "hipMemcpyAsync");
    }
    hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize");
  };
  for (uint32_t c = 0; c < ncand; ++c) {
    ex[c]->invoke_device(inputs, n_inputs, outputs, n_outputs, stream);
    read_outputs(c == 0 ? want : got);
    if (c > 0)
      for (size_t i = 0; i < n_outputs; ++i)
        if (got[i] != want[i])
          throw Error(Err::Unsupported, "launch candidate " + std::to_string(c) + " changed output " + std::to_string(i));
  }
  // Timing: candidates interleaved round by round, so that clock changes affect them alike.
  for (auto& e : ex) e->set_profiling(true);
  for (uint32_t r = 0; r < repeats; ++r)
    for (auto& e : ex) e->invoke_device(inputs, n_inputs, outputs, n_outputs, stream);
  hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize");

  // ACCY_TUNE_REPORT set: every candidate's mean goes to stderr (the artifact keeps the winner only).
  const bool report = std::getenv("ACCY_TUNE_REPORT") != nullptr;
  size_t recorded = 0;
  for (const Tunable& t : tun) {
    TuningSelection best;
    bool have = false;
    for (uint32_t c = 0; c < t.count; ++c) {
      const KernelTiming& kt = ex[c]->timings()[t.kernel];
      const uint64_t ns = (uint64_t)((double)kt.mean_ms * 1e6);
      if (report)
        std::fprintf(stderr, "tune %s candidate %u of %u: %.1f us over %u calls\n", t.key.c_str(), c, t.count,
                     kt.mean_ms * 1e3, kt.calls);
      if (!have || ns < best.mean_ns) {
        best = TuningSelection{c, ns, kt.calls};
        have = true;
      }
    }
    if (have && best.samples > 0) {
      table.record(t.key, t.count, best);
      ++recorded;
    }
  }
  return recorded;
}

}  // namespace accy
