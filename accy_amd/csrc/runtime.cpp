// HIP runtime for the gfx950 target. Kernels are compiled once per distinct source with hiprtc and
// cached for the life of the process; every executor owns its intermediate buffers and launches its
// plan in order on one stream (default priority).
#include "runtime.hpp"

#include <hip/hiprtc.h>

#include <algorithm>
#include <cstring>
#include <mutex>
#include <unordered_map>

namespace accy {

extern const char* const kCommonDeviceSource;
extern const char* const kGemmDeviceSource;
extern const char* const kAttentionDeviceSource;

namespace {

void check(hipError_t e, const char* what, int status = kStatusLaunchFailed) {
  if (e == hipSuccess) return;
  if (e == hipErrorOutOfMemory) status = kStatusOutOfMemory;
  throw HipFailure(status, std::string(what) + ": " + hipGetErrorString(e));
}

struct Module {
  hipModule_t module = nullptr;
  hipFunction_t function = nullptr;
};

std::mutex g_cache_mu;
std::unordered_map<std::string, Module>& module_cache() {
  static auto* c = new std::unordered_map<std::string, Module>();  // lives until process exit
  return *c;
}

hipFunction_t load_kernel(const std::string& body, const std::string& name) {
  std::string key = name + '\0' + body;
  {
    std::lock_guard<std::mutex> lock(g_cache_mu);
    auto it = module_cache().find(key);
    if (it != module_cache().end()) return it->second.function;
  }
  std::vector<char> code = compile_kernel_source(full_kernel_source(body), name);
  Module m;
  check(hipModuleLoadData(&m.module, code.data()), "hipModuleLoadData", kStatusCompileFailed);
  check(hipModuleGetFunction(&m.function, m.module, name.c_str()), "hipModuleGetFunction", kStatusCompileFailed);
  std::lock_guard<std::mutex> lock(g_cache_mu);
  module_cache()[key] = m;
  return m.function;
}

}  // namespace

// Generated kernels name the hand-written templates they instantiate with `#include "<name>"`; the
// template text (embedded in this library) replaces that line.
std::string full_kernel_source(const std::string& body) {
  std::string out = std::string(kCommonDeviceSource) + "\n";
  const std::pair<const char*, const char*> templates[] = {{"#include \"gemm\"\n", kGemmDeviceSource},
                                                           {"#include \"attention\"\n", kAttentionDeviceSource}};
  std::string rest = body;
  for (const auto& t : templates) {
    size_t p = rest.find(t.first);
    if (p != std::string::npos) rest.replace(p, std::strlen(t.first), std::string(t.second) + "\n");
  }
  return out + rest;
}

std::vector<char> compile_kernel_source(const std::string& source, const std::string& name) {
  hiprtcProgram prog;
  if (hiprtcCreateProgram(&prog, source.c_str(), (name + ".hip").c_str(), 0, nullptr, nullptr) != HIPRTC_SUCCESS)
    throw HipFailure(kStatusCompileFailed, "hiprtcCreateProgram failed");
  // Packed-f32 instructions stay disabled for every kernel this target builds. A source that
  // contains the line kMfmaVgprForm asks for MFMA results in VGPRs (the fused attention kernel,
  // whose VALU softmax reads every score: with accumulators in AGPRs each read is an extra copy).
  // The unroll threshold: loops marked `#pragma unroll` unroll whatever their size (a register-held
  // array indexed by the loop counter, such as a contraction's accumulator tile or a row cache, stays
  // in registers only when its loop unrolls fully; past LLVM's default size limit the loop stays and
  // the array moves to scratch memory).
  std::vector<const char*> opts = {"--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature",
                                   "-Xclang", "-packed-fp32-ops", "-mllvm", "-pragma-unroll-threshold=65536"};
  if (source.find(kMfmaVgprForm) != std::string::npos) {
    opts.push_back("-mllvm");
    opts.push_back("-amdgpu-mfma-vgpr-form");
  }
  hiprtcResult r = hiprtcCompileProgram(prog, (int)opts.size(), opts.data());
  if (r != HIPRTC_SUCCESS) {
    size_t n = 0;
    hiprtcGetProgramLogSize(prog, &n);
    std::string log(n, '\0');
    if (n) hiprtcGetProgramLog(prog, &log[0]);
    hiprtcDestroyProgram(&prog);
    throw HipFailure(kStatusCompileFailed, "hiprtc failed for " + name + ":\n" + log);
  }
  size_t size = 0;
  hiprtcGetCodeSize(prog, &size);
  std::vector<char> code(size);
  hiprtcGetCode(prog, code.data());
  hiprtcDestroyProgram(&prog);
  return code;
}

int device_count() {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n;
}

std::string device_arch() {
  int dev = 0;
  check(hipGetDevice(&dev), "hipGetDevice");
  hipDeviceProp_t p;
  check(hipGetDeviceProperties(&p, dev), "hipGetDeviceProperties");
  return p.gcnArchName;
}

Executor::Executor(Program program, Plan plan) : program_(std::move(program)), plan_(std::move(plan)) {
  if (device_count() <= 0) throw HipFailure(kStatusCompileFailed, "no HIP device");
  std::string arch = device_arch();
  if (arch.rfind("gfx950", 0) != 0) throw HipFailure(kStatusCompileFailed, "device is " + arch + ", not gfx950");
  owned_.assign(plan_.slots.size(), nullptr);
  bound_.assign(plan_.slots.size(), nullptr);
  try {
    check(hipStreamCreate(&stream_), "hipStreamCreate");
    for (size_t i = 0; i < plan_.slots.size(); ++i) {
      const SlotInfo& s = plan_.slots[i];
      if (s.role == SlotInfo::Input || s.role == SlotInfo::Output || s.bytes == 0) continue;
      check(hipMalloc(&owned_[i], s.bytes), "hipMalloc");
      if (s.role == SlotInfo::Const)
        check(hipMemcpy(owned_[i], s.data.data(), s.bytes, hipMemcpyHostToDevice), "hipMemcpy");
    }
    fn_.assign(plan_.steps.size(), nullptr);
    loops_.resize(plan_.steps.size());
    loop_bufs_.resize(plan_.steps.size());
    for (size_t i = 0; i < plan_.steps.size(); ++i) {
      const Step& st = plan_.steps[i];
      if (st.type != Step::Loop) continue;
      const Plan& bp = *st.loop.plan;
      loops_[i] = std::make_unique<Executor>(*st.loop.body, bp);
      const size_t nc = bp.input_slots.size();
      loop_bufs_[i].assign(2 * nc, nullptr);
      for (size_t c = 0; c < nc; ++c) {
        const uint64_t bytes = bp.slots[(size_t)bp.input_slots[c]].bytes;
        if (!bytes) continue;
        check(hipMalloc(&loop_bufs_[i][c], bytes), "hipMalloc");
        check(hipMalloc(&loop_bufs_[i][nc + c], bytes), "hipMalloc");
      }
    }
    // Scratch layout for allocation-free invocations: each intermediate buffer gets its own 256-byte
    // aligned range (temporaries, then per loop its carry buffers and its body's scratch).
    auto take = [&](uint64_t bytes) {
      const uint64_t off = scratch_total_;
      scratch_total_ += (bytes + 255) & ~uint64_t(255);
      return off;
    };
    scratch_off_.assign(plan_.slots.size(), 0);
    for (size_t i = 0; i < plan_.slots.size(); ++i)
      if (plan_.slots[i].role == SlotInfo::Temp) scratch_off_[i] = take(plan_.slots[i].bytes);
    loop_scratch_off_.resize(plan_.steps.size());
    for (size_t i = 0; i < plan_.steps.size(); ++i) {
      if (plan_.steps[i].type != Step::Loop) continue;
      const Plan& bp = *plan_.steps[i].loop.plan;
      const size_t nc = bp.input_slots.size();
      for (size_t b = 0; b < 2 * nc; ++b) loop_scratch_off_[i].push_back(take(bp.slots[(size_t)bp.input_slots[b % nc]].bytes));
      loop_scratch_off_[i].push_back(take(loops_[i]->scratch_bytes()));
    }
    int dev = 0, max_lds = 0;
    check(hipGetDevice(&dev), "hipGetDevice");
    check(hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev), "hipDeviceGetAttribute");
    for (size_t i = 0; i < plan_.steps.size(); ++i) {
      const Step& st = plan_.steps[i];
      if (st.type != Step::Kernel) continue;
      if ((int)st.kernel.shared_bytes > max_lds)
        throw HipFailure(kStatusCompileFailed, st.kernel.label + " needs " + std::to_string(st.kernel.shared_bytes) +
                                                   " bytes of LDS; the device allows " + std::to_string(max_lds));
      fn_[i] = load_kernel(st.kernel.source, st.kernel.name);
      KernelTiming t;
      t.label = st.kernel.label;
      t.klass = st.kernel.klass;
      t.algorithmic_bytes = st.kernel.algorithmic_bytes;
      t.algorithmic_flops = st.kernel.algorithmic_flops;
      timings_.push_back(t);
    }
    // Run-once kernels (lookup tables) depend on constants only: they fill their temporaries here, on
    // the executor's stream, before any invocation can be enqueued or captured into a graph, so every
    // later invocation on any stream finds the tables complete.
    for (size_t i = 0; i < plan_.slots.size(); ++i)
      if (plan_.slots[i].role == SlotInfo::Const || plan_.slots[i].role == SlotInfo::Temp) bound_[i] = owned_[i];
    bool any_once = false;
    for (size_t i = 0; i < plan_.steps.size(); ++i) {
      const Step& st = plan_.steps[i];
      if (st.type != Step::Kernel || !st.kernel.once) continue;
      for (int a : st.kernel.args) {
        const SlotInfo::Role r = plan_.slots[(size_t)a].role;
        if (r != SlotInfo::Const && r != SlotInfo::Temp)
          throw HipFailure(kStatusCompileFailed, st.kernel.label + ": a run-once kernel reads or writes a caller buffer");
      }
      launch(i, stream_);
      any_once = true;
    }
    if (any_once) check(hipStreamSynchronize(stream_), "hipStreamSynchronize");
  } catch (...) {
    if (stream_) (void)hipStreamSynchronize(stream_);  // a run-once kernel may still be running
    for (void* p : owned_)
      if (p) (void)hipFree(p);
    for (auto& bufs : loop_bufs_)
      for (void* p : bufs)
        if (p) (void)hipFree(p);
    if (stream_) (void)hipStreamDestroy(stream_);
    throw;
  }
}

Executor::~Executor() {
  if (stream_) (void)hipStreamSynchronize(stream_);
  for (hipEvent_t e : events_) (void)hipEventDestroy(e);
  for (void* p : owned_)
    if (p) (void)hipFree(p);
  for (auto& bufs : loop_bufs_)
    for (void* p : bufs)
      if (p) (void)hipFree(p);
  if (stream_) (void)hipStreamDestroy(stream_);
}

// Carries start as copies of the initial values; each iteration runs the body from one buffer set
// into the other on the same stream; the final carries are copied to the slots that read them.
void Executor::run_loop(size_t step, hipStream_t stream, uint8_t* scratch) {
  const LoopStep& L = plan_.steps[step].loop;
  const Plan& bp = *L.plan;
  const size_t nc = bp.input_slots.size();
  std::vector<void*> from_scratch;
  if (scratch) {
    from_scratch.resize(2 * nc);
    for (size_t b = 0; b < 2 * nc; ++b) from_scratch[b] = scratch + loop_scratch_off_[step][b];
  }
  std::vector<void*>& buf = scratch ? from_scratch : loop_bufs_[step];
  uint8_t* body_scratch = scratch ? scratch + loop_scratch_off_[step][2 * nc] : nullptr;
  auto bytes = [&](size_t c) { return bp.slots[(size_t)bp.input_slots[c]].bytes; };
  for (size_t c = 0; c < nc; ++c)
    if (bytes(c))
      check(hipMemcpyAsync(buf[c], bound_[(size_t)L.init_slots[c]], bytes(c), hipMemcpyDeviceToDevice, stream),
            "hipMemcpyAsync");
  size_t cur = 0;
  std::vector<const void*> in(nc);
  std::vector<void*> out(nc);
  for (int64_t it = 0; it < L.length; ++it) {
    for (size_t c = 0; c < nc; ++c) {
      in[c] = buf[cur * nc + c];
      out[c] = buf[(1 - cur) * nc + c];
    }
    loops_[step]->invoke_device(in.data(), nc, out.data(), nc, stream, body_scratch);
    cur = 1 - cur;
  }
  for (size_t c = 0; c < nc; ++c)
    if (L.result_slots[c] >= 0 && bytes(c))
      check(hipMemcpyAsync(bound_[(size_t)L.result_slots[c]], buf[cur * nc + c], bytes(c), hipMemcpyDeviceToDevice,
                           stream),
            "hipMemcpyAsync");
}

void Executor::set_profiling(bool on) {
  if (on) {
    recorded_ = 0;
    pending_ = false;
  }
  profiling_ = on;
}

const std::vector<KernelTiming>& Executor::timings() {
  if (!pending_) return timings_;
  const size_t nk = timings_.size(), n = std::min(recorded_, kProfiledCalls);
  const size_t last = (recorded_ - 1) % kProfiledCalls;
  // Each invocation's events are in stream order: its last end event completes after the others.
  for (size_t c = 0; c < n; ++c) check(hipEventSynchronize(events_[(c * nk + nk - 1) * 2 + 1]), "hipEventSynchronize");
  for (size_t k = 0; k < nk; ++k) {
    double sum = 0;
    for (size_t c = 0; c < n; ++c) {
      float ms = 0;
      check(hipEventElapsedTime(&ms, events_[(c * nk + k) * 2], events_[(c * nk + k) * 2 + 1]), "hipEventElapsedTime");
      if (skipped_[c * nk + k]) ms = 0.0f;
      sum += ms;
      if (c == last) timings_[k].last_ms = ms;
    }
    timings_[k].mean_ms = n ? (float)(sum / (double)n) : 0.0f;
    timings_[k].calls = (uint32_t)n;
  }
  pending_ = false;
  return timings_;
}

void Executor::launch(size_t step, hipStream_t stream) {
  const KernelStep& k = plan_.steps[step].kernel;
  std::vector<void*> ptrs(k.args.size());
  std::vector<void*> params(k.args.size());
  for (size_t a = 0; a < k.args.size(); ++a) {
    ptrs[a] = bound_[(size_t)k.args[a]];
    params[a] = &ptrs[a];
  }
  check(hipModuleLaunchKernel(fn_[step], k.grid[0], k.grid[1], k.grid[2], k.block[0], k.block[1], k.block[2],
                              k.shared_bytes, stream, params.data(), nullptr),
        "hipModuleLaunchKernel");
}

void Executor::run_steps(hipStream_t stream, uint8_t* scratch) {
  for (size_t i = 0; i < plan_.slots.size(); ++i) {
    if (plan_.slots[i].role == SlotInfo::Const) bound_[i] = owned_[i];
    if (plan_.slots[i].role == SlotInfo::Temp) bound_[i] = scratch ? scratch + scratch_off_[i] : owned_[i];
  }
  // Event slot of this invocation when profiling (created on first use; never with scratch).
  const size_t nk = timings_.size();
  hipEvent_t* ev = nullptr;
  uint8_t* skipped = nullptr;  // per kernel of this invocation: a run-once kernel skipped (0 ms)
  if (profiling_ && nk && !scratch) {
    const size_t slot = recorded_ % kProfiledCalls;
    if (events_.size() < (slot + 1) * nk * 2) {
      size_t old = events_.size();
      events_.resize((slot + 1) * nk * 2, nullptr);
      skipped_.resize((slot + 1) * nk, 0);
      for (size_t e = old; e < events_.size(); ++e) check(hipEventCreate(&events_[e]), "hipEventCreate");
    }
    ev = &events_[slot * nk * 2];
    skipped = &skipped_[slot * nk];
  }
  size_t ki = 0;
  for (size_t i = 0; i < plan_.steps.size(); ++i) {
    const Step& st = plan_.steps[i];
    if (st.type == Step::Copy) {
      check(hipMemcpyAsync(bound_[(size_t)st.copy.dst], bound_[(size_t)st.copy.src], st.copy.bytes,
                           hipMemcpyDeviceToDevice, stream),
            "hipMemcpyAsync");
      continue;
    }
    if (st.type == Step::Loop) {
      run_loop(i, stream, scratch);
      continue;
    }
    const KernelStep& k = st.kernel;
    if (k.once && !scratch) {  // filled by the constructor; the executor's own temporaries persist
      if (ev) {
        check(hipEventRecord(ev[2 * ki], stream), "hipEventRecord");
        check(hipEventRecord(ev[2 * ki + 1], stream), "hipEventRecord");
        skipped[ki] = 1;
      }
      ++ki;
      continue;
    }
    if (skipped) skipped[ki] = 0;
    if (ev) check(hipEventRecord(ev[2 * ki], stream), "hipEventRecord");
    launch(i, stream);
    if (ev) check(hipEventRecord(ev[2 * ki + 1], stream), "hipEventRecord");
    ++ki;
  }
  if (ev) {
    ++recorded_;
    pending_ = true;
  }
}

void Executor::invoke_device(const void* const* inputs, size_t n_inputs, void* const* outputs, size_t n_outputs,
                             hipStream_t stream, uint8_t* scratch) {
  if (n_inputs != plan_.input_slots.size() || n_outputs != plan_.output_slots.size())
    throw HipFailure(kStatusInvalidBuffer, "buffer count mismatch");
  // Buffers are used in place and the kernels read and write them with 16-byte vector accesses
  // (binding.zig:138-200 refuses an imported slice below the backend's minimum alignment).
  auto aligned = [](const void* p) { return ((uintptr_t)p & (kMinBufferAlignment - 1)) == 0; };
  for (size_t i = 0; i < n_inputs; ++i)
    if (!aligned(inputs[i])) throw HipFailure(kStatusInvalidBuffer, "input " + std::to_string(i) + " not 16-byte aligned");
  for (size_t i = 0; i < n_outputs; ++i)
    if (!aligned(outputs[i])) throw HipFailure(kStatusInvalidBuffer, "output " + std::to_string(i) + " not 16-byte aligned");
  // binding.zig:325-336 (expectDisjointOutputs): an output may share no byte with an input or with an
  // earlier output; kernels that read after another workgroup wrote would otherwise see its results.
  // Inputs may alias each other (they are only read).
  for (size_t o = 0; o < n_outputs; ++o) {
    const size_t ob = plan_.slots[(size_t)plan_.output_slots[o]].bytes;
    for (size_t i = 0; i < n_inputs; ++i)
      if (ranges_overlap(outputs[o], ob, inputs[i], plan_.slots[(size_t)plan_.input_slots[i]].bytes))
        throw HipFailure(kStatusInvalidBuffer, "output " + std::to_string(o) + " overlaps input " + std::to_string(i));
    for (size_t j = 0; j < o; ++j)
      if (ranges_overlap(outputs[o], ob, outputs[j], plan_.slots[(size_t)plan_.output_slots[j]].bytes))
        throw HipFailure(kStatusInvalidBuffer, "output " + std::to_string(o) + " overlaps output " + std::to_string(j));
  }
  for (size_t i = 0; i < n_inputs; ++i) bound_[(size_t)plan_.input_slots[i]] = const_cast<void*>(inputs[i]);
  for (size_t i = 0; i < n_outputs; ++i) bound_[(size_t)plan_.output_slots[i]] = outputs[i];
  run_steps(stream, scratch);
}

void Executor::invoke_host(const void* const* inputs, const size_t* input_lens, size_t n_inputs,
                           void* const* outputs, const size_t* output_lens, size_t n_outputs) {
  if (n_inputs != plan_.input_slots.size() || n_outputs != plan_.output_slots.size())
    throw HipFailure(kStatusInvalidBuffer, "buffer count mismatch");
  for (size_t i = 0; i < n_inputs; ++i)
    if (input_lens[i] != plan_.slots[(size_t)plan_.input_slots[i]].bytes)
      throw HipFailure(kStatusInvalidBuffer, "input " + std::to_string(i) + " size mismatch");
  for (size_t i = 0; i < n_outputs; ++i)
    if (output_lens[i] != plan_.slots[(size_t)plan_.output_slots[i]].bytes)
      throw HipFailure(kStatusInvalidBuffer, "output " + std::to_string(i) + " size mismatch");
  // Staging buffers for host invocations are allocated on first use and kept.
  for (int s : plan_.input_slots)
    if (!owned_[(size_t)s] && plan_.slots[(size_t)s].bytes) check(hipMalloc(&owned_[(size_t)s], plan_.slots[(size_t)s].bytes), "hipMalloc");
  for (int s : plan_.output_slots)
    if (!owned_[(size_t)s] && plan_.slots[(size_t)s].bytes) check(hipMalloc(&owned_[(size_t)s], plan_.slots[(size_t)s].bytes), "hipMalloc");
  std::vector<const void*> din(n_inputs);
  std::vector<void*> dout(n_outputs);
  for (size_t i = 0; i < n_inputs; ++i) {
    size_t s = (size_t)plan_.input_slots[i];
    din[i] = owned_[s];
    if (input_lens[i])
      check(hipMemcpyAsync(owned_[s], inputs[i], input_lens[i], hipMemcpyHostToDevice, stream_), "hipMemcpyAsync");
  }
  for (size_t i = 0; i < n_outputs; ++i) dout[i] = owned_[(size_t)plan_.output_slots[i]];
  invoke_device(din.data(), n_inputs, dout.data(), n_outputs, stream_);
  for (size_t i = 0; i < n_outputs; ++i)
    if (output_lens[i])
      check(hipMemcpyAsync(outputs[i], dout[i], output_lens[i], hipMemcpyDeviceToHost, stream_), "hipMemcpyAsync");
  check(hipStreamSynchronize(stream_), "hipStreamSynchronize");
}

}  // namespace accy
