// C ABI of the gfx950 target (include/accy_hip.h): a 64-entry handle table with generations, as the
// reference session keeps (src/tensor/session/session.zig:99-246), over HIP executors.
#include "../../include/accy_hip.h"

#include <algorithm>
#include <cstring>
#include <memory>
#include <mutex>
#include <new>
#include <string>

#include "plan.hpp"
#include "runtime.hpp"
#include "scratch.hpp"
#include "tuning.hpp"
#include "wire.hpp"

using namespace accy;

namespace {

thread_local std::string g_last_error;

struct Entry {
  bool live = false;
  uint32_t generation = 0;
  // Shared with every invocation in progress: a release on another thread retires the handle (its
  // generation moves on, so later calls get INVALID_HANDLE, session.zig:228-233) while an invocation
  // already running keeps the executor alive until it returns.
  std::shared_ptr<Executor> exec;
  // Descriptor storage: names and extents per input, then per output.
  std::vector<std::vector<std::string>> names;
  std::vector<std::vector<const char*>> name_ptrs;
  std::vector<std::vector<int64_t>> extents;
  std::vector<std::string> labels, klasses;
};

std::mutex g_mu;
Entry g_entries[ACCY_HIP_MAX_PROGRAMS];

int fail_with(int status, const std::string& msg) {
  g_last_error = msg;
  return status;
}

int status_of(const Error& e) {
  switch (e.code) {
    case Err::UnsupportedVersion: return ACCY_HIP_UNSUPPORTED_VERSION;
    case Err::Unsupported: return ACCY_HIP_COMPILE_FAILED;
    default: return ACCY_HIP_INVALID_PROGRAM;
  }
}

Entry* lookup(accy_hip_handle h) {
  if (h.index >= ACCY_HIP_MAX_PROGRAMS) return nullptr;
  Entry& e = g_entries[h.index];
  if (!e.live || e.generation != h.generation) return nullptr;
  return &e;
}

template <typename F>
int guarded(F&& f) {
  try {
    return f();
  } catch (const HipFailure& e) {
    return fail_with(e.status, e.what());
  } catch (const Error& e) {
    return fail_with(status_of(e), e.what());
  } catch (const std::bad_alloc&) {
    return fail_with(ACCY_HIP_OUT_OF_MEMORY, "out of memory");
  } catch (const std::exception& e) {
    return fail_with(ACCY_HIP_COMPILE_FAILED, e.what());
  }
}

// Sizes this target plans. A parameter or output over 1 TiB (more than one device's 288 GB of HBM)
// could never be allocated, and is refused when the program is decoded, with OUT_OF_MEMORY as an
// allocation would fail. Intermediates may be larger as long as they are fused away (a contraction
// spelled as a product and a sum has an [m, k, n] intermediate: 2 TiB of f32 at 8192^3), but no value
// may exceed 2^50 elements: with that bound every product of extents within a value fits in int64.
constexpr uint64_t kMaxMaterialBytes = 1ull << 40;
constexpr uint64_t kMaxValueElements = 1ull << 50;

void check_capacity(const Graph& g, bool top) {
  auto too_big = [](size_t i, const std::string& what) {
    throw HipFailure(kStatusOutOfMemory, "value %" + std::to_string(i) + " " + what);
  };
  for (size_t i = 0; i < g.ops.size(); ++i) {
    const Op& op = g.ops[i];
    const uint64_t n = op.result.elements();  // ShapeElementOverflow past 2^64
    if (n > kMaxValueElements) too_big(i, "has " + std::to_string(n) + " elements, more than this target plans");
    if (op.body) check_capacity(*op.body, false);
  }
  if (!top) return;
  std::vector<uint32_t> materialised = g.params;
  materialised.insert(materialised.end(), g.outputs.begin(), g.outputs.end());
  for (uint32_t id : materialised) {
    const uint64_t bytes = g.type(id).bytes();
    if (bytes > kMaxMaterialBytes) too_big(id, "needs " + std::to_string(bytes) + " bytes, more than one device holds");
  }
}

Program decode_program(const uint8_t* wire, size_t len) {
  if (!wire && len) throw Error(Err::InvalidArtifact, "null wire bytes");
  Program p = wire::decode(wire, len);
  check_capacity(p, true);
  return p;
}

void fill_descriptors(Entry& e) {
  const Program& p = e.exec->program();
  e.names.clear();
  e.name_ptrs.clear();
  e.extents.clear();
  auto add = [&](uint32_t vid) {
    const Type& t = p.type(vid);
    std::vector<std::string> n;
    std::vector<int64_t> x;
    for (const Dim& d : t.dims) {
      n.push_back(d.name);
      x.push_back(d.extent);
    }
    e.names.push_back(std::move(n));
    e.extents.push_back(std::move(x));
  };
  for (uint32_t v : p.params) add(v);
  for (uint32_t v : p.outputs) add(v);
  for (auto& n : e.names) {
    std::vector<const char*> ptrs;
    for (auto& s : n) ptrs.push_back(s.c_str());
    e.name_ptrs.push_back(std::move(ptrs));
  }
  e.labels.clear();
  e.klasses.clear();
  for (const auto& t : e.exec->timings()) {
    e.labels.push_back(t.label);
    e.klasses.push_back(t.klass);
  }
}

bool overlaps(const void* a, size_t an, const void* b, size_t bn) { return ranges_overlap(a, an, b, bn); }

// The executor of a live handle, held for the duration of a call made outside the table's lock.
std::shared_ptr<Executor> hold(accy_hip_handle h) {
  std::lock_guard<std::mutex> lock(g_mu);
  Entry* e = lookup(h);
  return e ? e->exec : nullptr;
}

}  // namespace

extern "C" {

int accy_hip_compile(const uint8_t* wire_bytes, size_t wire_len, accy_hip_handle* out) {
  return guarded([&]() -> int {
    if (!out) return fail_with(ACCY_HIP_INVALID_BUFFER, "null handle pointer");
    uint32_t index = ACCY_HIP_MAX_PROGRAMS;
    {
      std::lock_guard<std::mutex> lock(g_mu);
      for (uint32_t i = 0; i < ACCY_HIP_MAX_PROGRAMS; ++i)
        if (!g_entries[i].live) {
          index = i;
          break;
        }
    }
    if (index == ACCY_HIP_MAX_PROGRAMS) return fail_with(ACCY_HIP_TOO_MANY_PROGRAMS, "all 64 slots hold programs");
    Program prog;
    try {
      prog = decode_program(wire_bytes, wire_len);
    } catch (const Error& e) {
      return fail_with(e.code == Err::UnsupportedVersion ? ACCY_HIP_UNSUPPORTED_VERSION : ACCY_HIP_INVALID_PROGRAM,
                       e.what());
    }
    Plan plan;
    try {
      LowerOptions opt;
      opt.tuning = &process_tuning();
      plan = lower(prog, opt);
    } catch (const Error& e) {
      return fail_with(ACCY_HIP_COMPILE_FAILED, e.what());
    }
    auto exec = std::make_shared<Executor>(std::move(prog), std::move(plan));
    // The allocation-free entry point's device scratch: its address on this device is looked up now
    // (which may load the array's code object), so that accy_hip_invoke_device_scratch, possibly under
    // graph capture, only reads the kept address. A failure here is reported by that call.
    {
      void* base = nullptr;
      const char* why = "";
      (void)scratch_region(&base, &why);
    }
    std::lock_guard<std::mutex> lock(g_mu);
    Entry* e = &g_entries[index];
    if (e->live) {  // taken by another thread meanwhile
      index = ACCY_HIP_MAX_PROGRAMS;
      for (uint32_t i = 0; i < ACCY_HIP_MAX_PROGRAMS; ++i)
        if (!g_entries[i].live) {
          index = i;
          break;
        }
      if (index == ACCY_HIP_MAX_PROGRAMS) return fail_with(ACCY_HIP_TOO_MANY_PROGRAMS, "all 64 slots hold programs");
      e = &g_entries[index];
    }
    e->live = true;
    e->exec = std::move(exec);
    fill_descriptors(*e);
    out->index = index;
    out->generation = e->generation;
    return ACCY_HIP_OK;
  });
}

int accy_hip_counts(accy_hip_handle h, size_t* n_inputs, size_t* n_outputs) {
  std::lock_guard<std::mutex> lock(g_mu);
  Entry* e = lookup(h);
  if (!e) return fail_with(ACCY_HIP_INVALID_HANDLE, "stale or unknown handle");
  if (n_inputs) *n_inputs = e->exec->program().params.size();
  if (n_outputs) *n_outputs = e->exec->program().outputs.size();
  return ACCY_HIP_OK;
}

int accy_hip_describe(accy_hip_handle h, int which, size_t index, accy_hip_descriptor* out) {
  std::lock_guard<std::mutex> lock(g_mu);
  Entry* e = lookup(h);
  if (!e) return fail_with(ACCY_HIP_INVALID_HANDLE, "stale or unknown handle");
  const Program& p = e->exec->program();
  size_t n = which == 0 ? p.params.size() : p.outputs.size();
  if (index >= n || !out) return fail_with(ACCY_HIP_INVALID_BUFFER, "descriptor index out of range");
  size_t slot = which == 0 ? index : p.params.size() + index;
  const Type& t = p.type(which == 0 ? p.params[index] : p.outputs[index]);
  out->dtype = (uint32_t)t.dtype;
  out->rank = (uint32_t)t.rank();
  out->names = e->name_ptrs[slot].data();
  out->extents = e->extents[slot].data();
  out->byte_size = t.bytes();
  // session.zig:284 reports max(slot alignment, backend minimum): a borrowed device buffer must meet
  // the 16 bytes accy_hip_invoke_device checks.
  out->alignment = (uint32_t)std::max<size_t>(dtype_size(t.dtype), kMinBufferAlignment);
  return ACCY_HIP_OK;
}

int accy_hip_invoke(accy_hip_handle h, const void* const* inputs, const size_t* input_lens, size_t n_inputs,
                    void* const* outputs, const size_t* output_lens, size_t n_outputs) {
  std::shared_ptr<Executor> ex = hold(h);
  if (!ex) return fail_with(ACCY_HIP_INVALID_HANDLE, "stale or unknown handle");
  return guarded([&]() -> int {
    if (n_inputs && (!inputs || !input_lens)) return fail_with(ACCY_HIP_INVALID_BUFFER, "null input list");
    if (n_outputs && (!outputs || !output_lens)) return fail_with(ACCY_HIP_INVALID_BUFFER, "null output list");
    // session.zig:173-179: an output may share no bytes with an input or another output.
    for (size_t o = 0; o < n_outputs; ++o) {
      for (size_t i = 0; i < n_inputs; ++i)
        if (overlaps(outputs[o], output_lens[o], inputs[i], input_lens[i]))
          return fail_with(ACCY_HIP_INVALID_BUFFER, "output overlaps an input");
      for (size_t j = 0; j < o; ++j)
        if (overlaps(outputs[o], output_lens[o], outputs[j], output_lens[j]))
          return fail_with(ACCY_HIP_INVALID_BUFFER, "outputs overlap");
    }
    ex->invoke_host(inputs, input_lens, n_inputs, outputs, output_lens, n_outputs);
    return ACCY_HIP_OK;
  });
}

int accy_hip_invoke_device(accy_hip_handle h, const void* const* inputs, size_t n_inputs, void* const* outputs,
                           size_t n_outputs, void* stream) {
  std::shared_ptr<Executor> ex = hold(h);
  if (!ex) return fail_with(ACCY_HIP_INVALID_HANDLE, "stale or unknown handle");
  return guarded([&]() -> int {
    if (n_inputs && !inputs) return fail_with(ACCY_HIP_INVALID_BUFFER, "null input list");
    if (n_outputs && !outputs) return fail_with(ACCY_HIP_INVALID_BUFFER, "null output list");
    ex->invoke_device(inputs, n_inputs, outputs, n_outputs, (hipStream_t)stream);
    return ACCY_HIP_OK;
  });
}

int accy_hip_invoke_device_scratch(accy_hip_handle h, const void* const* inputs, size_t n_inputs,
                                   void* const* outputs, size_t n_outputs, void* stream) {
  std::shared_ptr<Executor> ex = hold(h);
  if (!ex) return fail_with(ACCY_HIP_INVALID_HANDLE, "stale or unknown handle");
  return guarded([&]() -> int {
    if (n_inputs && !inputs) return fail_with(ACCY_HIP_INVALID_BUFFER, "null input list");
    if (n_outputs && !outputs) return fail_with(ACCY_HIP_INVALID_BUFFER, "null output list");
    if (ex->scratch_bytes() > kScratchBytes)
      return fail_with(ACCY_HIP_OUT_OF_MEMORY, "the program's intermediate buffers need " +
                                                   std::to_string(ex->scratch_bytes()) +
                                                   " bytes; the device scratch holds " +
                                                   std::to_string(kScratchBytes));
    void* base = nullptr;
    const char* why = "";
    if (scratch_region(&base, &why) != 0) return fail_with(ACCY_HIP_LAUNCH_FAILED, std::string("device scratch: ") + why);
    ex->invoke_device(inputs, n_inputs, outputs, n_outputs, (hipStream_t)stream, (uint8_t*)base);
    return ACCY_HIP_OK;
  });
}

int accy_hip_release(accy_hip_handle h) {
  std::shared_ptr<Executor> dead;  // freed here unless an invocation still holds it
  {
    std::lock_guard<std::mutex> lock(g_mu);
    Entry* e = lookup(h);
    if (!e) return fail_with(ACCY_HIP_INVALID_HANDLE, "stale or unknown handle");
    dead = std::move(e->exec);
    uint32_t gen = e->generation + 1;
    *e = Entry();
    e->generation = gen;
  }
  return ACCY_HIP_OK;
}

int accy_hip_run(const uint8_t* wire_bytes, size_t wire_len, const void* const* inputs, const size_t* input_lens,
                 size_t n_inputs, void* const* outputs, const size_t* output_lens, size_t n_outputs) {
  accy_hip_handle h;
  int s = accy_hip_compile(wire_bytes, wire_len, &h);
  if (s != ACCY_HIP_OK) return s;
  s = accy_hip_invoke(h, inputs, input_lens, n_inputs, outputs, output_lens, n_outputs);
  std::string err = g_last_error;
  accy_hip_release(h);
  g_last_error = err;
  return s;
}

const char* accy_hip_last_error(void) { return g_last_error.c_str(); }

int accy_hip_set_profiling(accy_hip_handle h, int enable) {
  std::lock_guard<std::mutex> lock(g_mu);
  Entry* e = lookup(h);
  if (!e) return fail_with(ACCY_HIP_INVALID_HANDLE, "stale or unknown handle");
  return guarded([&]() -> int {
    e->exec->set_profiling(enable != 0);
    return ACCY_HIP_OK;
  });
}

int accy_hip_kernel_count(accy_hip_handle h, size_t* n) {
  std::lock_guard<std::mutex> lock(g_mu);
  Entry* e = lookup(h);
  if (!e) return fail_with(ACCY_HIP_INVALID_HANDLE, "stale or unknown handle");
  if (n) *n = e->exec->timings().size();
  return ACCY_HIP_OK;
}

int accy_hip_kernel_info(accy_hip_handle h, size_t index, accy_hip_kernel_stats* out) {
  std::lock_guard<std::mutex> lock(g_mu);
  Entry* e = lookup(h);
  if (!e) return fail_with(ACCY_HIP_INVALID_HANDLE, "stale or unknown handle");
  const auto& t = e->exec->timings();
  if (index >= t.size() || !out) return fail_with(ACCY_HIP_INVALID_BUFFER, "kernel index out of range");
  out->label = e->labels[index].c_str();
  out->klass = e->klasses[index].c_str();
  out->algorithmic_bytes = t[index].algorithmic_bytes;
  out->algorithmic_flops = t[index].algorithmic_flops;
  out->last_ms = t[index].last_ms;
  out->mean_ms = t[index].mean_ms;
  out->calls = t[index].calls;
  return ACCY_HIP_OK;
}

// Writes each step of a plan; a loop step's body plan follows, indented by its nesting depth.
static void append_plan_source(const Plan& plan, bool compile, const std::string& indent, std::string& text) {
  for (const Step& st : plan.steps) {
    if (st.type == Step::Copy) {
      text += indent + "// copy slot " + std::to_string(st.copy.src) + " -> " + std::to_string(st.copy.dst) + "\n";
      continue;
    }
    if (st.type == Step::Loop) {
      text += indent + "// loop " + std::to_string(st.loop.length) + " times over " +
              std::to_string(st.loop.init_slots.size()) + " carries {\n";
      append_plan_source(*st.loop.plan, compile, indent + "  ", text);
      text += indent + "// }\n";
      continue;
    }
    const KernelStep& k = st.kernel;
    text += indent + "// " + k.label + " grid " + std::to_string(k.grid[0]) + " block " + std::to_string(k.block[0]) + "\n";
    if (k.candidate_count > 1)
      text += indent + "// tuning " + k.tuning_key + " candidate " + std::to_string(k.candidate) + " of " +
              std::to_string(k.candidate_count) + "\n";
    text += k.source;
    if (compile) compile_kernel_source(full_kernel_source(k.source), k.name);
  }
}

int accy_hip_plan_source(const uint8_t* wire_bytes, size_t wire_len, int compile, char* buf, size_t cap,
                         size_t* needed) {
  return guarded([&]() -> int {
    Program prog;
    try {
      prog = decode_program(wire_bytes, wire_len);
    } catch (const Error& e) {
      return fail_with(e.code == Err::UnsupportedVersion ? ACCY_HIP_UNSUPPORTED_VERSION : ACCY_HIP_INVALID_PROGRAM,
                       e.what());
    }
    LowerOptions opt;
    opt.tuning = &process_tuning();
    Plan plan = lower(prog, opt);
    std::string text;
    append_plan_source(plan, compile != 0, "", text);
    if (needed) *needed = text.size() + 1;
    if (buf && cap) {
      size_t n = std::min(cap - 1, text.size());
      std::memcpy(buf, text.data(), n);
      buf[n] = '\0';
    }
    return ACCY_HIP_OK;
  });
}

int accy_hip_tune(const uint8_t* wire_bytes, size_t wire_len, const void* const* inputs, size_t n_inputs,
                  void* const* outputs, size_t n_outputs, uint32_t repeats, size_t* n_tuned) {
  return guarded([&]() -> int {
    if (n_inputs && !inputs) return fail_with(ACCY_HIP_INVALID_BUFFER, "null input list");
    if (n_outputs && !outputs) return fail_with(ACCY_HIP_INVALID_BUFFER, "null output list");
    Program prog;
    try {
      prog = decode_program(wire_bytes, wire_len);
    } catch (const Error& e) {
      return fail_with(e.code == Err::UnsupportedVersion ? ACCY_HIP_UNSUPPORTED_VERSION : ACCY_HIP_INVALID_PROGRAM,
                       e.what());
    }
    size_t n = 0;
    try {
      n = tune_program(prog, inputs, n_inputs, outputs, n_outputs, repeats, process_tuning());
    } catch (const Error& e) {
      return fail_with(ACCY_HIP_COMPILE_FAILED, e.what());
    }
    if (n_tuned) *n_tuned = n;
    return ACCY_HIP_OK;
  });
}

int accy_hip_tuning_export(uint8_t* buf, size_t cap, size_t* needed) {
  return guarded([&]() -> int {
    const std::vector<uint8_t> bytes = process_tuning().encode();
    if (needed) *needed = bytes.size();
    if (buf && cap) {
      if (cap < bytes.size()) return fail_with(ACCY_HIP_INVALID_BUFFER, "export buffer too small");
      std::memcpy(buf, bytes.data(), bytes.size());
    }
    return ACCY_HIP_OK;
  });
}

int accy_hip_tuning_import(const uint8_t* data, size_t len) {
  return guarded([&]() -> int {
    if (!data && len) return fail_with(ACCY_HIP_INVALID_BUFFER, "null artifact");
    process_tuning().merge(data, len);
    return ACCY_HIP_OK;
  });
}

int accy_hip_tuning_count(size_t* n) {
  if (!n) return fail_with(ACCY_HIP_INVALID_BUFFER, "null count pointer");
  *n = process_tuning().size();
  return ACCY_HIP_OK;
}

int accy_hip_tuning_clear(void) {
  process_tuning().clear();
  return ACCY_HIP_OK;
}

static int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return ACCY_HIP_OK;
  return fail_with(e == hipErrorOutOfMemory ? ACCY_HIP_OUT_OF_MEMORY : ACCY_HIP_LAUNCH_FAILED,
                   std::string(what) + ": " + hipGetErrorString(e));
}

int accy_hip_malloc(void** ptr, size_t bytes) {
  if (!ptr) return fail_with(ACCY_HIP_INVALID_BUFFER, "null pointer");
  *ptr = nullptr;
  if (bytes == 0) return ACCY_HIP_OK;
  return hip_status(hipMalloc(ptr, bytes), "hipMalloc");
}

int accy_hip_free(void* ptr) { return ptr ? hip_status(hipFree(ptr), "hipFree") : ACCY_HIP_OK; }

int accy_hip_memcpy(void* dst, const void* src, size_t bytes, int kind) {
  if (bytes == 0) return ACCY_HIP_OK;
  hipMemcpyKind k = kind == 1 ? hipMemcpyHostToDevice : kind == 2 ? hipMemcpyDeviceToHost : hipMemcpyDeviceToDevice;
  if (kind < 1 || kind > 3) return fail_with(ACCY_HIP_INVALID_BUFFER, "copy kind must be 1, 2 or 3");
  return hip_status(hipMemcpy(dst, src, bytes, k), "hipMemcpy");
}

int accy_hip_stream_create(void** stream) {
  if (!stream) return fail_with(ACCY_HIP_INVALID_BUFFER, "null pointer");
  return hip_status(hipStreamCreate((hipStream_t*)stream), "hipStreamCreate");
}

int accy_hip_stream_destroy(void* stream) { return hip_status(hipStreamDestroy((hipStream_t)stream), "hipStreamDestroy"); }

int accy_hip_stream_synchronize(void* stream) {
  return hip_status(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
}

int accy_hip_event_create(void** event) {
  if (!event) return fail_with(ACCY_HIP_INVALID_BUFFER, "null pointer");
  return hip_status(hipEventCreate((hipEvent_t*)event), "hipEventCreate");
}

int accy_hip_event_destroy(void* event) { return hip_status(hipEventDestroy((hipEvent_t)event), "hipEventDestroy"); }

int accy_hip_event_record(void* event, void* stream) {
  return hip_status(hipEventRecord((hipEvent_t)event, (hipStream_t)stream), "hipEventRecord");
}

int accy_hip_event_elapsed_ms(float* ms, void* start, void* end) {
  if (!ms) return fail_with(ACCY_HIP_INVALID_BUFFER, "null pointer");
  return hip_status(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)end), "hipEventElapsedTime");
}

int accy_hip_device_arch(char* buf, size_t cap) {
  return guarded([&]() -> int {
    if (device_count() <= 0) return fail_with(ACCY_HIP_LAUNCH_FAILED, "no HIP device");
    std::string a = device_arch();
    if (buf && cap) {
      size_t n = std::min(cap - 1, a.size());
      std::memcpy(buf, a.data(), n);
      buf[n] = '\0';
    }
    return ACCY_HIP_OK;
  });
}

}  // extern "C"
