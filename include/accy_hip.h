/* accy_hip.h — C ABI of the MI355X (gfx950) execution target for Accy tensor programs.
 *
 * A program crosses this boundary as ACTP v1 wire bytes, the language-neutral encoding the
 * reference writes with `tensor.wire.encode` (src/tensor/wire/encode.zig:28-230) and reads with
 * `tensor.wire.decode` (src/tensor/wire/decode.zig:31-120). Inputs and outputs are dense row-major
 * byte slices in the program's parameter / output order, each exactly its slot's size, as for
 * `tensor.runCpu` (src/tensor/execute.zig:54-63; src/executable/binding.zig:127).
 *
 * Every function returns a status number with the reference session's meanings
 * (src/tensor/session/session.zig:33-43). Invocations on one handle are not thread-safe with
 * respect to each other; the handle table itself is locked, and a release on another thread while
 * an invocation runs retires the handle (later calls get ACCY_HIP_INVALID_HANDLE) but frees the
 * program only when that invocation has returned.
 */
#ifndef ACCY_HIP_H
#define ACCY_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status numbers: src/tensor/session/session.zig:33-43. */
enum {
  ACCY_HIP_OK = 0,
  ACCY_HIP_INVALID_PROGRAM = 1,
  ACCY_HIP_UNSUPPORTED_VERSION = 2,
  ACCY_HIP_INVALID_HANDLE = 3,
  ACCY_HIP_INVALID_BUFFER = 4,
  ACCY_HIP_TOO_MANY_PROGRAMS = 5,
  ACCY_HIP_OUT_OF_MEMORY = 6,   /* also: a program with a value over 1 TiB (more than a device holds),
                                   refused when it is decoded */
  ACCY_HIP_COMPILE_FAILED = 7,
  ACCY_HIP_LAUNCH_FAILED = 8
};

/* At most this many programs are compiled at once (session.zig:16). */
#define ACCY_HIP_MAX_PROGRAMS 64

/* Slot index and generation; release bumps the generation so stale copies are refused
 * (session.zig:58-64). */
typedef struct {
  uint32_t index;
  uint32_t generation;
} accy_hip_handle;

/* One input or output (session.zig:66-74). `dtype` uses the wire dtype codes
 * (src/tensor/wire/format.zig:97-99: i1=0 … f16=9, bf16=10, f32=11, f64=12, key=13).
 * `alignment` is max(element size, 16): the 16-byte minimum accy_hip_invoke_device checks, as the
 * reference reports max(slot alignment, backend minimum) (session.zig:278-284).
 * `names` and `extents` stay valid until the program is released. */
typedef struct {
  uint32_t dtype;
  uint32_t rank;
  const char* const* names;
  const int64_t* extents;
  uint64_t byte_size;
  uint32_t alignment;
} accy_hip_descriptor;

/* One kernel of a compiled program, for measurement. While profiling is on, every invocation
 * records HIP events around each kernel on its launch stream without synchronising; reading the
 * stats waits for them. `last_ms` is the latest invocation, `mean_ms` the mean over the `calls`
 * invocations recorded since profiling was turned on (the latest 256). */
typedef struct {
  const char* label;
  const char* klass;
  double algorithmic_bytes;
  double algorithmic_flops;
  float last_ms;
  float mean_ms;
  uint32_t calls;
} accy_hip_kernel_stats;

/* One-shot run: compile, copy inputs in, launch, copy outputs out, release.
 * Replaces `tensor.runCpu(allocator, program, inputs, outputs)` (src/tensor/execute.zig:54-63). */
int accy_hip_run(const uint8_t* wire, size_t wire_len, const void* const* inputs, const size_t* input_lens,
                 size_t n_inputs, void* const* outputs, const size_t* output_lens, size_t n_outputs);

/* Compile once, launch many: `Cpu.init` (execute.zig:14-35) and `Session.compile`
 * (session.zig:120-161). */
int accy_hip_compile(const uint8_t* wire, size_t wire_len, accy_hip_handle* out);

/* Numbers of inputs and outputs of a compiled program. */
int accy_hip_counts(accy_hip_handle h, size_t* n_inputs, size_t* n_outputs);

/* `Session.inputDescriptors` / `outputDescriptors` (session.zig:163-171): which = 0 for inputs,
 * 1 for outputs. An index past the end returns ACCY_HIP_INVALID_BUFFER. */
int accy_hip_describe(accy_hip_handle h, int which, size_t index, accy_hip_descriptor* out);

/* `Cpu.launch` (execute.zig:44-51) / `Session.invoke` (session.zig:180-210) on host memory.
 * Counts or sizes that do not match the descriptors, and outputs that overlap an input or another
 * output, return ACCY_HIP_INVALID_BUFFER. Synchronous. */
int accy_hip_invoke(accy_hip_handle h, const void* const* inputs, const size_t* input_lens, size_t n_inputs,
                    void* const* outputs, const size_t* output_lens, size_t n_outputs);

/* The same launch on device memory already resident in HBM: `inputs` / `outputs` are device
 * pointers sized by the descriptors, and the work is enqueued on `stream` (a hipStream_t; NULL is
 * the null stream) without synchronising. Borrowed in place as `binding.prepareBorrowed` does
 * (src/executable/binding.zig:138-200), which refuses a slice below the backend's minimum
 * alignment: here 16 bytes (hipMalloc's pointers are 256-byte aligned); a misaligned pointer, a
 * count that does not match, or an output whose descriptor-sized range overlaps an input or an earlier
 * output (binding.zig:325-336) returns ACCY_HIP_INVALID_BUFFER before anything is launched. */
int accy_hip_invoke_device(accy_hip_handle h, const void* const* inputs, size_t n_inputs, void* const* outputs,
                           size_t n_outputs, void* stream);

/* No counterpart in the reference. For callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc): accy_hip_invoke_device with
 * every intermediate buffer of the run (temporaries between kernels, chunked-fold partials, scan
 * carries) placed in one static device array of 512 MiB that each GPU the library runs on holds until
 * the process ends. The call itself calls no hipMalloc / hipFree and records no profiling events;
 * accy_hip_compile, which the caller runs beforehand, still allocates the executor's own buffers
 * (constants, and the intermediates that accy_hip_invoke_device uses) and looks up the array's address
 * on the current device. A program whose intermediates need more than 512 MiB returns
 * ACCY_HIP_OUT_OF_MEMORY before anything is launched. Every call on one GPU uses the same array and
 * leaves the last call's contents in it (each kernel writes an intermediate in full before it is
 * read, so nothing needs clearing): calls that overlap on one GPU, on any streams, race. */
int accy_hip_invoke_device_scratch(accy_hip_handle h, const void* const* inputs, size_t n_inputs,
                                   void* const* outputs, size_t n_outputs, void* stream);

/* `Cpu.deinit` / `Session.release` (session.zig:216-226). */
int accy_hip_release(accy_hip_handle h);

/* Why the last failing call on this thread failed (`Session.last_cause`, session.zig:88-97). */
const char* accy_hip_last_error(void);

/* Per-kernel timing with HIP events recorded on the launch stream (the counterpart of
 * `FragmentInstrumentation`, src/executable/phase.zig:3-56). */
int accy_hip_set_profiling(accy_hip_handle h, int enable);
int accy_hip_kernel_count(accy_hip_handle h, size_t* n);
int accy_hip_kernel_info(accy_hip_handle h, size_t index, accy_hip_kernel_stats* out);

/* Host-only: lowers a program without a device and writes the generated HIP sources (NUL-terminated)
 * into `buf`; `*needed` receives the full length + 1. With `compile` set, each kernel is also
 * compiled for gfx950 with hiprtc, so a CPU-only host can check that the program builds. */
int accy_hip_plan_source(const uint8_t* wire, size_t wire_len, int compile, char* buf, size_t cap, size_t* needed);

/* Name of the current HIP device's architecture (e.g. "gfx950:sramecc+:xnack-"). */
int accy_hip_device_arch(char* buf, size_t cap);

/* Launch tuning, the gfx950 counterpart of the reference's launch-tuning cache
 * (src/executable/tuning.zig:9-289: candidate measurements, one selection per kernel key,
 * `selectionForKernel`; :291-468 the artifact's encoding).
 * A tunable kernel (a row kernel's element-loop unroll, a 16-bit contraction's N tile) has a few
 * launch candidates with bit-identical results; compile and plan_source take the selection recorded
 * for the kernel's key in the process-wide table (loaded from $ACCY_TUNING_FILE on first use when
 * set), else the default.
 * accy_hip_tune: compiles every candidate plan of `wire`, runs each on the device buffers given (as
 * accy_hip_invoke_device; outputs are overwritten), requires every candidate's outputs to equal the
 * default's byte for byte (else ACCY_HIP_COMPILE_FAILED), times `repeats` invocations per candidate
 * and records the fastest per kernel; `*n_tuned` = kernels recorded.
 * accy_hip_tuning_export: writes the table as an artifact ("ACTT", version 1) into `buf` when `cap`
 * is large enough; `*needed` = its size. accy_hip_tuning_import: merges an artifact (a record replaces
 * one of the same key only when faster); a bad magic, version or record leaves the table unchanged
 * and returns ACCY_HIP_INVALID_PROGRAM or ACCY_HIP_UNSUPPORTED_VERSION. */
int accy_hip_tune(const uint8_t* wire, size_t wire_len, const void* const* inputs, size_t n_inputs,
                  void* const* outputs, size_t n_outputs, uint32_t repeats, size_t* n_tuned);
int accy_hip_tuning_export(uint8_t* buf, size_t cap, size_t* needed);
int accy_hip_tuning_import(const uint8_t* data, size_t len);
int accy_hip_tuning_count(size_t* n);
int accy_hip_tuning_clear(void);

/* Device memory, streams and events of the runtime this library is linked against, for callers
 * that keep inputs and outputs resident in HBM (the buffer half of the backend vtable:
 * allocate_buffer / write_buffer / read_buffer / synchronize / destroy_object,
 * deps/lib/compiler/gpu/src/contract.zig:2048-2084). `kind`: 1 host to device, 2 device to host,
 * 3 device to device. All streams are created at the default priority. */
int accy_hip_malloc(void** ptr, size_t bytes);
int accy_hip_free(void* ptr);
int accy_hip_memcpy(void* dst, const void* src, size_t bytes, int kind);
int accy_hip_stream_create(void** stream);
int accy_hip_stream_destroy(void* stream);
int accy_hip_stream_synchronize(void* stream);
int accy_hip_event_create(void** event);
int accy_hip_event_destroy(void* event);
int accy_hip_event_record(void* event, void* stream);
int accy_hip_event_elapsed_ms(float* ms, void* start, void* end);

#ifdef __cplusplus
}
#endif

#endif /* ACCY_HIP_H */
