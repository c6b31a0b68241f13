// Launch tuning for gfx950: the measured launch candidate of each tunable kernel, keyed by the
// device family and the kernel's signature, kept in a process-wide table and persisted as a small
// binary artifact (src/executable/tuning.zig:173-289 is the reference's cache: candidate
// measurements, a selection per key, import / export of records; :291-468 its artifact).
//
// A tunable kernel offers a few launch candidates that compute bit-identical results (a row kernel's
// element-loop unroll, a contraction's N tile); candidate 0 is the planner's default. The planner
// asks the table for a key's selection; `tune` (runtime) measures every candidate and records the
// fastest.
#pragma once
#include <cstddef>
#include <cstdint>
#include <map>
#include <mutex>
#include <optional>
#include <string>
#include <utility>
#include <vector>

#include "ir.hpp"

namespace accy {

struct TuningSelection {
  uint32_t candidate = 0;
  uint64_t mean_ns = 0;  // mean duration of the selected candidate over `samples` invocations
  uint32_t samples = 0;  // invocations measured
};

class TuningTable {
 public:
  // The selection recorded for a kernel key with this many candidates, if any.
  std::optional<TuningSelection> find(const std::string& key, uint32_t candidate_count) const;
  // Keeps the faster of the recorded and the new selection (tuning.zig:251-268).
  void record(const std::string& key, uint32_t candidate_count, const TuningSelection& s);
  // Artifact: "ACTT" magic, u32 version, u32 record count, then per record u32 key length, key
  // bytes, u32 candidate count, u32 candidate, u64 mean ns, u32 samples (all little-endian),
  // records sorted by key.
  std::vector<uint8_t> encode() const;
  // Merges an artifact's records (each kept only where it beats the table's); all or nothing.
  // Throws accy::Error: BadMagic, UnsupportedVersion, or InvalidArtifact (truncation, trailing bytes,
  // a candidate out of range, zero samples, an empty key).
  void merge(const uint8_t* data, size_t len);
  size_t size() const;
  void clear();

  static constexpr uint32_t kMagic = 0x54544341u;  // "ACTT"
  static constexpr uint32_t kVersion = 1;

 private:
  mutable std::mutex mu_;
  std::map<std::pair<std::string, uint32_t>, TuningSelection> sel_;
};

// The table that compile and plan consult (loaded from $ACCY_TUNING_FILE on first use when set).
TuningTable& process_tuning();

// Measures every launch candidate of the program's tunable kernels on device buffers (the inputs
// resident, as for accy_hip_invoke_device), `repeats` invocations per candidate interleaved across
// candidates, and records the fastest candidate per kernel key in `table`. Every candidate's outputs
// must equal candidate 0's byte for byte (else Error(Unsupported)). Returns the kernels recorded.
size_t tune_program(const Program& program, const void* const* inputs, size_t n_inputs, void* const* outputs,
                    size_t n_outputs, uint32_t repeats, TuningTable& table);

// 64-bit FNV-1a of a string, as 16 hex digits (kernel signatures in keys).
std::string fingerprint(const std::string& s);

}  // namespace accy
