// Device scratch of the allocation-free entry point (accy_hip_invoke_device_scratch).
#pragma once

#include <cstddef>
#include <cstdint>

namespace accy {

// Size of the static device array every GPU the library runs on holds: 512 MiB, 0.18 % of an
// MI355X's 288 GB. The largest benchmark program (the full-size C5 decoder block) fits.
constexpr uint64_t kScratchBytes = 512ull << 20;

// The current device's address of the array (looked up with hipGetSymbolAddress on the first call on
// that device, with it current, and kept). Returns 0, or -1 with a message in *error.
int scratch_region(void** ptr, const char** error);

}  // namespace accy
