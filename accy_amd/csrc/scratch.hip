// Device scratch for allocation-free invocations (accy_hip_invoke_device_scratch): one file-scope
// device array that the HIP runtime places on every GPU this library's code object is loaded on, held
// until the process ends. Host code never passes the array's name to a kernel or a copy (in host code
// it is only a stand-in for the symbol); it uses the address hipGetSymbolAddress returns for the
// current device, looked up once per device and kept.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>

#include "scratch.hpp"

namespace {

__device__ __align__(256) static unsigned char scratch[accy::kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

}  // namespace

namespace accy {

int scratch_region(void** ptr, const char** error) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    *error = "hipGetDevice failed";
    return -1;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    *error = "device ordinal beyond the scratch table";
    return -1;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t rc = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (rc != hipSuccess || !p) {
      *error = hipGetErrorString(rc);
      return -1;
    }
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return 0;
}

}  // namespace accy
