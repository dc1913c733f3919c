// static_scratch.hip -- the fixed device workspace behind the decode entry
// point that allocates nothing (osm_moe_layer_decode_device_static).
//
// The workspace is a file-scope device array: every GPU the library runs on
// holds its own copy, at its own address, from the first use of the module
// until the process ends. Its name is only a host-side stand-in for that
// memory, so host code never passes it to a kernel or a copy: the address is
// looked up once per device with hipGetSymbolAddress (with that device
// current, at context creation) and kept here, and callers use that address.
#include <hip/hip_runtime.h>

#include <mutex>

#include "osm_device.h"

namespace {

__device__ __align__(256) unsigned char scratch[OSMD_STATIC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_addr[kMaxDevices] = {};

}  // namespace

extern "C" {

int osmd_static_scratch_init(int device) {
  if (device < 0 || device >= kMaxDevices) return static_cast<int>(hipErrorInvalidDevice);
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_addr[device] != nullptr) return 0;
  int current = -1;
  hipError_t e = hipGetDevice(&current);
  if (e != hipSuccess) return static_cast<int>(e);
  if (current != device) return static_cast<int>(hipErrorInvalidDevice);
  void* p = nullptr;
  e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return static_cast<int>(e);
  if (p == nullptr) return static_cast<int>(hipErrorInvalidSymbol);
  g_addr[device] = p;
  return 0;
}

int osmd_static_scratch(int device, void** out) {
  if (out == nullptr) return static_cast<int>(hipErrorInvalidValue);
  *out = nullptr;
  if (device < 0 || device >= kMaxDevices) return static_cast<int>(hipErrorInvalidDevice);
  {
    std::lock_guard<std::mutex> lock(g_mu);
    *out = g_addr[device];
  }
  if (*out != nullptr) return 0;
  // Not looked up at context creation (it failed there): once more, now.
  const int rc = osmd_static_scratch_init(device);
  if (rc != 0) return rc;
  std::lock_guard<std::mutex> lock(g_mu);
  *out = g_addr[device];
  return 0;
}

}  // extern "C"
