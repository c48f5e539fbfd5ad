// Host helpers shared by the launcher entry points of libggemm_vark.so.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <cstring>

#include "../../include/ggemm_vark.h"

namespace ggemm {
namespace host {

constexpr int kMaxDevices = 64;

// per-device cache: 0 = unknown, -1 = unusable, >0 = CU count of a gfx950 device
inline std::atomic<int> g_cus[kMaxDevices];

// CU count of the current device (the persistent grid size), or an error code when it is not a
// gfx950 device.
inline int device_cus(int* cus_out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return GGEMM_E_DEVICE;
  int c = g_cus[dev].load(std::memory_order_relaxed);
  if (c == 0) {
    hipDeviceProp_t p;
    e = hipGetDeviceProperties(&p, dev);
    if (e != hipSuccess) return (int)e;
    c = (std::strncmp(p.gcnArchName, "gfx950", 6) == 0 && p.multiProcessorCount > 0) ? p.multiProcessorCount : -1;
    g_cus[dev].store(c, std::memory_order_relaxed);
  }
  if (c < 0) return GGEMM_E_DEVICE;
  *cus_out = c;
  return GGEMM_OK;
}

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

}  // namespace host
}  // namespace ggemm
