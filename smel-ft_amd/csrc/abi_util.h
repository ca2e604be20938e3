// Host-side argument checking and error reporting shared by the C-ABI entry points.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/smel_moe.h"

namespace smel {
void set_error(const char* fmt, ...);

// Returns hipGetLastError() of the launch just made as the entry point's result.
inline int launch_status() {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("kernel launch failed: %s", hipGetErrorString(e));
    return (int)e;
  }
  return 0;
}

// Compute units of the current device, queried once per device (the grid of the persistent kernels).
inline int cu_count() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}
}  // namespace smel

#define SMEL_REQUIRE(cond, code, ...)  \
  do {                                 \
    if (!(cond)) {                     \
      smel::set_error(__VA_ARGS__);    \
      return (code);                   \
    }                                  \
  } while (0)
