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
}  // namespace smel

#define SMEL_REQUIRE(cond, code, ...)  \
  do {                                 \
    if (!(cond)) {                     \
      smel::set_error(__VA_ARGS__);    \
      return (code);                   \
    }                                  \
  } while (0)
