// Error reporting of the C-ABI (smel_moe.h).
#include <stdarg.h>
#include <stdio.h>

#include "abi_util.h"

namespace {
thread_local char g_msg[512] = "";
}

namespace smel {
void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_msg, sizeof(g_msg), fmt, ap);
  va_end(ap);
}
}  // namespace smel

extern "C" const char* smel_last_error(void) { return g_msg; }
extern "C" int smel_abi_version(void) { return 23; }
