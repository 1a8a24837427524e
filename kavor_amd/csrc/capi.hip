// Error channel and version of libkvpath.so (see include/kvpath.h).
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace kvp {

static thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_last_error[0] = '\0'; }

int launch_status(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    fail(static_cast<int>(err), "%s: launch failed: %s", what, hipGetErrorString(err));
    return static_cast<int>(err);
  }
  return KVP_OK;
}

}  // namespace kvp

extern "C" const char* kvp_last_error(void) { return kvp::g_last_error; }

extern "C" const char* kvp_version(void) { return "kvpath 0.1 gfx950"; }
