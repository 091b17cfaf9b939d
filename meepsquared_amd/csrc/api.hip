// Library identity and the per-thread error message of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "common.hpp"

namespace mlora {

static thread_local char g_error[1024] = {0};

int fail(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return 1;
}

void clear_error() { g_error[0] = 0; }

int launch_status(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail("%s: launch failed: %s", what, hipGetErrorString(err));
  return 0;
}

}  // namespace mlora

extern "C" const char* mlora_version(void) { return "mlora 0.1 gfx950"; }

extern "C" const char* mlora_last_error(void) { return mlora::g_error; }
