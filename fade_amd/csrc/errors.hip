// Error reporting for the C ABI: one message buffer per calling thread.
#include <stdarg.h>
#include <stdio.h>

#include "fade_common.h"

namespace fade {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int einval(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return FADE_EINVAL;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return FADE_ERUNTIME;
  }
  return FADE_OK;
}

}  // namespace fade

FADE_API int fade_hip_abi_version(void) { return FADE_ABI_VERSION; }

FADE_API const char* fade_hip_last_error(void) { return fade::g_last_error; }
