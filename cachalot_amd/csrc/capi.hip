// Library identity and the thread-local error channel of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace cachalot {

static thread_local char g_last_error[1024] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(CACHALOT_EHIP, "%s: %s", what, hipGetErrorString(e));
  return CACHALOT_OK;
}

}  // namespace cachalot

extern "C" int cachalot_version(void) { return 1; }

extern "C" const char* cachalot_last_error(void) { return cachalot::g_last_error; }
