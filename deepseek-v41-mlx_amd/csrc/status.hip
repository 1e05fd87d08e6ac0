// Library identification and the thread-local last-error message of the C ABI.
#include <stdarg.h>
#include <string.h>

#include "common.h"

namespace dsv41 {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error((int)e, "%s: launch failed: %s", what, hipGetErrorString(e));
  g_last_error[0] = '\0';
  return 0;
}

}  // namespace dsv41

extern "C" const char* dsv41_version(void) { return "dsv41 0.1 gfx950"; }

extern "C" const char* dsv41_last_error_string(void) { return dsv41::g_last_error; }
