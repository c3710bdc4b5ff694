// Thread-local error reporting for the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "../../include/longspark_amd.h"

namespace ls {

static thread_local char g_last_error[512] = "";

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

}  // namespace ls

extern "C" const char* ls_last_error(void) { return ls::g_last_error; }
extern "C" const char* ls_version(void) { return "longspark_amd 0.1.0 gfx950"; }
