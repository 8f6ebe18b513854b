// Error state and version of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "../../include/noise_amd.h"

static thread_local char g_error[1024] = "";

int noise_set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

extern "C" const char* noise_last_error(void) { return g_error; }

extern "C" int noise_abi_version(void) { return 1; }
