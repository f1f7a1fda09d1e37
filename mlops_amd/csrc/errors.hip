// Error reporting of the C ABI: one thread-local message per host thread.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

static thread_local char g_last_error[512] = "";

void mi355x_set_error(const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, args);
  va_end(args);
}

extern "C" const char* mi355x_last_error(void) { return g_last_error; }

extern "C" int mi355x_abi_version(void) { return 1; }
