// Library-wide entry points: ABI version and the thread-local error channel.
#include <stdarg.h>
#include <stdio.h>

#include "tk_common.hpp"

namespace {
thread_local char g_last_error[512] = "";
}

namespace tk {

int fail(const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, args);
  va_end(args);
  return 1;
}

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail("%s: launch failed: %s", what, hipGetErrorString(err));
  return 0;
}

}  // namespace tk

extern "C" int tk_abi_version(void) { return TK_ABI_VERSION; }

extern "C" const char* tk_last_error(void) { return g_last_error; }
