// Error state of the C ABI: one message per calling thread.
#include <stdarg.h>
#include <stdio.h>

#include "klc_common.h"

namespace klc {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return set_error(KLC_ERR_HIP, "%s: %s", what, hipGetErrorString(err));
  return KLC_OK;
}

}  // namespace klc

extern "C" const char* klc_last_error(void) { return klc::g_last_error; }

extern "C" int klc_abi_version(void) { return KLC_ABI_VERSION; }
