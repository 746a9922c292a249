// Library-wide entry points: ABI version and the thread-local error string.
#include <stdarg.h>
#include <stdio.h>

#include "nf_device.h"

namespace {
thread_local char g_last_error[512] = "";
}

namespace nf {

int set_error(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char *what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(NF_ERR_LAUNCH, "%s: kernel launch failed: %s", what,
                     hipGetErrorString(e));
  return NF_OK;
}

}  // namespace nf

extern "C" int nf_abi_version(void) { return NF_ABI_VERSION; }

extern "C" const char *nf_last_error(void) { return g_last_error; }
