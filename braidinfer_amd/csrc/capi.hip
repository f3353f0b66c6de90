// Library-wide C ABI: version and per-thread error text.
#include <stdarg.h>
#include <stdio.h>

#include "bfa_host.h"

namespace bfa {

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
  if (e != hipSuccess) {
    return set_error(BFA_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  }
  return BFA_OK;
}

}  // namespace bfa

extern "C" int bfa_abi_version(void) { return BFA_ABI_VERSION; }

extern "C" const char* bfa_last_error(void) { return bfa::g_last_error; }
