// Error reporting and ABI version of the sid C-ABI library.
#include "common.h"

#include <cstring>

namespace sid {

static thread_local char g_last_error[512] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(err));
    return SID_ERR_LAUNCH;
  }
  return SID_OK;
}

}  // namespace sid

extern "C" const char* sid_last_error(void) { return sid::g_last_error; }

extern "C" int sid_abi_version(void) { return 22; }
