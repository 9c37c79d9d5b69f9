// Error reporting and version query shared by every libdsa entry point.
#include "dsa_common.h"

#include <string.h>

namespace {
thread_local char g_error[512] = {0};
}

namespace dsa {

int set_error(int code, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, args);
  va_end(args);
  return code;
}

void clear_error() { g_error[0] = '\0'; }

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess)
    return set_error(DSA_ELAUNCH, "%s: launch failed: %s", what, hipGetErrorString(err));
  return DSA_OK;
}

}  // namespace dsa

extern "C" const char* dsa_last_error(void) { return g_error; }

extern "C" int dsa_version(void) { return 1; }
