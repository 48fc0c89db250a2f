// Error channel and library metadata for libvdnmi.
#include "common.h"

#include <stdarg.h>
#include <stdio.h>

namespace vdn {

static thread_local char g_last_error[1024] = "";

int set_error(int status, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, args);
  va_end(args);
  return status;
}

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return set_error(kLaunchFailed, "%s: launch failed: %s", what, hipGetErrorString(err));
  }
  return kOk;
}

}  // namespace vdn

VDN_API const char* vdn_last_error(void) { return vdn::g_last_error; }

VDN_API int vdn_abi_version(void) { return 6; }
