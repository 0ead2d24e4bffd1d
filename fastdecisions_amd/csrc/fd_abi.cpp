// Error reporting and version entry points of the C ABI (include/fd_kernels.h).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>

#include "../../include/fd_kernels.h"

namespace {
thread_local char g_last_error[512] = "";
}

int fd_set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int fd_check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return fd_set_error(FD_ERR_LAUNCH, "%s: kernel launch failed: %s (%d)", what, hipGetErrorString(err),
                        static_cast<int>(err));
  }
  return FD_OK;
}

extern "C" int fd_abi_version(void) { return FD_ABI_VERSION; }

extern "C" const char* fd_last_error(void) { return g_last_error; }
