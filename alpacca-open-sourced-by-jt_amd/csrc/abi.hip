// Version, error reporting and device checks of the C-ABI.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "alpx_common.h"

namespace {
thread_local char g_error[1024] = "";
}

namespace alpx {

int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return status;
}

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return fail(ALPX_EHIP, "%s: kernel launch failed: %s", what, hipGetErrorString(err));
  }
  return ALPX_OK;
}

}  // namespace alpx

extern "C" {

int alpx_abi_version(void) { return ALPX_ABI_VERSION; }

const char* alpx_last_error(void) { return g_error; }

int alpx_device_arch(int device, char* buf, int buf_len) {
  if (buf == nullptr || buf_len <= 0) return alpx::fail(ALPX_EINVAL, "alpx_device_arch: null buffer");
  hipDeviceProp_t prop;
  hipError_t err = hipGetDeviceProperties(&prop, device);
  if (err != hipSuccess) {
    return alpx::fail(ALPX_EHIP, "hipGetDeviceProperties(%d): %s", device, hipGetErrorString(err));
  }
  snprintf(buf, (size_t)buf_len, "%s", prop.gcnArchName);
  return ALPX_OK;
}

}  // extern "C"
