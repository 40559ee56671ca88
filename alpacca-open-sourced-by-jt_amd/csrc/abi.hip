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

int resident_blocks(const void* kernel, int block, size_t lds) {
  struct Entry {
    const void* kernel;
    int device;
    int value;
  };
  static thread_local Entry cache[32];
  static thread_local int used = 0;
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) device = 0;
  for (int i = 0; i < used; ++i)
    if (cache[i].kernel == kernel && cache[i].device == device) return cache[i].value;
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block, lds) != hipSuccess ||
      per_cu <= 0)
    per_cu = 1;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
      cus <= 0)
    cus = 256;
  const int value = per_cu * cus;
  if (used < 32) cache[used++] = {kernel, device, value};
  return value;
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
