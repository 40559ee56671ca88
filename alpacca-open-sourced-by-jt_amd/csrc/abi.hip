// Version, error reporting and device checks of the C-ABI.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>

#include "alpx_common.h"

namespace {
thread_local char g_error[1024] = "";

// Kernel-choice overrides: taken from the environment once, when the
// library loads, then changed only by alpx_set_override.
std::atomic<int> g_override[ALPX_OVERRIDES];
constexpr int kOverrideMax[ALPX_OVERRIDES] = {1, 1, 3, 1, 1};

struct OverridesFromEnvironment {
  OverridesFromEnvironment() {
    g_override[ALPX_OVERRIDE_DECODE_GENERIC] = getenv("ALPX_DECODE_GENERIC") != nullptr;
    g_override[ALPX_OVERRIDE_PREFILL_GENERIC] = getenv("ALPX_PREFILL_GENERIC") != nullptr;
    g_override[ALPX_OVERRIDE_GDN_SEQUENTIAL] = getenv("ALPX_GDN_SEQUENTIAL") != nullptr;
    g_override[ALPX_OVERRIDE_RECURRENT_UNFUSED] = getenv("ALPX_RECURRENT_UNFUSED") != nullptr;
    const char* k = getenv("ALPX_PREFILL_KERNEL");
    int kernel = 0;
    if (k != nullptr && strcmp(k, "single") == 0) kernel = 1;
    if (k != nullptr && strcmp(k, "pair") == 0) kernel = 2;
    if (k != nullptr && strcmp(k, "shared") == 0) kernel = 3;
    g_override[ALPX_OVERRIDE_PREFILL_KERNEL] = kernel;
  }
} g_overrides_from_environment;
}  // namespace

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

int override_value(int which) {
  return which >= 0 && which < ALPX_OVERRIDES ? g_override[which].load(std::memory_order_relaxed)
                                              : 0;
}

int multiprocessor_count() {
  static thread_local int cached_device = -1, cached = 0;
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) device = 0;
  if (device != cached_device) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
        cus <= 0)
      cus = 256;
    cached_device = device;
    cached = cus;
  }
  return cached;
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
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block, lds) != hipSuccess ||
      per_cu <= 0)
    per_cu = 1;
  const int value = per_cu * multiprocessor_count();
  if (used < 32) cache[used++] = {kernel, device, value};
  return value;
}

}  // namespace alpx

extern "C" {

int alpx_abi_version(void) { return ALPX_ABI_VERSION; }

const char* alpx_last_error(void) { return g_error; }

int alpx_set_override(int which, int value) {
  if (which < 0 || which >= ALPX_OVERRIDES)
    return alpx::fail(ALPX_EINVAL, "alpx_set_override: unknown override %d", which);
  if (value < 0 || value > kOverrideMax[which])
    return alpx::fail(ALPX_EINVAL, "alpx_set_override: value %d out of range for override %d",
                      value, which);
  return g_override[which].exchange(value);
}

int alpx_get_override(int which) {
  if (which < 0 || which >= ALPX_OVERRIDES)
    return alpx::fail(ALPX_EINVAL, "alpx_get_override: unknown override %d", which);
  return g_override[which].load();
}

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

int alpx_host_device_pointer(void* host, void** device_pointer) {
  if (host == nullptr || device_pointer == nullptr)
    return alpx::fail(ALPX_EINVAL, "alpx_host_device_pointer: null pointer");
  void* dev = nullptr;
  hipError_t err = hipHostGetDevicePointer(&dev, host, 0);
  if (err != hipSuccess || dev == nullptr) {
    (void)hipGetLastError();  // leave no sticky error for the caller's next HIP call
    return alpx::fail(ALPX_EINVAL, "alpx_host_device_pointer: %p is not page-locked HIP host "
                                   "memory (%s)", host, hipGetErrorString(err));
  }
  *device_pointer = dev;
  return ALPX_OK;
}

}  // extern "C"
