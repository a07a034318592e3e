// Library-level entry points of libkf950: version, error reporting, device check.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "kf_common.h"

static thread_local char g_last_error[512] = "";

extern "C" __attribute__((visibility("hidden"))) void kf_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

extern "C" int kf_abi_version(void) { return KF_ABI_VERSION; }

extern "C" const char* kf_last_error(void) { return g_last_error; }

extern "C" int kf_device_ok(int device) {
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) {
    kf_set_error("kf_device_ok: %s", hipGetErrorString(e));
    return -(int)e;
  }
  return strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

// Compute units of the current device, cached per device ordinal (grid sizing of the
// persistent and grid-stride kernels).
namespace kf {
int cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}
}  // namespace kf
