// libmxgg: version, error reporting and device gate of the C ABI (include/mxgg.h).
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "mxgg_host.h"

namespace mxgg {

static thread_local char g_err[512];

void clear_error() { g_err[0] = 0; }

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    fail((int)e, "%s: launch failed: %s", what, hipGetErrorString(e));
    return (int)e;
  }
  return MXGG_OK;
}

// Per-device cache of "is gfx950" (devices are few; 64 covers any node).
static int g_dev_ok[64];  // 0 unknown, 1 yes, 2 no

int require_device() {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(MXGG_ERR_NO_DEVICE, "no HIP device: %s", hipGetErrorString(e));
  if (dev >= 0 && dev < 64 && g_dev_ok[dev]) {
    return g_dev_ok[dev] == 1 ? MXGG_OK
                              : fail(MXGG_ERR_NO_DEVICE, "device %d is not gfx950", dev);
  }
  hipDeviceProp_t p;
  e = hipGetDeviceProperties(&p, dev);
  if (e != hipSuccess) return fail(MXGG_ERR_NO_DEVICE, "hipGetDeviceProperties: %s", hipGetErrorString(e));
  bool ok = strncmp(p.gcnArchName, "gfx950", 6) == 0;
  if (dev >= 0 && dev < 64) g_dev_ok[dev] = ok ? 1 : 2;
  return ok ? MXGG_OK : fail(MXGG_ERR_NO_DEVICE, "device %d is %s, not gfx950", dev, p.gcnArchName);
}

}  // namespace mxgg

extern "C" int mxgg_version(void) { return MXGG_VERSION; }

extern "C" const char* mxgg_last_error_string(void) { return mxgg::g_err; }

extern "C" int mxgg_device_supported(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
    (void)hipGetLastError();
    return 0;
  }
  return mxgg::require_device() == MXGG_OK ? 1 : 0;
}
