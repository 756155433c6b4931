// Library identity and error reporting for the C ABI.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "common.h"

namespace {
thread_local char g_last_error[512] = "";

__global__ void arch_probe_kernel(int* out) {
#if defined(__gfx950__)
  if (threadIdx.x == 0) out[0] = 950;
#else
  if (threadIdx.x == 0) out[0] = -1;
#endif
}
}  // namespace

int forge_set_error(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}

extern "C" const char* forge_version(void) { return "forge-hip 0.1 (gfx950)"; }

extern "C" const char* forge_last_error(void) { return g_last_error; }

// 1 when the current device is a gfx950 and this library's code object for
// it loads (the probe kernel's attributes resolve on that device); 0 when no
// device is visible, the device is another architecture, or the fat binary
// has no gfx950 image.
extern "C" int forge_arch_ok(void) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) {
    (void)hipGetLastError();
    return 0;
  }
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, dev) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) return 0;
  hipFuncAttributes attr;
  if (hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&arch_probe_kernel)) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return 1;
}
