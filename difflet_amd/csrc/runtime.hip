// Library identity and error reporting for the C ABI.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "common.hpp"

#ifndef DIFFLET_ROCM_VERSION
#define DIFFLET_ROCM_VERSION "0.1.0"
#endif

static thread_local char g_err[512] = "";

void dlt_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int dlt_check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    dlt_set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return DIFFLET_ELAUNCH;
  }
  return DIFFLET_OK;
}

extern "C" const char* difflet_rocm_last_error(void) { return g_err; }

extern "C" const char* difflet_rocm_version(void) {
  return "difflet-rocm " DIFFLET_ROCM_VERSION " (gfx950)";
}

extern "C" int difflet_rocm_abi_version(void) { return 7; }

extern "C" int difflet_rocm_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  int found = 0;
  for (int i = 0; i < n; ++i) {
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, i) == hipSuccess && strncmp(p.gcnArchName, "gfx950", 6) == 0)
      ++found;
  }
  return found;
}
