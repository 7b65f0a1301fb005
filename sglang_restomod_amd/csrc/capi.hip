// Library-wide C-ABI entry points: version and the per-thread last error.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>

#include "capi_internal.h"

namespace {
thread_local char g_last_error[512] = "";
}

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

extern "C" const char* ma_last_error(void) { return g_last_error; }

extern "C" int ma_abi_version(void) { return MA_ABI_VERSION; }

extern "C" int ma_device_arch(char* buf, int len) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return set_error(MA_ELAUNCH, "hipGetDevice failed");
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return set_error(MA_ELAUNCH, "hipGetDeviceProperties failed");
  if (buf && len > 0) snprintf(buf, (size_t)len, "%s", prop.gcnArchName);
  return MA_OK;
}
