// Error reporting, library metadata and the per-device CU count (the only
// state the library keeps) for the EntmaxKV C ABI.
#include <stdarg.h>
#include <stdio.h>

#include <atomic>

#include "ekv_common.h"
#include "../../include/entmaxkv.h"

namespace {
thread_local char g_err[512] = "";
}

namespace ekv {

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v > 0) return v;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    cus = 256;
  cache[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(EKV_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return EKV_OK;
}

}  // namespace ekv

extern "C" const char* ekv_last_error(void) { return g_err; }

extern "C" int ekv_abi_version(void) { return EKV_ABI_VERSION; }

#ifndef EKV_BUILD_ID
#define EKV_BUILD_ID "unknown"
#endif

extern "C" const char* ekv_build_id(void) { return EKV_BUILD_ID; }
