// Error reporting and library metadata for the EntmaxKV C ABI.
#include <stdarg.h>
#include <stdio.h>

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

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(EKV_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return EKV_OK;
}

}  // namespace ekv

extern "C" const char* ekv_last_error(void) { return g_err; }

extern "C" int ekv_abi_version(void) { return EKV_ABI_VERSION; }
