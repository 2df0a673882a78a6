// abi.hip - version and error reporting of the C ABI (include/pcamd_fp8.h).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>

#include "abi_util.h"
#include "fp8_common.h"

namespace pcamd {

static thread_local char g_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_error[0] = '\0'; }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(PCAMD_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  return PCAMD_OK;
}

}  // namespace pcamd

extern "C" int pcamd_abi_version(void) { return PCAMD_ABI_VERSION; }
extern "C" const char* pcamd_last_error(void) { return pcamd::g_error; }
