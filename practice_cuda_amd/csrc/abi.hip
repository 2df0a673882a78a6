// abi.hip - version and error reporting of the C ABI (include/pcamd_fp8.h).
#include <hip/hip_runtime.h>

#include <atomic>
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

int device_cu_count() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cache[kMaxDevices];  // 0: not queried yet
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  const bool cached = dev >= 0 && dev < kMaxDevices;
  if (cached) {
    const int c = cache[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (cached && n > 0) cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

}  // namespace pcamd

extern "C" int pcamd_abi_version(void) { return PCAMD_ABI_VERSION; }
extern "C" const char* pcamd_last_error(void) { return pcamd::g_error; }
