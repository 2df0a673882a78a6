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

int stream_device(hipStream_t st) {
  int dev = -1;
  if (st == nullptr) return hipGetDevice(&dev) == hipSuccess ? dev : -1;
  return hipStreamGetDevice(st, &dev) == hipSuccess ? dev : -1;
}

int device_cu_count(hipStream_t st) {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cache[kMaxDevices];  // 0: not queried yet
  const int dev = stream_device(st);
  if (dev < 0) return 0;
  const bool cached = dev < kMaxDevices;
  if (cached) {
    const int c = cache[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (cached && n > 0) cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

int ensure_dynamic_lds(const void* kern, int bytes, hipStream_t st, std::atomic<uint64_t>& done) {
  const int dev = stream_device(st);
  if (dev < 0) return set_error(PCAMD_ERR_LAUNCH, "cannot determine the stream's device");
  const uint64_t bit = dev < 64 ? uint64_t{1} << dev : 0;
  if (bit && (done.load(std::memory_order_acquire) & bit)) return PCAMD_OK;
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess) return set_error(PCAMD_ERR_LAUNCH, "hipGetDevice failed");
  if (cur != dev && hipSetDevice(dev) != hipSuccess)
    return set_error(PCAMD_ERR_LAUNCH, "hipSetDevice(%d) failed", dev);
  const hipError_t e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (cur != dev) (void)hipSetDevice(cur);
  if (e != hipSuccess) return set_error(PCAMD_ERR_LAUNCH, "hipFuncSetAttribute: %s", hipGetErrorString(e));
  // concurrent first calls may both set the attribute: the call is idempotent
  if (bit) done.fetch_or(bit, std::memory_order_acq_rel);
  return PCAMD_OK;
}

}  // namespace pcamd

extern "C" int pcamd_abi_version(void) { return PCAMD_ABI_VERSION; }
extern "C" const char* pcamd_last_error(void) { return pcamd::g_error; }
