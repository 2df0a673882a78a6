// abi_util.h - error reporting shared by the C-ABI entry points.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>

namespace pcamd {

// Records a formatted, thread-local message for pcamd_last_error() and
// returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();
// hipGetLastError() after a launch; PCAMD_ERR_LAUNCH with the HIP message.
int check_launch(const char* what);
// Device the stream belongs to (the current device for the null stream);
// -1 if the query fails.
int stream_device(hipStream_t st);
// Compute units of the stream's device (cached per device; 0 if the query fails).
int device_cu_count(hipStream_t st);
// Raises kern's dynamic-LDS limit to `bytes` on the stream's device, once per
// device: `done` is the caller's per-kernel bit set of devices already set up
// (one bit per device ordinal below 64). The attribute call runs with the
// stream's device current and restores the caller's device afterwards.
int ensure_dynamic_lds(const void* kern, int bytes, hipStream_t st, std::atomic<uint64_t>& done);

}  // namespace pcamd
