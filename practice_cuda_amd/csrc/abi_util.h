// abi_util.h - error reporting shared by the C-ABI entry points.
#pragma once

#include <hip/hip_runtime.h>

namespace pcamd {

// Records a formatted, thread-local message for pcamd_last_error() and
// returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();
// hipGetLastError() after a launch; PCAMD_ERR_LAUNCH with the HIP message.
int check_launch(const char* what);
// Compute units of the current device (cached per device; 0 if the query fails).
int device_cu_count();

}  // namespace pcamd
