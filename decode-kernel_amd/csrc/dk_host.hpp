// Host-side helpers shared by the C-ABI translation units.
#pragma once

#include <hip/hip_runtime_api.h>

namespace dk {

// Record a formatted message for dk_last_error() on this thread; returns code.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// DK_ERR_HIP with the runtime's message for `e`.
int hip_error(hipError_t e, const char* what);

// DK_OK, or DK_ERR_HIP if the last launch on this thread failed.
int check_launch(const char* what);

}  // namespace dk
