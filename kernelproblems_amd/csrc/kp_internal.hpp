// Host-side helpers shared by the C-ABI entry points (not part of the ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/kp.h"

namespace kp {

// Records a failure for kp_last_error_message() and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Checks hipGetLastError() after a launch; KP_EHIP with the message recorded on failure.
int check_launch(const char* what);
// Number of compute units of the current device (cached per device ordinal).
int cu_count();

// Timing hook (kp_profile_dominant_kernel): record the caller's events right
// before / after the dominant kernel launch of an entry point.
void prof_begin(hipStream_t s);
void prof_end(hipStream_t s);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace kp
