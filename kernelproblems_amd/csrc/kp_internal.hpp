// Host-side helpers shared by the C-ABI entry points (not part of the ABI).
#pragma once

#include <hip/hip_ext.h>
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

// Timing hook (kp_profile_dominant_kernel): the caller's events, or nullptr.
hipEvent_t prof_start_event();
hipEvent_t prof_stop_event();

// Block timeline hook (kp_debug_block_trace): the caller's buffer, or nullptr,
// and how many blocks' records (kBlockTraceWords 64-bit words each) it holds.
constexpr int kBlockTraceWords = 4;
unsigned long long* block_trace_buf();
int block_trace_blocks();

// Launches an entry point's dominant kernel.  With timing events set, the
// launch goes through hipExtLaunchKernel, which stamps the events at the
// kernel's own start and completion, so they time that kernel alone.
void launch_dominant_raw(const void* fn, dim3 grid, dim3 block, void** args, size_t shmem, hipStream_t s);

// Sums P fp32 weight-gradient partial rows (the row kernels' layout,
// [ceil(N / 16)][P][16]) into dw in a fixed order (kp_rmsnorm.hip), for
// other row passes that write the same partial rows.
int rms_dw_finalize_launch(const float* partial, int P, int64_t N, float* dw_f32, uint16_t* dw_bf16, int round_f32,
                           hipStream_t s, const char* who);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace kp

// The first / last launch of a multi-launch pipeline whose whole span is
// timed: the start event is stamped at the first kernel's start, the stop
// event at the last kernel's completion (kp_profile_dominant_kernel).
#define KP_LAUNCH_SPAN(first, last, kernel, grid, block, shmem, stream, ...)                            \
  do {                                                                                                  \
    hipEvent_t kp_ev_a_ = ::kp::prof_start_event(), kp_ev_b_ = ::kp::prof_stop_event();               \
    if (kp_ev_a_ && kp_ev_b_)                                                                           \
      hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream, (first) ? kp_ev_a_ : nullptr,          \
                            (last) ? kp_ev_b_ : nullptr, 0, __VA_ARGS__);                               \
    else                                                                                                \
      hipLaunchKernelGGL(kernel, grid, block, shmem, stream, __VA_ARGS__);                              \
  } while (0)

#define KP_LAUNCH_DOMINANT(kernel, grid, block, shmem, stream, ...)                                       \
  do {                                                                                                  \
    hipEvent_t kp_ev_a_ = ::kp::prof_start_event(), kp_ev_b_ = ::kp::prof_stop_event();               \
    if (kp_ev_a_ && kp_ev_b_)                                                                           \
      hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream, kp_ev_a_, kp_ev_b_, 0, __VA_ARGS__);    \
    else                                                                                                \
      hipLaunchKernelGGL(kernel, grid, block, shmem, stream, __VA_ARGS__);                              \
  } while (0)
