// Error reporting and device-property cache behind the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include <atomic>

#include "kp_internal.hpp"

namespace kp {

namespace {
thread_local int t_last_hip = 0;
thread_local char t_msg[512] = "";
thread_local hipEvent_t t_prof_start = nullptr;
thread_local hipEvent_t t_prof_stop = nullptr;
thread_local void* t_trace_buf = nullptr;
thread_local size_t t_trace_bytes = 0;

constexpr int kMaxDevices = 64;
std::atomic<int> g_cu_count[kMaxDevices];
}  // namespace

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(t_msg, sizeof(t_msg), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) return KP_OK;
  t_last_hip = static_cast<int>(e);
  return fail(KP_EHIP, "%s: %s", what, hipGetErrorString(e));
}

hipEvent_t prof_start_event() { return t_prof_start; }
hipEvent_t prof_stop_event() { return t_prof_stop; }
unsigned long long* block_trace_buf() { return static_cast<unsigned long long*>(t_trace_buf); }
int block_trace_blocks() {
  const size_t n = t_trace_bytes / (kBlockTraceWords * sizeof(unsigned long long));
  return n > 0x7fffffff ? 0x7fffffff : (int)n;
}

void launch_dominant_raw(const void* fn, dim3 grid, dim3 block, void** args, size_t shmem, hipStream_t s) {
  if (t_prof_start && t_prof_stop)
    (void)hipExtLaunchKernel(fn, grid, block, args, shmem, s, t_prof_start, t_prof_stop, 0);
  else
    (void)hipLaunchKernel(fn, grid, block, args, shmem, s);
}

int cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  int n = g_cu_count[dev].load(std::memory_order_relaxed);
  if (n > 0) return n;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
  g_cu_count[dev].store(n, std::memory_order_relaxed);
  return n;
}

}  // namespace kp

extern "C" {

const char* kp_version(void) { return "kernelproblems_amd 0.1.0 (gfx950)"; }
int kp_last_hip_error(void) { return kp::t_last_hip; }
const char* kp_last_error_message(void) { return kp::t_msg; }
void kp_debug_block_trace(void* buf, size_t bytes) {
  kp::t_trace_buf = bytes >= kp::kBlockTraceWords * sizeof(unsigned long long) ? buf : nullptr;
  kp::t_trace_bytes = kp::t_trace_buf ? bytes : 0;
}

void kp_profile_dominant_kernel(void* start_event, void* stop_event) {
  kp::t_prof_start = reinterpret_cast<hipEvent_t>(start_event);
  kp::t_prof_stop = reinterpret_cast<hipEvent_t>(stop_event);
}

}  // extern "C"
