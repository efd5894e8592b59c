// Streaming-ceiling probe for gfx950: the bandwidth this GPU reaches for a
// given mix of array reads and writes, measured with the same access form
// as the fragment kernels (16-byte non-temporal loads and stores, 1 KiB per
// wave instruction).  It computes nothing of the hot path; bench.py times it
// on each workload's own buffers so that every kernel's rate can be set
// against what plain streaming of the same bytes achieves.
//
// One-shot grid: block b owns the 16-byte chunks [b * 256 U, (b + 1) * 256 U)
// of every array (256 threads x U chunks, thread t holding chunks t + 256 u),
// so each array is covered exactly once.  U = 1 or 4: on MI355X one chunk per
// thread streams a 1:1 copy ~8% faster than four, while mixes of several
// reads per write prefer four -- the caller times both.  Outputs receive the
// 32-bit lane-wise sum of the inputs (an index pattern when there are none).
#include "kp_common.hpp"
#include "kp_internal.hpp"

namespace kp {
namespace {

constexpr int kThreads = 256;

struct ProbeArgs {
  const u32x4* in[4];
  u32x4* out[3];
  int64_t in_chunks, out_chunks;  // 16-byte chunks per input / per output array
};

template <int NR, int NW, int kPerThread>
__global__ __launch_bounds__(kThreads) void stream_probe(ProbeArgs a) {
  const int64_t base = (int64_t)blockIdx.x * kThreads * kPerThread + threadIdx.x;
  u32x4 v[NR > 0 ? NR : 1][kPerThread];
#pragma unroll
  for (int r = 0; r < NR; ++r)
#pragma unroll
    for (int u = 0; u < kPerThread; ++u) {
      const int64_t i = base + (int64_t)u * kThreads;
      v[r][u] = i < a.in_chunks ? ld16_stream(a.in[r] + i) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
  for (int u = 0; u < kPerThread; ++u) {
    const int64_t i = base + (int64_t)u * kThreads;
    u32x4 s = NR > 0 ? v[0][u] : u32x4{(uint32_t)i, 0u, 0u, 0u};
#pragma unroll
    for (int r = 1; r < NR; ++r) s += v[r][u];
#pragma unroll
    for (int w = 0; w < NW; ++w)
      if (i < a.out_chunks) st16_stream(a.out[w] + i, s + u32x4{(uint32_t)w, 0u, 0u, 0u});
  }
}

typedef void (*ProbeKernel)(ProbeArgs);

template <int U>
ProbeKernel probe_kernel_u(int nr, int nw) {
  switch (nr * 10 + nw) {
    case 1: return stream_probe<0, 1, U>;
    case 2: return stream_probe<0, 2, U>;
    case 11: return stream_probe<1, 1, U>;
    case 12: return stream_probe<1, 2, U>;
    case 21: return stream_probe<2, 1, U>;
    case 22: return stream_probe<2, 2, U>;
    case 31: return stream_probe<3, 1, U>;
    case 32: return stream_probe<3, 2, U>;
    case 41: return stream_probe<4, 1, U>;
    case 42: return stream_probe<4, 2, U>;
    case 33: return stream_probe<3, 3, U>;
  }
  return nullptr;
}

ProbeKernel probe_kernel(int nr, int nw, int per_thread) {
  return per_thread == 1 ? probe_kernel_u<1>(nr, nw) : probe_kernel_u<4>(nr, nw);
}

}  // namespace
}  // namespace kp

using namespace kp;

extern "C" {

int kp_stream_probe(const void* const* in, int n_in, int64_t in_bytes, void* const* out, int n_out,
                    int64_t out_bytes, int chunks_per_thread, void* stream) {
  static const char* who = "kp_stream_probe";
  if (n_in < 0 || n_in > 4 || n_out < 1 || n_out > 3 || (n_out == 3 && n_in != 3))
    return fail(KP_EINVAL, "%s: needs 0..4 input and 1..2 output arrays, or 3 and 3", who);
  if (in_bytes < 0 || out_bytes < 0 || (in_bytes & 15) != 0 || (out_bytes & 15) != 0)
    return fail(KP_EINVAL, "%s: array sizes must be non-negative multiples of 16 bytes", who);
  if (n_in > 0 && (in == nullptr)) return fail(KP_EINVAL, "%s: input pointer list is NULL", who);
  if (out == nullptr) return fail(KP_EINVAL, "%s: output pointer list is NULL", who);
  if (chunks_per_thread != 1 && chunks_per_thread != 4)
    return fail(KP_EINVAL, "%s: chunks_per_thread must be 1 or 4", who);
  ProbeArgs a{};
  for (int i = 0; i < n_in; ++i) {
    if (in[i] == nullptr || !aligned16(in[i])) return fail(KP_EINVAL, "%s: input %d is NULL or not 16-byte aligned", who, i);
    a.in[i] = static_cast<const u32x4*>(in[i]);
  }
  for (int i = 0; i < n_out; ++i) {
    if (out[i] == nullptr || !aligned16(out[i]))
      return fail(KP_EINVAL, "%s: output %d is NULL or not 16-byte aligned", who, i);
    a.out[i] = static_cast<u32x4*>(out[i]);
  }
  a.in_chunks = n_in > 0 ? in_bytes / 16 : 0;
  a.out_chunks = out_bytes / 16;
  const int64_t chunks = a.in_chunks > a.out_chunks ? a.in_chunks : a.out_chunks;
  if (chunks == 0) return KP_OK;
  const int64_t blocks = ceil_div(chunks, (int64_t)kThreads * chunks_per_thread);
  if (blocks > 0x7fffffffLL) return fail(KP_EUNSUPPORTED, "%s: arrays too large for one launch", who);
  void* args[] = {&a};
  launch_dominant_raw(reinterpret_cast<const void*>(probe_kernel(n_in, n_out, chunks_per_thread)), dim3((unsigned)blocks),
                      dim3(kThreads), args, 0, as_stream(stream));
  return check_launch(who);
}

}  // extern "C"
