// Streaming-ceiling probe for gfx950: the bandwidth this GPU reaches for a
// given mix of array reads and writes, measured with the same access form
// as the fragment kernels (16-byte accesses, 1 KiB per wave instruction).
// It computes nothing of the hot path; bench.py times it on each workload's
// own byte mix, under every tile size and store policy below, and takes the
// fastest as the streaming ceiling that the workload's kernel is set against.
//
// One-shot grid: block b owns the 16-byte chunks [b * 256 U, (b + 1) * 256 U)
// of every array (256 threads x U chunks, thread t holding chunks t + 256 u),
// so each array is covered exactly once.  Accesses are raw buffer operations
// on one descriptor per array: a load past an input's end returns zeros and a
// store past an output's end is dropped, so arrays of different lengths need
// no branches.  Loads are non-temporal; stores are non-temporal or, with
// KP_STORE_WRITE_THROUGH, device-scope write-through (sc1).  Outputs receive
// the 32-bit lane-wise sum of the inputs plus the output's number in
// component 0 (an index pattern when there are no inputs).  On MI355X one
// chunk per thread streams copy-like mixes fastest, two to four chunks the
// mixes of several reads and writes; write-through stores help write-only
// and small mixes by ~2-5% and cost up to ~3% elsewhere.
#include "kp_common.hpp"
#include "kp_internal.hpp"

namespace kp {
namespace {

constexpr int kThreads = 256;
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int kLoadNT = 2;        // cache policy bits of the loads: nt
constexpr int kStoreNT = 2;       // nt
constexpr int kStoreWT = 16;      // sc1: device-scope write-through

struct ProbeArgs {
  const void* in[4];
  void* out[3];
  uint32_t in_bytes, out_bytes;  // per array; below 2^32 (checked on the host)
};

__device__ __forceinline__ rsrc_t array_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

template <int NR, int NW, int U, int SP>
__global__ __launch_bounds__(kThreads) void stream_probe(ProbeArgs a) {
  const uint32_t c0 = blockIdx.x * (uint32_t)(kThreads * U) + threadIdx.x;  // first chunk of this thread
  u32x4 v[NR > 0 ? NR : 1][U];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const rsrc_t ri = array_rsrc(a.in[r], a.in_bytes);
#pragma unroll
    for (int u = 0; u < U; ++u) v[r][u] = __builtin_amdgcn_raw_buffer_load_b128(ri, (c0 + u * kThreads) * 16u, 0, kLoadNT);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t c = c0 + u * kThreads;
    u32x4 s = NR > 0 ? v[0][u] : u32x4{c, 0u, 0u, 0u};
#pragma unroll
    for (int r = 1; r < NR; ++r) s += v[r][u];
#pragma unroll
    for (int w = 0; w < NW; ++w)
      __builtin_amdgcn_raw_buffer_store_b128(s + u32x4{(uint32_t)w, 0u, 0u, 0u}, array_rsrc(a.out[w], a.out_bytes),
                                             c * 16u, 0, SP == KP_STORE_WRITE_THROUGH ? kStoreWT : kStoreNT);
  }
}

typedef void (*ProbeKernel)(ProbeArgs);

template <int U, int SP>
ProbeKernel probe_kernel_us(int nr, int nw) {
  switch (nr * 10 + nw) {
    case 1: return stream_probe<0, 1, U, SP>;
    case 2: return stream_probe<0, 2, U, SP>;
    case 11: return stream_probe<1, 1, U, SP>;
    case 12: return stream_probe<1, 2, U, SP>;
    case 21: return stream_probe<2, 1, U, SP>;
    case 22: return stream_probe<2, 2, U, SP>;
    case 31: return stream_probe<3, 1, U, SP>;
    case 32: return stream_probe<3, 2, U, SP>;
    case 41: return stream_probe<4, 1, U, SP>;
    case 42: return stream_probe<4, 2, U, SP>;
    case 33: return stream_probe<3, 3, U, SP>;
  }
  return nullptr;
}

template <int SP>
ProbeKernel probe_kernel_s(int nr, int nw, int per_thread) {
  switch (per_thread) {
    case 1: return probe_kernel_us<1, SP>(nr, nw);
    case 2: return probe_kernel_us<2, SP>(nr, nw);
    case 4: return probe_kernel_us<4, SP>(nr, nw);
    case 8: return probe_kernel_us<8, SP>(nr, nw);
  }
  return nullptr;
}

ProbeKernel probe_kernel(int nr, int nw, int per_thread, int store_policy) {
  return store_policy == KP_STORE_WRITE_THROUGH ? probe_kernel_s<KP_STORE_WRITE_THROUGH>(nr, nw, per_thread)
                                                : probe_kernel_s<KP_STORE_NONTEMPORAL>(nr, nw, per_thread);
}

}  // namespace
}  // namespace kp

using namespace kp;

extern "C" {

int kp_stream_probe(const void* const* in, int n_in, int64_t in_bytes, void* const* out, int n_out,
                    int64_t out_bytes, int chunks_per_thread, int store_policy, void* stream) {
  static const char* who = "kp_stream_probe";
  if (n_in < 0 || n_in > 4 || n_out < 1 || n_out > 3 || (n_out == 3 && n_in != 3))
    return fail(KP_EINVAL, "%s: needs 0..4 input and 1..2 output arrays, or 3 and 3", who);
  if (in_bytes < 0 || out_bytes < 0 || (in_bytes & 15) != 0 || (out_bytes & 15) != 0)
    return fail(KP_EINVAL, "%s: array sizes must be non-negative multiples of 16 bytes", who);
  if (n_in > 0 && (in == nullptr)) return fail(KP_EINVAL, "%s: input pointer list is NULL", who);
  if (out == nullptr) return fail(KP_EINVAL, "%s: output pointer list is NULL", who);
  if (chunks_per_thread != 1 && chunks_per_thread != 2 && chunks_per_thread != 4 && chunks_per_thread != 8)
    return fail(KP_EINVAL, "%s: chunks_per_thread must be 1, 2, 4 or 8", who);
  if (store_policy != KP_STORE_NONTEMPORAL && store_policy != KP_STORE_WRITE_THROUGH)
    return fail(KP_EINVAL, "%s: unknown store policy %d", who, store_policy);
  ProbeArgs a{};
  for (int i = 0; i < n_in; ++i) {
    if (in[i] == nullptr || !aligned16(in[i])) return fail(KP_EINVAL, "%s: input %d is NULL or not 16-byte aligned", who, i);
    a.in[i] = in[i];
  }
  for (int i = 0; i < n_out; ++i) {
    if (out[i] == nullptr || !aligned16(out[i]))
      return fail(KP_EINVAL, "%s: output %d is NULL or not 16-byte aligned", who, i);
    a.out[i] = out[i];
  }
  const int64_t span = in_bytes > out_bytes ? in_bytes : out_bytes;
  const int64_t tile_bytes = (int64_t)kThreads * chunks_per_thread * 16;
  // every buffer offset of the grid (up to one tile past the longer array) fits 32 bits
  if (span + tile_bytes > 0xffffffffLL) return fail(KP_EUNSUPPORTED, "%s: arrays of 4 GiB or more", who);
  a.in_bytes = (uint32_t)(n_in > 0 ? in_bytes : 0);
  a.out_bytes = (uint32_t)out_bytes;
  if (span == 0) return KP_OK;
  const int64_t blocks = ceil_div(span, tile_bytes);
  void* args[] = {&a};
  launch_dominant_raw(reinterpret_cast<const void*>(probe_kernel(n_in, n_out, chunks_per_thread, store_policy)),
                      dim3((unsigned)blocks), dim3(kThreads), args, 0, as_stream(stream));
  return check_launch(who);
}

}  // extern "C"
