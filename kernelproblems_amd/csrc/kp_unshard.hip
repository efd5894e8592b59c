// FSDP parameter unshard: column ranges of a row-strided bf16 flat-buffer view
// copied to contiguous per-parameter outputs, all segments in one launch.
//
// One-shot grid: every block copies one 4 KiB chunk (256 threads x 16 B) of
// one shard row of one segment, the launch shape that streams fastest on
// gfx950.  Chunks are enumerated shard row first, then the segments' chunks
// in row order, so consecutive blocks read one source row front to back.
#include <algorithm>

#include "kp_common.hpp"
#include "kp_internal.hpp"

namespace kp {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxSeg = 16;
constexpr int64_t kChunkElems = kThreads * 8;  // bf16 elements per block

struct UnshardArgs {
  const uint16_t* src;
  int64_t stride;
  Div32 per_row;           // chunks per shard row, over all kept segments
  int32_t first[kMaxSeg];  // first chunk of each segment within a row; INT32_MAX past the last
  int64_t off[kMaxSeg], len[kMaxSeg];
  uint16_t* dst[kMaxSeg];
};

template <bool VEC>
__global__ __launch_bounds__(kThreads) void unshard_kernel(UnshardArgs a) {
  const uint32_t b = blockIdx.x;
  const uint32_t row = div32(b, a.per_row);
  const int32_t cc = (int32_t)(b - row * a.per_row.d);
  // The chunk's segment as a count over fixed argument slots, which the
  // compiler fetches in one batch of scalar loads; a search loop would wait
  // for one load per segment before the block's first data load.
  int s = 0;
  int32_t start = 0;
#pragma unroll
  for (int k = 1; k < kMaxSeg; ++k) {
    const bool in = cc >= a.first[k];
    s = in ? k : s;
    start = in ? a.first[k] : start;
  }
  const uint16_t* sp = a.src + (int64_t)row * a.stride + a.off[s];
  const int64_t len = a.len[s];
  uint16_t* dp = a.dst[s] + (int64_t)row * len;
  const int64_t c0 = (int64_t)(cc - start) * kChunkElems;
  if constexpr (VEC) {
    const int64_t c = c0 + (int64_t)threadIdx.x * 8;
    if (c < len) st16(dp + c, ld16_stream(sp + c));
  } else {
    for (int64_t c = c0 + threadIdx.x; c < min(len, c0 + kChunkElems); c += kThreads) dp[c] = sp[c];
  }
}

}  // namespace
}  // namespace kp

using namespace kp;

extern "C" int kp_unshard_bf16(const void* src, int64_t shards, int64_t shard_stride, const int64_t* col_off,
                               const int64_t* col_len, void* const* dst, int n_seg, void* stream) {
  static const char* who = "kp_unshard_bf16";
  if (n_seg < 0 || n_seg > kMaxSeg) return fail(KP_EINVAL, "%s: 0..%d segments", who, kMaxSeg);
  if (n_seg == 0 || shards == 0) return KP_OK;
  if (src == nullptr || col_off == nullptr || col_len == nullptr || dst == nullptr || shards < 0 || shard_stride < 0)
    return fail(KP_EINVAL, "%s: NULL pointer or negative size", who);
  UnshardArgs a{};
  a.src = static_cast<const uint16_t*>(src);
  a.stride = shard_stride;
  bool vec = aligned16(src) && (shard_stride % 8) == 0;
  int64_t per_row = 0;
  for (int s = 0; s < n_seg; ++s) {
    if (col_off[s] < 0 || col_len[s] < 0 || (col_len[s] > 0 && dst[s] == nullptr))
      return fail(KP_EINVAL, "%s: bad segment %d", who, s);
    if (shards > 1 && col_off[s] + col_len[s] > shard_stride)
      return fail(KP_EINVAL, "%s: segment %d runs past the shard row", who, s);
    a.off[s] = col_off[s];
    a.len[s] = col_len[s];
    a.dst[s] = static_cast<uint16_t*>(dst[s]);
    a.first[s] = (int32_t)std::min<int64_t>(per_row, INT32_MAX);
    per_row += ceil_div(col_len[s], kChunkElems);
    vec = vec && (col_off[s] % 8) == 0 && (col_len[s] % 8) == 0 && aligned16(dst[s]);
  }
  for (int s = n_seg; s < kMaxSeg; ++s) a.first[s] = INT32_MAX;
  if (per_row == 0) return KP_OK;
  // Every block index (row * per_row + chunk) stays below 2^31, which
  // div32 requires.
  if (per_row > 0x7fffffffLL / shards) return fail(KP_EUNSUPPORTED, "%s: too many blocks", who);
  const int64_t blocks = per_row * shards;
  a.per_row = make_div32((uint32_t)per_row);
  hipStream_t s = as_stream(stream);
  if (vec) KP_LAUNCH_DOMINANT(unshard_kernel<true>, dim3((unsigned)blocks), dim3(kThreads), 0, s, a);
  else KP_LAUNCH_DOMINANT(unshard_kernel<false>, dim3((unsigned)blocks), dim3(kThreads), 0, s, a);
  return check_launch(who);
}
