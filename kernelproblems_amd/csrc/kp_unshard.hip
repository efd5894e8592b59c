// FSDP parameter unshard: column ranges of a row-strided bf16 flat-buffer view
// copied to contiguous per-parameter outputs, all segments in one launch.
//
// One-shot grid: every block copies one 4 KiB chunk (256 threads x 16 B) of
// one shard row of one segment, the launch shape that streams fastest on
// gfx950.  Chunks are enumerated segment-major, then shard row, then column.
#include "kp_common.hpp"
#include "kp_internal.hpp"

namespace kp {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxSeg = 16;
constexpr int64_t kChunkElems = kThreads * 8;  // bf16 elements per block

struct UnshardArgs {
  const uint16_t* src;
  int64_t shards, stride;
  int n_seg;
  int64_t off[kMaxSeg], len[kMaxSeg], nchunk[kMaxSeg], first_block[kMaxSeg + 1];
  uint16_t* dst[kMaxSeg];
};

template <bool VEC>
__global__ __launch_bounds__(kThreads) void unshard_kernel(UnshardArgs a) {
  const int64_t b = blockIdx.x;
  int s = 0;
  while (s + 1 < a.n_seg && b >= a.first_block[s + 1]) ++s;
  const int64_t local = b - a.first_block[s];
  const int64_t row = local / a.nchunk[s], chunk = local % a.nchunk[s];
  if (row >= a.shards) return;
  const uint16_t* sp = a.src + row * a.stride + a.off[s];
  uint16_t* dp = a.dst[s] + row * a.len[s];
  const int64_t c0 = chunk * kChunkElems;
  if constexpr (VEC) {
    const int64_t c = c0 + (int64_t)threadIdx.x * 8;
    if (c < a.len[s]) st16(dp + c, ld16_stream(sp + c));
  } else {
    for (int64_t c = c0 + threadIdx.x; c < min(a.len[s], c0 + kChunkElems); c += kThreads) dp[c] = sp[c];
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
  a.shards = shards;
  a.stride = shard_stride;
  a.n_seg = n_seg;
  bool vec = aligned16(src) && (shard_stride % 8) == 0;
  int64_t blocks = 0;
  for (int s = 0; s < n_seg; ++s) {
    if (col_off[s] < 0 || col_len[s] < 0 || (col_len[s] > 0 && dst[s] == nullptr))
      return fail(KP_EINVAL, "%s: bad segment %d", who, s);
    if (shards > 1 && col_off[s] + col_len[s] > shard_stride)
      return fail(KP_EINVAL, "%s: segment %d runs past the shard row", who, s);
    a.off[s] = col_off[s];
    a.len[s] = col_len[s];
    a.dst[s] = static_cast<uint16_t*>(dst[s]);
    a.nchunk[s] = ceil_div(col_len[s], kChunkElems);
    a.first_block[s] = blocks;
    blocks += a.nchunk[s] * shards;
    vec = vec && (col_off[s] % 8) == 0 && (col_len[s] % 8) == 0 && aligned16(dst[s]);
  }
  a.first_block[n_seg] = blocks;
  if (blocks == 0) return KP_OK;
  if (blocks > 0x7fffffffLL) return fail(KP_EUNSUPPORTED, "%s: too many blocks", who);
  hipStream_t s = as_stream(stream);
  if (vec) KP_LAUNCH_DOMINANT(unshard_kernel<true>, dim3((unsigned)blocks), dim3(kThreads), 0, s, a);
  else KP_LAUNCH_DOMINANT(unshard_kernel<false>, dim3((unsigned)blocks), dim3(kThreads), 0, s, a);
  return check_launch(who);
}
