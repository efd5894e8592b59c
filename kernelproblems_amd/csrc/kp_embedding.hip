// Embedding gather (forward) and deterministic dense scatter-add (backward) for gfx950.
//
// Forward: one wave64 per token row, 16-byte vector copies (1 KiB per wave
// instruction).  Table rows are read with ordinary (cacheable) loads because
// Zipf-distributed ids hit the same rows repeatedly; output rows are written
// with non-temporal stores.
//
// Backward pipeline (five launches on one stream, no float atomics):
//   K1 emb_sort_chunks : keys (id << tbits | t) of each 2048-token chunk are
//                        bitonic-sorted in LDS.  Padding / out-of-range ids get
//                        the sentinel key and sort last.
//   K2 emb_merge_rank  : rank of a key = its index in its chunk + the number of
//                        smaller keys in every other chunk (binary search);
//                        the key is scattered to that rank.  Keys are unique,
//                        so the global order is fully determined.
//   K3 emb_plan        : one block walks the sorted keys, finds id segments,
//                        splits segments into runs of kRun tokens ("parts"),
//                        builds the work lists, the touched-row bitmap and
//                        resets the work-queue counter.
//   K4 emb_dense       : persistent blocks pull work items from the queue:
//                        a part sums its run of grad rows in ascending t (fp32)
//                        and writes the output row (single-part segment) or an
//                        fp32 partial row; a zero item writes the untouched
//                        rows of a kZeroRows vocab range as zeros.
//   K5 emb_combine     : segments with several parts add their partial rows in
//                        part order and write the output row.
// Every output row is written exactly once.
#include "kp_common.hpp"
#include "kp_internal.hpp"

namespace kp {
namespace {

constexpr int kThreads = 256;
constexpr int kChunk = 2048;  // keys per K1 block (256 threads x 8)
constexpr int kRun = 32;      // tokens per part
constexpr int kZeroRows = 16; // vocab rows per zero-fill item
constexpr int kPlanThreads = 1024;
constexpr uint32_t kSentinel = 0xffffffffu;

__device__ __forceinline__ int64_t load_index(const void* idx, int ib, int64_t t) {
  return ib == 8 ? static_cast<const int64_t*>(idx)[t] : (int64_t) static_cast<const int32_t*>(idx)[t];
}

// =============================================================== forward
struct EmbFwdArgs {
  const uint16_t* table;
  int64_t V, D, trs;
  const void* idx;
  int ib;
  int64_t T;
  uint16_t* out;
  int64_t ors;
  int32_t* err;
};

template <bool VEC>
__global__ __launch_bounds__(kThreads) void emb_fwd(EmbFwdArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t w0 = (int64_t)blockIdx.x * (kThreads / 64) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t nw = (int64_t)gridDim.x * (kThreads / 64);
  for (int64_t t = w0; t < a.T; t += nw) {
    const int64_t id = load_index(a.idx, a.ib, t);
    const bool ok = id >= 0 && id < a.V;
    if (!ok && lane == 0 && a.err) *a.err = 1;
    const uint16_t* src = a.table + (ok ? id : 0) * a.trs;
    uint16_t* dst = a.out + t * a.ors;
    if constexpr (VEC) {
      constexpr int U = 8;
      for (int64_t c0 = 0; c0 < a.D; c0 += 512 * U) {
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int64_t c = c0 + (int64_t)(u * 64 + lane) * 8;
          v[u] = (ok && c < a.D) ? ld16(src + c) : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int64_t c = c0 + (int64_t)(u * 64 + lane) * 8;
          if (c < a.D) st16_stream(dst + c, v[u]);
        }
      }
    } else {
      for (int64_t c = lane; c < a.D; c += 64) dst[c] = ok ? src[c] : (uint16_t)0;
    }
  }
}

// =============================================================== backward
struct EmbHeader {
  int32_t n_valid;  // tokens that contribute (id in range, != padding_idx)
  int32_t n_seg;    // distinct contributing ids
  int32_t n_items;  // parts (segment runs)
  int32_t n_multi;  // segments with more than one part
  int32_t queue;    // K4 work-queue counter
  int32_t pad[3];
};

struct EmbBwdArgs {
  const uint16_t* grad;
  int64_t grs;
  const void* idx;
  int ib;
  int64_t T, V, D, padding_idx;
  int scale;       // scale_grad_by_freq
  void* out;
  int out_bf16;
  int round_bf16;
  int tbits;
  int nchunks;
  int32_t* err;
  // workspace views
  EmbHeader* hdr;
  uint32_t* keys_chunk;  // [nchunks * kChunk]
  uint32_t* keys;        // [T] globally sorted valid keys
  int32_t* chunk_valid;  // [nchunks]
  int32_t* seg_id;       // [T]
  int32_t* seg_start;    // [T + 1]
  int32_t* part_base;    // [T] first partial slot of a multi-part segment (-1 otherwise)
  int32_t* item_seg;     // [max_items]
  int32_t* item_part;    // [max_items]
  int32_t* multi;        // [max_multi]
  uint32_t* bitmap;      // [ceil(V / 32)]
  float* partials;       // [max_partials, D]
};

// ---- K1: sort each chunk of keys (bitonic, ascending) --------------------
__global__ __launch_bounds__(kThreads) void emb_sort_chunks(EmbBwdArgs a) {
  __shared__ uint32_t s[kChunk];
  const int tid = threadIdx.x;
  const int64_t base = (int64_t)blockIdx.x * kChunk;
  for (int i = tid; i < kChunk; i += kThreads) {
    const int64_t t = base + i;
    uint32_t key = kSentinel;
    if (t < a.T) {
      const int64_t id = load_index(a.idx, a.ib, t);
      const bool in_range = id >= 0 && id < a.V;
      if (!in_range && a.err) *a.err = 1;
      if (in_range && id != a.padding_idx) key = ((uint32_t)id << a.tbits) | (uint32_t)t;
    }
    s[i] = key;
  }
  for (int k = 2; k <= kChunk; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      __syncthreads();
      const int lj = __builtin_ctz(j);
#pragma unroll
      for (int r = 0; r < kChunk / 2 / kThreads; ++r) {
        const int p = r * kThreads + tid;  // pair index
        const int i = ((p >> lj) << (lj + 1)) | (p & (j - 1));
        const int l = i | j;
        const uint32_t x = s[i], y = s[l];
        const bool up = (i & k) == 0;
        if ((x > y) == up) {
          s[i] = y;
          s[l] = x;
        }
      }
    }
  }
  __syncthreads();
  for (int i = tid; i < kChunk; i += kThreads) a.keys_chunk[base + i] = s[i];
}

// number of entries < key in the ascending array v[0..n)
__device__ __forceinline__ int lower_bound_u32(const uint32_t* v, int n, uint32_t key) {
  int lo = 0, hi = n;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (v[mid] < key) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

// ---- K2: global rank of every valid key ---------------------------------
// All sorted chunks are staged in LDS when they fit (dynamic LDS), else read
// from global memory.
template <bool IN_LDS>
__global__ __launch_bounds__(kThreads) void emb_merge_rank(EmbBwdArgs a) {
  extern __shared__ uint32_t lds_keys[];
  const int c = blockIdx.x;
  const int total = a.nchunks * kChunk;
  const uint32_t* keys = a.keys_chunk;
  if constexpr (IN_LDS) {
    for (int i = threadIdx.x; i < total; i += kThreads) lds_keys[i] = a.keys_chunk[i];
    __syncthreads();
    keys = lds_keys;
  }
  const uint32_t* mine = keys + (int64_t)c * kChunk;
  if (threadIdx.x == 0) a.chunk_valid[c] = lower_bound_u32(mine, kChunk, kSentinel);
  for (int i = threadIdx.x; i < kChunk; i += kThreads) {
    const uint32_t key = mine[i];
    if (key == kSentinel) continue;
    int rank = i;
    for (int o = 0; o < a.nchunks; ++o)
      if (o != c) rank += lower_bound_u32(keys + (int64_t)o * kChunk, kChunk, key);
    if (rank < a.T) a.keys[rank] = key;  // always true for unique keys; bounds the store regardless
  }
}

// Exclusive scan of one int per thread over the 1024-thread block; returns the
// block total through *total.  `buf` holds 1024 + 16 ints of LDS.
__device__ __forceinline__ int block_exclusive_scan(int v, int* buf, int* total) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // inclusive scan within the wave (Hillis-Steele over lanes)
  int x = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(x, d, 64);
    if (lane >= d) x += y;
  }
  int* wsum = buf + kPlanThreads;
  if (lane == 63) wsum[wave] = x;
  __syncthreads();
  if (tid == 0) {
    int run = 0;
    for (int w = 0; w < kPlanThreads / 64; ++w) {
      const int t = wsum[w];
      wsum[w] = run;
      run += t;
    }
    buf[0] = run;
  }
  __syncthreads();
  const int res = x - v + wsum[wave];
  *total = buf[0];
  __syncthreads();
  return res;
}

// ---- K3: segments, parts, work lists, bitmap (one block) -----------------
__global__ __launch_bounds__(kPlanThreads) void emb_plan(EmbBwdArgs a) {
  __shared__ int buf[kPlanThreads + 16];
  __shared__ int carry[4];
  const int tid = threadIdx.x;

  // bitmap := 0 (rows set below, after a barrier)
  const int64_t nwords = (a.V + 31) / 32;
  for (int64_t w = tid; w < nwords; w += kPlanThreads) a.bitmap[w] = 0u;

  int n_valid = 0;
  for (int c = 0; c < a.nchunks; ++c) n_valid += a.chunk_valid[c];

  // Pass 1: segment heads -> seg_id / seg_start.
  if (tid == 0) carry[0] = 0;
  __syncthreads();
  for (int base = 0; base < n_valid; base += kPlanThreads) {
    const int i = base + tid;
    int head = 0;
    uint32_t id = 0;
    if (i < n_valid) {
      id = a.keys[i] >> a.tbits;
      head = (i == 0) || ((a.keys[i - 1] >> a.tbits) != id);
    }
    int tot;
    const int off = block_exclusive_scan(head, buf, &tot);
    const int c0 = carry[0];
    if (head) {
      a.seg_id[c0 + off] = (int32_t)id;
      a.seg_start[c0 + off] = i;
    }
    __syncthreads();
    if (tid == 0) carry[0] = c0 + tot;
    __syncthreads();
  }
  const int n_seg = carry[0];
  if (tid == 0) a.seg_start[n_seg] = n_valid;
  __threadfence_block();
  __syncthreads();

  // Bitmap words of touched rows: the first segment falling in a 32-row word
  // gathers the bits of all segments in that word and stores the word (plain
  // stores only; ordered after the zeroing above by the block barriers).
  for (int s = tid; s < n_seg; s += kPlanThreads) {
    const uint32_t w = (uint32_t)a.seg_id[s] >> 5;
    if (s > 0 && ((uint32_t)a.seg_id[s - 1] >> 5) == w) continue;
    uint32_t bits = 0u;
    for (int q = s; q < n_seg; ++q) {
      const uint32_t iq = (uint32_t)a.seg_id[q];
      if ((iq >> 5) != w) break;
      bits |= 1u << (iq & 31);
    }
    a.bitmap[w] = bits;
  }

  // Pass 2: parts per segment -> items, multi list, partial slots.
  if (tid == 0) {
    carry[0] = 0;  // items
    carry[1] = 0;  // multi segments
    carry[2] = 0;  // partial slots
  }
  __syncthreads();
  for (int base = 0; base < n_seg; base += kPlanThreads) {
    const int s = base + tid;
    int nparts = 0;
    if (s < n_seg) {
      const int len = a.seg_start[s + 1] - a.seg_start[s];
      nparts = (len + kRun - 1) / kRun;
    }
    const int is_multi = nparts > 1;
    int t_items, t_multi, t_slots;
    const int o_items = block_exclusive_scan(nparts, buf, &t_items);
    const int o_multi = block_exclusive_scan(is_multi, buf, &t_multi);
    const int o_slots = block_exclusive_scan(is_multi ? nparts : 0, buf, &t_slots);
    const int c_items = carry[0], c_multi = carry[1], c_slots = carry[2];
    if (s < n_seg) {
      for (int p = 0; p < nparts; ++p) {
        a.item_seg[c_items + o_items + p] = s;
        a.item_part[c_items + o_items + p] = p;
      }
      a.part_base[s] = is_multi ? c_slots + o_slots : -1;
      if (is_multi) a.multi[c_multi + o_multi] = s;
    }
    __syncthreads();
    if (tid == 0) {
      carry[0] = c_items + t_items;
      carry[1] = c_multi + t_multi;
      carry[2] = c_slots + t_slots;
    }
    __syncthreads();
  }
  if (tid == 0) {
    a.hdr->n_valid = n_valid;
    a.hdr->n_seg = n_seg;
    a.hdr->n_items = carry[0];
    a.hdr->n_multi = carry[1];
    a.hdr->queue = 0;
  }
}

// Stores 8 consecutive output values (fp32 or bf16) at column c of row r.
__device__ __forceinline__ void store_out8(const EmbBwdArgs& a, int64_t r, int64_t c, const float* v) {
  if (a.out_bf16) {
    st16_stream(static_cast<uint16_t*>(a.out) + r * a.D + c, pack8(v));
  } else {
    float* o = static_cast<float*>(a.out) + r * a.D + c;
    if (a.round_bf16) {
      float q[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) q[e] = round_bf(v[e]);
      st16f_stream(o, f32x4{q[0], q[1], q[2], q[3]});
      st16f_stream(o + 4, f32x4{q[4], q[5], q[6], q[7]});
    } else {
      st16f_stream(o, f32x4{v[0], v[1], v[2], v[3]});
      st16f_stream(o + 4, f32x4{v[4], v[5], v[6], v[7]});
    }
  }
}
__device__ __forceinline__ void store_out1(const EmbBwdArgs& a, int64_t r, int64_t c, float v) {
  if (a.out_bf16) {
    static_cast<uint16_t*>(a.out)[r * a.D + c] = f_to_bf(v);
  } else {
    static_cast<float*>(a.out)[r * a.D + c] = a.round_bf16 ? round_bf(v) : v;
  }
}

// ---- K4: parts and zero-fill, pulled from a work queue --------------------
template <bool VEC>
__device__ void emb_do_part(const EmbBwdArgs& a, int item) {
  const int s = a.item_seg[item];
  const int p = a.item_part[item];
  const int s0 = a.seg_start[s], s1 = a.seg_start[s + 1];
  const int j0 = s0 + p * kRun;
  const int j1 = min(s1, j0 + kRun);
  const int64_t row = a.seg_id[s];
  const int pb = a.part_base[s];
  const float cnt = (float)(s1 - s0);
  const uint32_t tmask = (1u << a.tbits) - 1u;
  if constexpr (VEC) {
    for (int64_t c = (int64_t)threadIdx.x * 8; c < a.D; c += kThreads * 8) {
      float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      int j = j0;
      for (; j + 4 <= j1; j += 4) {
        u32x4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int64_t t = a.keys[j + u] & tmask;
          v[u] = ld16_stream(a.grad + t * a.grs + c);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          float f[8];
          unpack8(v[u], f);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[e] += a.scale ? f[e] / cnt : f[e];
        }
      }
      for (; j < j1; ++j) {
        const int64_t t = a.keys[j] & tmask;
        float f[8];
        unpack8(ld16_stream(a.grad + t * a.grs + c), f);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] += a.scale ? f[e] / cnt : f[e];
      }
      if (pb < 0) {
        store_out8(a, row, c, acc);
      } else {
        float* o = a.partials + (int64_t)(pb + p) * a.D + c;
        *reinterpret_cast<f32x4*>(o) = f32x4{acc[0], acc[1], acc[2], acc[3]};
        *reinterpret_cast<f32x4*>(o + 4) = f32x4{acc[4], acc[5], acc[6], acc[7]};
      }
    }
  } else {
    for (int64_t c = threadIdx.x; c < a.D; c += kThreads) {
      float acc = 0.f;
      for (int j = j0; j < j1; ++j) {
        const int64_t t = a.keys[j] & tmask;
        const float f = bf_to_f(a.grad[t * a.grs + c]);
        acc += a.scale ? f / cnt : f;
      }
      if (pb < 0) store_out1(a, row, c, acc);
      else a.partials[(int64_t)(pb + p) * a.D + c] = acc;
    }
  }
}

template <bool VEC>
__device__ void emb_do_zero(const EmbBwdArgs& a, int64_t z) {
  const int64_t r0 = z * kZeroRows;
  const int64_t r1 = min(a.V, r0 + kZeroRows);
  for (int64_t r = r0; r < r1; ++r) {
    const uint32_t word = a.bitmap[r >> 5];
    if ((word >> (r & 31)) & 1u) continue;
    if constexpr (VEC) {
      const float zeros[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      for (int64_t c = (int64_t)threadIdx.x * 8; c < a.D; c += kThreads * 8) store_out8(a, r, c, zeros);
    } else {
      for (int64_t c = threadIdx.x; c < a.D; c += kThreads) store_out1(a, r, c, 0.f);
    }
  }
}

template <bool VEC>
__global__ __launch_bounds__(kThreads) void emb_dense(EmbBwdArgs a) {
  __shared__ int s_item;
  const int n_items = a.hdr->n_items;
  const int64_t n_zero = (a.V + kZeroRows - 1) / kZeroRows;
  const int64_t total = (int64_t)n_items + n_zero;
  for (;;) {
    if (threadIdx.x == 0) s_item = atomicAdd(&a.hdr->queue, 1);
    __syncthreads();
    const int64_t item = s_item;
    __syncthreads();
    if (item >= total) break;
    if (item < n_items) emb_do_part<VEC>(a, (int)item);
    else emb_do_zero<VEC>(a, item - n_items);
  }
}

// ---- K5: multi-part segments: partial rows added in part order -----------
template <bool VEC>
__global__ __launch_bounds__(kThreads) void emb_combine(EmbBwdArgs a) {
  const int n_multi = a.hdr->n_multi;
  constexpr int kCols = kThreads * 8;
  const int64_t nq = (a.D + kCols - 1) / kCols;
  for (int64_t it = blockIdx.x; it < (int64_t)n_multi * nq; it += gridDim.x) {
    const int s = a.multi[it / nq];
    const int64_t q = it % nq;
    const int len = a.seg_start[s + 1] - a.seg_start[s];
    const int nparts = (len + kRun - 1) / kRun;
    const int pb = a.part_base[s];
    const int64_t row = a.seg_id[s];
    if constexpr (VEC) {
      const int64_t c = q * kCols + (int64_t)threadIdx.x * 8;
      if (c < a.D) {
        float acc[8];
        const float* p0 = a.partials + (int64_t)pb * a.D + c;
        f32x4 u = *reinterpret_cast<const f32x4*>(p0), v = *reinterpret_cast<const f32x4*>(p0 + 4);
        for (int e = 0; e < 4; ++e) {
          acc[e] = u[e];
          acc[4 + e] = v[e];
        }
        for (int p = 1; p < nparts; ++p) {
          const float* pp = a.partials + (int64_t)(pb + p) * a.D + c;
          u = *reinterpret_cast<const f32x4*>(pp);
          v = *reinterpret_cast<const f32x4*>(pp + 4);
          for (int e = 0; e < 4; ++e) {
            acc[e] += u[e];
            acc[4 + e] += v[e];
          }
        }
        store_out8(a, row, c, acc);
      }
    } else {
      for (int64_t c = q * kCols + threadIdx.x; c < min(a.D, (q + 1) * kCols); c += kThreads) {
        float acc = a.partials[(int64_t)pb * a.D + c];
        for (int p = 1; p < nparts; ++p) acc += a.partials[(int64_t)(pb + p) * a.D + c];
        store_out1(a, row, c, acc);
      }
    }
  }
}

// ------------------------------------------------------------- workspace
int bits_for(int64_t n) {  // bits needed to represent values 0..n-1
  int b = 0;
  while (b < 63 && ((int64_t)1 << b) < n) ++b;
  return b;
}

struct Layout {
  size_t hdr, keys_chunk, keys, chunk_valid, seg_id, seg_start, part_base, item_seg, item_part, multi, bitmap,
      partials, total;
  int nchunks;
  int64_t max_items, max_multi, max_partials;
};

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

Layout make_layout(int64_t T, int64_t V, int64_t D) {
  Layout L{};
  L.nchunks = (int)ceil_div(T > 0 ? T : 1, kChunk);
  L.max_items = ceil_div(T, kRun) + T;
  L.max_multi = ceil_div(T, kRun) + 1;
  L.max_partials = 2 * ceil_div(T, kRun) + 1;
  size_t o = 0;
  L.hdr = o;
  o = align256(o + sizeof(EmbHeader));
  L.keys_chunk = o;
  o = align256(o + (size_t)L.nchunks * kChunk * 4);
  L.keys = o;
  o = align256(o + (size_t)T * 4);
  L.chunk_valid = o;
  o = align256(o + (size_t)L.nchunks * 4);
  L.seg_id = o;
  o = align256(o + (size_t)T * 4);
  L.seg_start = o;
  o = align256(o + (size_t)(T + 1) * 4);
  L.part_base = o;
  o = align256(o + (size_t)T * 4);
  L.item_seg = o;
  o = align256(o + (size_t)L.max_items * 4);
  L.item_part = o;
  o = align256(o + (size_t)L.max_items * 4);
  L.multi = o;
  o = align256(o + (size_t)L.max_multi * 4);
  L.bitmap = o;
  o = align256(o + (size_t)ceil_div(V, 32) * 4);
  L.partials = o;
  o = align256(o + (size_t)L.max_partials * (size_t)D * 4);
  L.total = o;
  return L;
}

}  // namespace
}  // namespace kp

using namespace kp;

extern "C" {

int kp_embedding_fwd_bf16(const void* table, int64_t V, int64_t D, int64_t table_row_stride, const void* indices,
                          int index_bytes, int64_t T, void* out, int64_t out_row_stride, int32_t* error_flag,
                          void* stream) {
  static const char* who = "kp_embedding_fwd_bf16";
  if (table == nullptr || out == nullptr || (T > 0 && indices == nullptr))
    return fail(KP_EINVAL, "%s: NULL table, indices or out", who);
  if (V <= 0 || D <= 0 || T < 0) return fail(KP_EINVAL, "%s: need V > 0, D > 0, T >= 0", who);
  if (index_bytes != 4 && index_bytes != 8) return fail(KP_EINVAL, "%s: index_bytes must be 4 or 8", who);
  if (table_row_stride < D || out_row_stride < D) return fail(KP_EINVAL, "%s: row strides must be >= D", who);
  if (T == 0) return KP_OK;
  EmbFwdArgs a{static_cast<const uint16_t*>(table), V, D, table_row_stride, indices, index_bytes, T,
               static_cast<uint16_t*>(out), out_row_stride, error_flag};
  const bool vec = (D % 8) == 0 && aligned16(table) && aligned16(out) && (table_row_stride % 8) == 0 &&
                   (out_row_stride % 8) == 0;
  const int64_t blocks_needed = ceil_div(T, kThreads / 64);
  const int64_t cap = (int64_t)cu_count() * 16;
  const int grid = (int)(blocks_needed < cap ? blocks_needed : cap);
  hipStream_t s = as_stream(stream);
  prof_begin(s);
  if (vec) hipLaunchKernelGGL(emb_fwd<true>, dim3(grid), dim3(kThreads), 0, s, a);
  else hipLaunchKernelGGL(emb_fwd<false>, dim3(grid), dim3(kThreads), 0, s, a);
  prof_end(s);
  return check_launch(who);
}

size_t kp_embedding_bwd_workspace_size(int64_t T, int64_t V, int64_t D) {
  if (T < 0 || V <= 0 || D <= 0) return 0;
  return make_layout(T, V, D).total;
}

int kp_embedding_bwd_bf16(const void* grad, int64_t grad_row_stride, const void* indices, int index_bytes, int64_t T,
                          int64_t V, int64_t D, int64_t padding_idx, int scale_grad_by_freq, void* grad_table,
                          int out_dtype, int out_round_bf16, void* workspace, size_t workspace_bytes,
                          int32_t* error_flag, void* stream) {
  static const char* who = "kp_embedding_bwd_bf16";
  if (grad_table == nullptr || (T > 0 && (grad == nullptr || indices == nullptr)))
    return fail(KP_EINVAL, "%s: NULL grad, indices or grad_table", who);
  if (V <= 0 || D <= 0 || T < 0) return fail(KP_EINVAL, "%s: need V > 0, D > 0, T >= 0", who);
  if (index_bytes != 4 && index_bytes != 8) return fail(KP_EINVAL, "%s: index_bytes must be 4 or 8", who);
  if (out_dtype != KP_DTYPE_F32 && out_dtype != KP_DTYPE_BF16) return fail(KP_EINVAL, "%s: bad out_dtype", who);
  if (T > 0 && grad_row_stride < D) return fail(KP_EINVAL, "%s: grad row stride must be >= D", who);
  const int tbits = bits_for(T > 0 ? T : 1);
  const int vbits = bits_for(V);
  if (T > 32768 || vbits + tbits > 31)
    return fail(KP_EUNSUPPORTED, "%s: T=%lld, V=%lld exceed this build's sort (T <= 32768, log2 V + log2 T <= 31)", who,
                (long long)T, (long long)V);
  const Layout L = make_layout(T, V, D);
  if (workspace == nullptr || workspace_bytes < L.total || !aligned16(workspace))
    return fail(KP_EWORKSPACE, "%s: workspace needs %zu bytes, 16-byte aligned (got %zu)", who, L.total,
                workspace_bytes);

  uint8_t* ws = static_cast<uint8_t*>(workspace);
  EmbBwdArgs a{};
  a.grad = static_cast<const uint16_t*>(grad);
  a.grs = grad_row_stride;
  a.idx = indices;
  a.ib = index_bytes;
  a.T = T;
  a.V = V;
  a.D = D;
  a.padding_idx = padding_idx;
  a.scale = scale_grad_by_freq ? 1 : 0;
  a.out = grad_table;
  a.out_bf16 = out_dtype == KP_DTYPE_BF16;
  a.round_bf16 = out_round_bf16 ? 1 : 0;
  a.tbits = tbits;
  a.nchunks = L.nchunks;
  a.err = error_flag;
  a.hdr = reinterpret_cast<EmbHeader*>(ws + L.hdr);
  a.keys_chunk = reinterpret_cast<uint32_t*>(ws + L.keys_chunk);
  a.keys = reinterpret_cast<uint32_t*>(ws + L.keys);
  a.chunk_valid = reinterpret_cast<int32_t*>(ws + L.chunk_valid);
  a.seg_id = reinterpret_cast<int32_t*>(ws + L.seg_id);
  a.seg_start = reinterpret_cast<int32_t*>(ws + L.seg_start);
  a.part_base = reinterpret_cast<int32_t*>(ws + L.part_base);
  a.item_seg = reinterpret_cast<int32_t*>(ws + L.item_seg);
  a.item_part = reinterpret_cast<int32_t*>(ws + L.item_part);
  a.multi = reinterpret_cast<int32_t*>(ws + L.multi);
  a.bitmap = reinterpret_cast<uint32_t*>(ws + L.bitmap);
  a.partials = reinterpret_cast<float*>(ws + L.partials);

  const bool vec = (D % 8) == 0 && aligned16(grad_table) && (T == 0 || (aligned16(grad) && grad_row_stride % 8 == 0));
  hipStream_t s = as_stream(stream);
  int st;
  hipLaunchKernelGGL(emb_sort_chunks, dim3(L.nchunks), dim3(kThreads), 0, s, a);
  if ((st = check_launch(who)) != KP_OK) return st;
  const size_t keys_bytes = (size_t)L.nchunks * kChunk * 4;
  if (keys_bytes <= 64 * 1024) {
    hipLaunchKernelGGL(emb_merge_rank<true>, dim3(L.nchunks), dim3(kThreads), keys_bytes, s, a);
  } else {
    hipLaunchKernelGGL(emb_merge_rank<false>, dim3(L.nchunks), dim3(kThreads), 0, s, a);
  }
  if ((st = check_launch(who)) != KP_OK) return st;
  hipLaunchKernelGGL(emb_plan, dim3(1), dim3(kPlanThreads), 0, s, a);
  if ((st = check_launch(who)) != KP_OK) return st;
  const int grid = cu_count() * 4;
  prof_begin(s);
  if (vec) hipLaunchKernelGGL(emb_dense<true>, dim3(grid), dim3(kThreads), 0, s, a);
  else hipLaunchKernelGGL(emb_dense<false>, dim3(grid), dim3(kThreads), 0, s, a);
  prof_end(s);
  if ((st = check_launch(who)) != KP_OK) return st;
  if (vec) hipLaunchKernelGGL(emb_combine<true>, dim3(grid), dim3(kThreads), 0, s, a);
  else hipLaunchKernelGGL(emb_combine<false>, dim3(grid), dim3(kThreads), 0, s, a);
  return check_launch(who);
}

}  // extern "C"
