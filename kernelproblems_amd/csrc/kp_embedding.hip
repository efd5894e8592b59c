// Embedding gather (forward) and deterministic dense scatter-add (backward) for gfx950.
//
// Forward: one wave64 per token row, 16-byte vector copies (1 KiB per wave
// instruction).  Table rows are read with ordinary (cacheable) loads because
// Zipf-distributed ids hit the same rows repeatedly; output rows are written
// with non-temporal stores.
//
// Backward pipeline (four launches on one stream, no float atomics):
//   K1 emb_sort_chunks : keys (id << tbits | t) of each 2048-token chunk are
//                        bitonic-sorted (registers, lane shuffles, LDS only for
//                        the cross-wave stages); padding / out-of-range ids get
//                        the sentinel key and sort last.  K1 also clears the
//                        touched-row bitmap.
//   K2 emb_rank        : one thread per key.  Binary searches in every sorted
//                        chunk give the key's global rank (keys are unique, so
//                        the order is fully determined) and the bounds [lo, hi)
//                        of its id's run in the global order; the key and its
//                        bounds are scattered to that rank and the first key of
//                        a run sets the id's bit in the bitmap.
//   K3 emb_dense       : one-shot grid.  A window block covers kWin
//                        consecutive sorted positions x 1024 columns: each run
//                        piece inside it is summed in ascending t (fp32) and
//                        written as the output row when the run lies inside the
//                        window, else as an fp32 piece row.  Every other block
//                        writes 1024 zero columns of one untouched vocab row.
//   K4 emb_combine     : runs that span windows: the window holding the run's
//                        start adds the pieces in window order and writes the row.
// Every output row is written exactly once.
#include "kp_common.hpp"
#include "kp_internal.hpp"

namespace kp {
namespace {

constexpr int kThreads = 256;
constexpr int kChunk = 2048;   // keys per K1 block (256 threads x 8)
constexpr int kWin = 32;       // sorted positions per K3 window item
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
  int32_t n_valid;  // contributing tokens (id in range, != padding_idx)
  int32_t pad[3];
};

struct EmbBwdArgs {
  const uint16_t* grad;
  int64_t grs;
  const void* idx;
  int ib;
  int64_t T, V, D, padding_idx;
  int scale;  // scale_grad_by_freq
  void* out;
  int out_bf16;
  int round_bf16;
  int tbits;
  int nchunks;
  int32_t* err;
  // workspace views
  EmbHeader* hdr;
  uint32_t* keys_chunk;  // [nchunks * kChunk] chunk-sorted keys
  int32_t* chunk_valid;  // [nchunks]
  uint32_t* keys;        // [T] globally sorted valid keys
  int32_t* run_lo;       // [T] start of the key's id run in the sorted order
  int32_t* run_hi;       // [T] end of the run
  uint32_t* bitmap;      // [ceil(V / 32)] touched rows
  float* pieces;         // [2 * nwin, D] piece rows of runs that span windows
};

// ---- K1: sort each chunk of keys (bitonic, ascending) --------------------
// Thread t holds positions 8t..8t+7.  Stages with partner distance j < 8 are
// register min/max, 8 <= j < 512 exchange within the wave (lane t ^ j/8),
// j >= 512 go through LDS with block barriers.
__global__ __launch_bounds__(kThreads) void emb_sort_chunks(EmbBwdArgs a) {
  __shared__ uint32_t s[kChunk];
  const int tid = threadIdx.x;
  const int64_t base = (int64_t)blockIdx.x * kChunk;

  // clear this block's share of the bitmap (K2 sets bits after this kernel)
  const int64_t nwords = (a.V + 31) / 32;
  const int64_t per = (nwords + gridDim.x - 1) / gridDim.x;
  for (int64_t w = blockIdx.x * per + tid; w < min(nwords, (int64_t)(blockIdx.x + 1) * per); w += kThreads)
    a.bitmap[w] = 0u;

  // The keys are unique, so their initial placement does not change the
  // sorted result: load them coalesced (element e of thread tid is token
  // base + e * 256 + tid) and sort positions 8 * tid + e.
  // All 8 index loads go out before any of them is used: the error-flag
  // store below may alias the index buffer as far as the compiler knows, so
  // loading and checking one index at a time serializes 8 memory round trips.
  // Slots past the end re-read the last index (never used); with no tokens
  // at all (the index buffer may be NULL) nothing is read.
  // The index width is tested once for the whole batch (a per-load branch
  // makes the compiler wait after every int32 load).
  int64_t id8[8];
  if (a.T > 0 && a.ib == 8) {
    const int64_t* ix = static_cast<const int64_t*>(a.idx);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int64_t t = base + e * kThreads + tid;
      id8[e] = ix[t < a.T ? t : a.T - 1];
    }
  } else if (a.T > 0) {
    const int32_t* ix = static_cast<const int32_t*>(a.idx);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int64_t t = base + e * kThreads + tid;
      id8[e] = ix[t < a.T ? t : a.T - 1];
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) id8[e] = 0;
  }
  uint32_t k8[8];
  int nvalid = 0;
  bool bad = false;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int64_t t = base + e * kThreads + tid;
    const int64_t id = id8[e];
    uint32_t key = kSentinel;
    if (t < a.T) {
      const bool in_range = id >= 0 && id < a.V;
      bad |= !in_range;
      if (in_range && id != a.padding_idx) {
        key = ((uint32_t)id << a.tbits) | (uint32_t)t;
        ++nvalid;
      }
    }
    k8[e] = key;
  }
  if (bad && a.err) *a.err = 1;

#pragma unroll
  for (int k = 2; k <= kChunk; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      if (j >= 512) {
#pragma unroll
        for (int e = 0; e < 8; ++e) s[tid * 8 + e] = k8[e];
        __syncthreads();
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int i = tid * 8 + e, l = i ^ j;
          const uint32_t o = s[l];
          const bool take_min = ((i < l) == ((i & k) == 0));
          k8[e] = take_min ? min(k8[e], o) : max(k8[e], o);
        }
        __syncthreads();
      } else if (j >= 8) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int i = tid * 8 + e, l = i ^ j;
          const uint32_t o = (uint32_t)__shfl_xor((int)k8[e], j >> 3, 64);
          const bool take_min = ((i < l) == ((i & k) == 0));
          k8[e] = take_min ? min(k8[e], o) : max(k8[e], o);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if (e & j) continue;
          const int i = tid * 8 + e;
          const bool up = (i & k) == 0;
          const uint32_t x = k8[e], y = k8[e | j];
          k8[e] = up ? min(x, y) : max(x, y);
          k8[e | j] = up ? max(x, y) : min(x, y);
        }
      }
    }
  }
  uint32_t* dst = a.keys_chunk + base + tid * 8;
  *reinterpret_cast<u32x4*>(dst) = u32x4{k8[0], k8[1], k8[2], k8[3]};
  *reinterpret_cast<u32x4*>(dst + 4) = u32x4{k8[4], k8[5], k8[6], k8[7]};
  // valid keys of the chunk (integer sum: order-independent)
  __shared__ int s_cnt;
  if (tid == 0) s_cnt = 0;
  __syncthreads();
  if (nvalid) atomicAdd(&s_cnt, nvalid);
  __syncthreads();
  if (tid == 0) a.chunk_valid[blockIdx.x] = s_cnt;
}

// ---- K2: global rank and run bounds of every valid key -------------------
// For each key, three counts over every sorted chunk: keys < key (rank),
// keys < (id << tbits) (run start) and keys < ((id + 1) << tbits) (run end).
// The 3 * nchunks binary searches advance in lockstep so their LDS reads
// overlap.  The sorted chunks are staged in LDS when they fit (<= 64 KiB,
// i.e. up to kMaxLdsChunks chunks), else read from global memory.
constexpr int kMaxLdsChunks = 8;

template <bool IN_LDS>
__global__ __launch_bounds__(kThreads) void emb_rank(EmbBwdArgs a) {
  extern __shared__ uint32_t lds_keys[];
  const int total = a.nchunks * kChunk;
  if constexpr (IN_LDS) {
    // up to kMaxLdsChunks * kChunk keys = 16 vectors per thread, all loads
    // issued before the LDS writes (a load-write loop waits per iteration)
    constexpr int kPer = kMaxLdsChunks * kChunk / (kThreads * 4);
    u32x4 v[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int i = (k * kThreads + threadIdx.x) * 4;
      v[k] = *reinterpret_cast<const u32x4*>(a.keys_chunk + (i < total ? i : 0));
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int i = (k * kThreads + threadIdx.x) * 4;
      if (i < total) *reinterpret_cast<u32x4*>(lds_keys + i) = v[k];
    }
    __syncthreads();
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    int n = 0;
    for (int c = 0; c < a.nchunks; ++c) n += a.chunk_valid[c];
    a.hdr->n_valid = n;
  }
  const int i = blockIdx.x * kThreads + threadIdx.x;
  if (i >= total) return;
  const uint32_t key = IN_LDS ? lds_keys[i] : a.keys_chunk[i];
  if (key == kSentinel) return;
  const int c = i / kChunk;
  const uint32_t id = key >> a.tbits;
  const uint32_t q[3] = {key, id << a.tbits, (id + 1) << a.tbits};  // (id + 1) << tbits <= 2^31
  int rank = i - c * kChunk, lo = 0, hi = 0;
  if constexpr (IN_LDS) {
    int pos[kMaxLdsChunks][3];
#pragma unroll
    for (int o = 0; o < kMaxLdsChunks; ++o)
#pragma unroll
      for (int k = 0; k < 3; ++k) pos[o][k] = 0;
#pragma unroll
    for (int step = kChunk >> 1; step > 0; step >>= 1) {
#pragma unroll
      for (int o = 0; o < kMaxLdsChunks; ++o) {
        if (o >= a.nchunks) break;
#pragma unroll
        for (int k = 0; k < 3; ++k)
          if (lds_keys[o * kChunk + pos[o][k] + step - 1] < q[k]) pos[o][k] += step;
      }
    }
#pragma unroll
    for (int o = 0; o < kMaxLdsChunks; ++o) {
      if (o >= a.nchunks) break;
      int cnt[3];
#pragma unroll
      for (int k = 0; k < 3; ++k) cnt[k] = pos[o][k] + (lds_keys[o * kChunk + pos[o][k]] < q[k] ? 1 : 0);
      if (o != c) rank += cnt[0];
      lo += cnt[1];
      hi += cnt[2];
    }
  } else {
    for (int o = 0; o < a.nchunks; ++o) {
      const uint32_t* v = a.keys_chunk + (int64_t)o * kChunk;
      int pos[3] = {0, 0, 0};
#pragma unroll
      for (int step = kChunk >> 1; step > 0; step >>= 1)
#pragma unroll
        for (int k = 0; k < 3; ++k)
          if (v[pos[k] + step - 1] < q[k]) pos[k] += step;
      int cnt[3];
#pragma unroll
      for (int k = 0; k < 3; ++k) cnt[k] = pos[k] + (v[pos[k]] < q[k] ? 1 : 0);
      if (o != c) rank += cnt[0];
      lo += cnt[1];
      hi += cnt[2];
    }
  }
  if (rank >= a.T) return;  // impossible for unique keys; bounds the stores regardless
  a.keys[rank] = key;
  a.run_lo[rank] = lo;
  a.run_hi[rank] = hi;
  if (rank == lo) atomicOr(a.bitmap + (id >> 5), 1u << (id & 31));
}

// Column ownership in K3/K4: a block handles one 1024-column chunk q of a
// row and thread t the 4 columns [q*1024 + 4t, q*1024 + 4t + 4); every wave
// load of grad (8 B per lane) and every fp32 store (16 B per lane) then covers
// one contiguous span of the row.
constexpr int kColStep = kThreads * 4;

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ u32x2 ld8_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
}

// Stores 4 consecutive output values (fp32 or bf16) at column c of row r.
__device__ __forceinline__ void store_out4(const EmbBwdArgs& a, int64_t r, int64_t c, f32x4 v) {
  if (a.out_bf16) {
    const u32x2 pk = {pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3])};
    __builtin_nontemporal_store(pk, reinterpret_cast<u32x2*>(static_cast<uint16_t*>(a.out) + r * a.D + c));
  } else {
    if (a.round_bf16) v = f32x4{round_bf(v[0]), round_bf(v[1]), round_bf(v[2]), round_bf(v[3])};
    st16f_stream(static_cast<float*>(a.out) + r * a.D + c, v);
  }
}
__device__ __forceinline__ void store_out1(const EmbBwdArgs& a, int64_t r, int64_t c, float v) {
  if (a.out_bf16) {
    static_cast<uint16_t*>(a.out)[r * a.D + c] = f_to_bf(v);
  } else {
    static_cast<float*>(a.out)[r * a.D + c] = a.round_bf16 ? round_bf(v) : v;
  }
}

// Workspace reads in K3/K4 are clamped to their valid ranges, so even a
// corrupted workspace cannot steer a load or store out of bounds.
__device__ __forceinline__ int64_t token_of(const EmbBwdArgs& a, int64_t r) {
  const int64_t t = (int64_t)(a.keys[r] & ((1u << a.tbits) - 1u));
  return t < a.T ? t : 0;
}
__device__ __forceinline__ int clamp_pos(int v, int n_valid) { return v < 0 ? 0 : (v > n_valid ? n_valid : v); }

// Where a finished piece [p0, p1) of the run [lo, hi) inside window [w0, w1) goes.
__device__ __forceinline__ void emit_piece(const EmbBwdArgs& a, int64_t w, int64_t w0, int64_t w1, int lo, int hi,
                                           int64_t c, const f32x4& acc) {
  if (lo >= w0 && hi <= w1) {
    const int64_t row = (int64_t)(a.keys[lo] >> a.tbits);
    if (row < a.V) store_out4(a, row, c, acc);
  } else {
    const int slot = lo < w0 ? 0 : 1;  // 0: continues from an earlier window; 1: run starts here
    *reinterpret_cast<f32x4*>(a.pieces + (2 * w + slot) * a.D + c) = acc;
  }
}
__device__ __forceinline__ void emit_piece1(const EmbBwdArgs& a, int64_t w, int64_t w0, int64_t w1, int lo, int hi,
                                            int64_t c, float acc) {
  if (lo >= w0 && hi <= w1) {
    const int64_t row = (int64_t)(a.keys[lo] >> a.tbits);
    if (row < a.V) store_out1(a, row, c, acc);
  } else {
    const int slot = lo < w0 ? 0 : 1;
    a.pieces[(2 * w + slot) * a.D + c] = acc;
  }
}

// ---- K3: windows and zero-fill -------------------------------------------
// A window block sums its sorted positions in order for its 1024 columns:
// U grad rows are loaded before any of them is added (U independent 8-byte
// loads per thread), and each column's additions run in ascending position
// order.  Run boundaries are block-uniform (run_lo / run_hi of the position).
template <bool VEC>
__device__ void emb_do_window(const EmbBwdArgs& a, int64_t w, int64_t q, int n_valid) {
  const int64_t w0 = w * kWin;
  const int64_t w1 = min((int64_t)n_valid, w0 + kWin);
  if constexpr (VEC) {
    constexpr int U = 16;
    const int64_t col = q * kColStep + threadIdx.x * 4;
    const bool on = col < a.D;
    int lo = min(clamp_pos(a.run_lo[w0], n_valid), (int)w0);
    int hi = max(clamp_pos(a.run_hi[w0], n_valid), (int)w0 + 1);
    float cnt = (float)(hi - lo);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int64_t r0 = w0; r0 < w1; r0 += U) {
      u32x2 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool have = r0 + u < w1;
        const int64_t t = have ? token_of(a, r0 + u) : 0;
        v[u] = (have && on) ? ld8_stream(a.grad + t * a.grs + col) : u32x2{0u, 0u};
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t r = r0 + u;
        if (r < w1) {
          if (r == hi) {  // a new run starts at r
            lo = min(clamp_pos(a.run_lo[r], n_valid), (int)r);
            hi = max(clamp_pos(a.run_hi[r], n_valid), (int)r + 1);
            cnt = (float)(hi - lo);
            acc = f32x4{0.f, 0.f, 0.f, 0.f};
          }
          f32x4 f = {bf_lo(v[u][0]), bf_hi(v[u][0]), bf_lo(v[u][1]), bf_hi(v[u][1])};
          if (a.scale) f = f32x4{f[0] / cnt, f[1] / cnt, f[2] / cnt, f[3] / cnt};
          acc += f;
          if ((r + 1 == hi || r + 1 == w1) && on) emit_piece(a, w, w0, w0 + kWin, lo, hi, col, acc);
        }
      }
    }
  } else {
    for (int64_t c = q * kColStep + threadIdx.x; c < min(a.D, (q + 1) * kColStep); c += kThreads) {
      int64_t r = w0;
      while (r < w1) {
        const int lo = min(clamp_pos(a.run_lo[r], n_valid), (int)r);
        const int hi = max(clamp_pos(a.run_hi[r], n_valid), (int)r + 1);
        const float cnt = (float)(hi - lo);
        const int64_t pe = min((int64_t)hi, w1);
        float acc = 0.f;
        for (; r < pe; ++r) {
          const float f = bf_to_f(a.grad[token_of(a, r) * a.grs + c]);
          acc += a.scale ? f / cnt : f;
        }
        emit_piece1(a, w, w0, w0 + kWin, lo, hi, c, acc);
      }
    }
  }
}

// One-shot dense writer.  Blocks [0, n_win_blocks) are window blocks, one per
// (window, 1024-column chunk); they come first in the grid so the heavy runs
// start early.  Every later block writes one 1024-column chunk of one vocab
// row as zeros, unless the row is touched (its window block writes it): one
// 16-byte store per thread, the launch shape that streams fastest on gfx950.
template <bool VEC>
__global__ __launch_bounds__(kThreads) void emb_dense(EmbBwdArgs a, int64_t n_win_blocks) {
  const int64_t nq = (a.D + kColStep - 1) / kColStep;
  const int64_t b = blockIdx.x;
  if (b < n_win_blocks) {
    const int n_valid = (int)min((int64_t)max(a.hdr->n_valid, 0), a.T);
    const int64_t w = b / nq, q = b % nq;
    if (w * kWin >= n_valid) return;
    emb_do_window<VEC>(a, w, q, n_valid);
    return;
  }
  const int64_t zb = b - n_win_blocks;
  const int64_t r = zb / nq, q = zb % nq;
  if (r >= a.V) return;
  if ((a.bitmap[r >> 5] >> (r & 31)) & 1u) return;
  if constexpr (VEC) {
    const int64_t c = q * kColStep + (int64_t)threadIdx.x * 4;
    if (c < a.D) store_out4(a, r, c, f32x4{0.f, 0.f, 0.f, 0.f});
  } else {
    for (int64_t c = q * kColStep + threadIdx.x; c < min(a.D, (q + 1) * kColStep); c += kThreads) store_out1(a, r, c, 0.f);
  }
}

// ---- K4: runs spanning windows, pieces added in window order ---------------
template <bool VEC>
__global__ __launch_bounds__(kThreads) void emb_combine(EmbBwdArgs a) {
  const int n_valid = (int)min((int64_t)max(a.hdr->n_valid, 0), a.T);
  const int64_t n_win = (n_valid + kWin - 1) / kWin;
  const int64_t nq = (a.D + kColStep - 1) / kColStep;
  for (int64_t it = blockIdx.x; it < n_win * nq; it += gridDim.x) {
    const int64_t w = it / nq, q = it % nq;
    const int64_t w0 = w * kWin, w1 = w0 + kWin;
    if (w1 >= n_valid) continue;  // the last window cannot hold a run that spans past it
    const int lo = clamp_pos(a.run_lo[w1 - 1], n_valid), hi = clamp_pos(a.run_hi[w1 - 1], n_valid);
    if (!(lo >= w0 && hi > w1)) continue;  // only the window where a spanning run starts combines it
    const int64_t wl = (hi - 1) / kWin;   // window holding the run's last position
    const int64_t row = a.keys[lo] >> a.tbits;
    if (row >= a.V) continue;
    if constexpr (VEC) {
      const int64_t c = q * kColStep + (int64_t)threadIdx.x * 4;
      if (c >= a.D) continue;
      f32x4 acc = *reinterpret_cast<const f32x4*>(a.pieces + (2 * w + 1) * a.D + c);
      constexpr int U = 16;
      for (int64_t w2 = w + 1; w2 <= wl; w2 += U) {
        f32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u)
          v[u] = (w2 + u <= wl) ? *reinterpret_cast<const f32x4*>(a.pieces + (2 * (w2 + u)) * a.D + c)
                                : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < U; ++u)
          if (w2 + u <= wl) acc += v[u];
      }
      store_out4(a, row, c, acc);
    } else {
      for (int64_t c = q * kColStep + threadIdx.x; c < min(a.D, (q + 1) * kColStep); c += kThreads) {
        float acc = a.pieces[(2 * w + 1) * a.D + c];
        for (int64_t w2 = w + 1; w2 <= wl; ++w2) acc += a.pieces[(2 * w2) * a.D + c];
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
  size_t hdr, keys_chunk, chunk_valid, keys, run_lo, run_hi, bitmap, pieces, total;
  int nchunks;
  int64_t nwin;
};

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

Layout make_layout(int64_t T, int64_t V, int64_t D) {
  Layout L{};
  L.nchunks = (int)ceil_div(T > 0 ? T : 1, kChunk);
  L.nwin = ceil_div(T, kWin);
  size_t o = 0;
  L.hdr = o;
  o = align256(o + sizeof(EmbHeader));
  L.keys_chunk = o;
  o = align256(o + (size_t)L.nchunks * kChunk * 4);
  L.chunk_valid = o;
  o = align256(o + (size_t)L.nchunks * 4);
  L.keys = o;
  o = align256(o + (size_t)T * 4);
  L.run_lo = o;
  o = align256(o + (size_t)T * 4);
  L.run_hi = o;
  o = align256(o + (size_t)T * 4);
  L.bitmap = o;
  o = align256(o + (size_t)ceil_div(V, 32) * 4);
  L.pieces = o;
  o = align256(o + (size_t)(2 * L.nwin + 1) * (size_t)D * 4);
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
  if ((T > 0 && (table == nullptr || out == nullptr || indices == nullptr)))
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
  if (vec) KP_LAUNCH_DOMINANT(emb_fwd<true>, dim3(grid), dim3(kThreads), 0, s, a);
  else KP_LAUNCH_DOMINANT(emb_fwd<false>, dim3(grid), dim3(kThreads), 0, s, a);
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
  a.chunk_valid = reinterpret_cast<int32_t*>(ws + L.chunk_valid);
  a.keys = reinterpret_cast<uint32_t*>(ws + L.keys);
  a.run_lo = reinterpret_cast<int32_t*>(ws + L.run_lo);
  a.run_hi = reinterpret_cast<int32_t*>(ws + L.run_hi);
  a.bitmap = reinterpret_cast<uint32_t*>(ws + L.bitmap);
  a.pieces = reinterpret_cast<float*>(ws + L.pieces);

  const bool vec = (D % 4) == 0 && aligned16(grad_table) &&
                   (T == 0 || ((reinterpret_cast<uintptr_t>(grad) & 7u) == 0 && grad_row_stride % 4 == 0));
  hipStream_t s = as_stream(stream);
  int st;
  hipLaunchKernelGGL(emb_sort_chunks, dim3(L.nchunks), dim3(kThreads), 0, s, a);
  if ((st = check_launch(who)) != KP_OK) return st;
  const int total_keys = L.nchunks * kChunk;
  const size_t keys_bytes = (size_t)total_keys * 4;
  const dim3 rgrid((unsigned)ceil_div(total_keys, kThreads));
  if (keys_bytes <= 64 * 1024) hipLaunchKernelGGL(emb_rank<true>, rgrid, dim3(kThreads), keys_bytes, s, a);
  else hipLaunchKernelGGL(emb_rank<false>, rgrid, dim3(kThreads), 0, s, a);
  if ((st = check_launch(who)) != KP_OK) return st;
  const int64_t nq = ceil_div(D, kColStep);
  const int64_t n_win_blocks = L.nwin * nq;
  const int64_t dense_blocks = n_win_blocks + V * nq;
  if (dense_blocks > 0x7fffffffLL) return fail(KP_EUNSUPPORTED, "%s: V * D too large for one launch", who);
  if (vec) KP_LAUNCH_DOMINANT(emb_dense<true>, dim3((unsigned)dense_blocks), dim3(kThreads), 0, s, a, n_win_blocks);
  else KP_LAUNCH_DOMINANT(emb_dense<false>, dim3((unsigned)dense_blocks), dim3(kThreads), 0, s, a, n_win_blocks);
  const int grid = cu_count() * 4;
  if ((st = check_launch(who)) != KP_OK) return st;
  if (vec) hipLaunchKernelGGL(emb_combine<true>, dim3(grid), dim3(kThreads), 0, s, a);
  else hipLaunchKernelGGL(emb_combine<false>, dim3(grid), dim3(kThreads), 0, s, a);
  return check_launch(who);
}

}  // extern "C"
