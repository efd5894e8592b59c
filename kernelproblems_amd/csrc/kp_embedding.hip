// Embedding gather (forward) and deterministic dense scatter-add (backward) for gfx950.
//
// Forward: one wave64 per token row, 16-byte vector copies (1 KiB per wave
// instruction).  Table rows are read with ordinary (cacheable) loads because
// Zipf-distributed ids hit the same rows repeatedly; output rows are written
// with non-temporal stores.
//
// Backward pipeline (four launches on one stream, no float atomics).  The
// token ids are sorted by (id, token) in 2048-token chunks and ranked
// globally; the dense [V, D] result is then written by window blocks (summed
// runs) and zero blocks (untouched rows).  The first three launches are
// latency chains over a few hundred KB; each carries, behind its own blocks
// in the grid, a share of the zero fill, so that the HBM streams while they
// wait:
//   K1 emb_sort_chunks : keys (id << 11 | t mod 2048) of each 2048-token chunk
//                        are bitonic-sorted (registers, lane shuffles, LDS for
//                        the cross-wave stages); padding / out-of-range ids get
//                        the sentinel key and sort last.  K1 also clears the
//                        touched-row bitmap.  Zero blocks: rows at the top of
//                        the vocabulary, written unconditionally (the bitmap is
//                        not known yet; a touched row there is written again
//                        by K3 / K4).
//   K2 emb_rank        : one thread per key.  Two binary searches per sorted
//                        chunk count the keys of smaller ids and of ids up to
//                        its own; with ties ordered by chunk (= token order)
//                        these give the key's global rank and the bounds
//                        [lo, hi) of its id's run.  Sorted ids and token
//                        indices are scattered to the rank and the first key
//                        of a run sets the id's bit in the bitmap.  Zero
//                        blocks: the next rows down, unconditionally.
//   K3 emb_dense       : window blocks cover kWin consecutive sorted positions
//                        x 1024 columns: each run piece inside a window is
//                        summed in ascending token order (fp32) and written as
//                        the output row when the run lies inside the window,
//                        else as an fp32 piece row.  Zero blocks: 1024 zero
//                        columns of each untouched row of the rest.
//   K4 emb_combine     : runs that span windows: the window holding the run's
//                        start adds the pieces in window order and writes the
//                        row.  Zero blocks: the untouched rows of the last share.
// Results are bitwise reproducible; rows outside the unconditional shares are
// written exactly once.
#include <stdlib.h>

#include <type_traits>

#include "kp_common.hpp"
#include "kp_internal.hpp"
#include "kp_rmsnorm_kernels.hpp"

namespace kp {
namespace {

constexpr int kThreads = 256;
constexpr int kChunk = 2048;   // keys per K1 block (256 threads x 8)
constexpr int kChunkBits = 11;
constexpr int kWin = 32;       // sorted positions per K3 window item
constexpr uint32_t kSentinel = 0xffffffffu;
// ids fit 21 bits so that (id << 11 | 2047) stays below the sentinel.
constexpr int64_t kMaxVocab = ((int64_t)1 << (32 - kChunkBits)) - 1;

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

// One wave per token, one token per wave (the grid covers T).  The index
// width is a template argument, so a wave's id arrives by one scalar load
// issued before any store, and a row is read unconditionally (an out-of-range
// id reads row 0) and masked to zero on the way out: the eight 16-byte loads
// of a 4096-column chunk issue back to back, with no branch between them.
// Taking the width at run time, with the loads predicated on the id's range,
// cost 35.6 us at C3 against 31.1 us in this form; a grid-stride token loop
// turned the id into a vector load waited on in full (the loop's stores
// might alias it), 32.1 us.
template <int IB>
__global__ __launch_bounds__(kThreads) void emb_fwd_vec(EmbFwdArgs a) {
  typedef typename std::conditional<IB == 8, int64_t, int32_t>::type idx_t;
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * (kThreads / 64) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (t >= a.T) return;
  constexpr int U = 8;  // 16-byte chunks per lane per 4096 columns
  const int64_t id = (int64_t) static_cast<const idx_t*>(a.idx)[t];
  const bool ok = id >= 0 && id < a.V;
  if (!ok && lane == 0 && a.err) *a.err = 1;
  const uint32_t m = ok ? 0xffffffffu : 0u;
  const uint16_t* src = a.table + (ok ? id : 0) * a.trs;
  uint16_t* dst = a.out + t * a.ors;
  int64_t c0 = 0;
#pragma unroll 1
  for (; c0 + 512 * U <= a.D; c0 += 512 * U) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = ld16(src + c0 + (u * 64 + lane) * 8);
    // all eight loads, then all eight masks, then the eight stores: the
    // chunk's 8 KB leave as one burst (stores interleaved with the waits for
    // the loads took 33.2 against 31.2 us at C3)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] &= m;
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < U; ++u) st16_stream(dst + c0 + (u * 64 + lane) * 8, v[u]);
  }
  if (c0 < a.D) {  // the last partial chunk of a row whose width is not a multiple of 4096
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t c = c0 + (int64_t)(u * 64 + lane) * 8;
      v[u] = c < a.D ? ld16(src + c) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t c = c0 + (int64_t)(u * 64 + lane) * 8;
      if (c < a.D) st16_stream(dst + c, v[u] & m);
    }
  }
}

// Any row width or alignment: one bf16 per lane access.
__global__ __launch_bounds__(kThreads) void emb_fwd_scalar(EmbFwdArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t w0 = (int64_t)blockIdx.x * (kThreads / 64) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t nw = (int64_t)gridDim.x * (kThreads / 64);
  for (int64_t t = w0; t < a.T; t += nw) {
    const int64_t id = load_index(a.idx, a.ib, t);
    const bool ok = id >= 0 && id < a.V;
    if (!ok && lane == 0 && a.err) *a.err = 1;
    const uint16_t* src = a.table + (ok ? id : 0) * a.trs;
    uint16_t* dst = a.out + t * a.ors;
    for (int64_t c = lane; c < a.D; c += 64) dst[c] = ok ? src[c] : (uint16_t)0;
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
  // V: rows of this pass's vocabulary slab [id_lo, id_lo + V) of the whole
  // vocabulary [0, v_all); ids, rows, bitmap and out are slab-relative.
  int64_t T, V, D, padding_idx;
  int64_t id_lo, v_all;
  int scale;  // scale_grad_by_freq
  void* out;
  int out_bf16;
  int round_bf16;
  int nchunks;
  int32_t* err;
  // workspace views
  EmbHeader* hdr;
  uint32_t* keys_chunk;  // [nchunks * kChunk] chunk-sorted keys
  int32_t* chunk_valid;  // [nchunks]
  uint32_t* sid;         // [T] ids in (id, token) order
  uint32_t* stok;        // [T] token indices in (id, token) order
  int32_t* run_lo;       // [T] start of the position's id run in the sorted order
  int32_t* run_hi;       // [T] end of the run
  uint32_t* bitmap;      // [ceil(V / 32)] touched rows
  float* pieces;         // [2 * nwin + 1, D] piece rows of runs that span windows
};

// Rows [lo, hi) of the zero fill carried by one launch; `cond` skips rows
// whose bit is set in the touched-row bitmap.
struct ZeroShare {
  int64_t lo, hi;
  int cond;
};

// Column ownership in the dense writer: a block handles one 1024-column chunk
// q of a row and thread t the 4 columns [q*1024 + 4t, q*1024 + 4t + 4); every
// wave load of grad (8 B per lane) and every fp32 store (16 B per lane) then
// covers one contiguous span of the row.
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

// Zero block zb of a share: 1024 columns of one row (skipped when the share
// is conditional and the row is touched).  The block's threads store one
// 16-byte (or 8-byte bf16) vector each.
template <bool VEC>
__device__ __forceinline__ void zero_block(const EmbBwdArgs& a, const ZeroShare& z, int64_t zb) {
  const int64_t nq = (a.D + kColStep - 1) / kColStep;
  const int64_t r = z.lo + zb / nq, q = zb % nq;
  if (r >= z.hi || r >= a.V) return;
  if (z.cond && ((a.bitmap[r >> 5] >> (r & 31)) & 1u)) return;
  if constexpr (VEC) {
    const int64_t c = q * kColStep + (int64_t)threadIdx.x * 4;
    if (c < a.D) store_out4(a, r, c, f32x4{0.f, 0.f, 0.f, 0.f});
  } else {
    for (int64_t c = q * kColStep + threadIdx.x; c < min(a.D, (q + 1) * kColStep); c += kThreads) store_out1(a, r, c, 0.f);
  }
}

// ---- K1: sort each chunk of keys (bitonic, ascending) --------------------
// Thread t holds positions 8t..8t+7.  Stages with partner distance j < 8 are
// register min/max, 8 <= j < 512 exchange within the wave (lane t ^ j/8),
// j >= 512 go through LDS with block barriers.  Blocks past nchunks are the
// launch's zero share.
template <bool VEC>
__global__ __launch_bounds__(kThreads) void emb_sort_chunks(EmbBwdArgs a, ZeroShare z) {
  if ((int64_t)blockIdx.x >= a.nchunks) {
    zero_block<VEC>(a, z, (int64_t)blockIdx.x - a.nchunks);
    return;
  }
  __shared__ uint32_t s[kChunk];
  const int tid = threadIdx.x;
  const int64_t base = (int64_t)blockIdx.x * kChunk;

  // clear this block's share of the bitmap (K2 sets bits after this kernel)
  const int64_t nwords = (a.V + 31) / 32;
  const int64_t per = (nwords + a.nchunks - 1) / a.nchunks;
  for (int64_t w = blockIdx.x * per + tid; w < min(nwords, (int64_t)(blockIdx.x + 1) * per); w += kThreads)
    a.bitmap[w] = 0u;

  // Element e of thread tid is token base + e * 256 + tid (coalesced index
  // loads); the keys are unique within the chunk, so their placement does
  // not change the sorted result.  All 8 index loads go out before any of
  // them is used: the error-flag store below may alias the index buffer as
  // far as the compiler knows, so loading and checking one index at a time
  // serializes 8 memory round trips.  Slots past the end re-read the last
  // index (never used); with no tokens at all (the index buffer may be NULL)
  // nothing is read.  The index width is tested once for the whole batch (a
  // per-load branch makes the compiler wait after every int32 load).
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
      const bool in_range = id >= 0 && id < a.v_all;
      bad |= !in_range;
      const int64_t rel = id - a.id_lo;  // ids of other slabs contribute nothing to this pass
      if (in_range && rel >= 0 && rel < a.V && id != a.padding_idx) {
        key = ((uint32_t)rel << kChunkBits) | (uint32_t)(e * kThreads + tid);
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
// Position i of the chunk-sorted keys (chunk c, place p in it) holds id v.
// Per chunk o: lo_o = #keys of ids < v, hi_o = #keys of ids <= v (two
// branch-free binary searches; the 11-step searches of a batch of chunks
// advance in lockstep so their loads overlap).  Run bounds: lo = sum lo_o,
// hi = sum hi_o.  Rank in (id, token) order: p + sum_{o < c} hi_o +
// sum_{o > c} lo_o -- equal ids of earlier chunks are earlier tokens.  The
// sorted chunks (a few hundred KB at most) are read through the caches.
constexpr int kRankBatch = 8;

template <bool VEC>
__global__ __launch_bounds__(kThreads) void emb_rank(EmbBwdArgs a, int rank_blocks, ZeroShare z) {
  if ((int)blockIdx.x >= rank_blocks) {
    zero_block<VEC>(a, z, (int64_t)blockIdx.x - rank_blocks);
    return;
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    int n = 0;
    for (int c = 0; c < a.nchunks; ++c) n += a.chunk_valid[c];
    a.hdr->n_valid = n;
  }
  const int64_t total = (int64_t)a.nchunks * kChunk;
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= total) return;
  const uint32_t key = a.keys_chunk[i];
  if (key == kSentinel) return;
  const int c = (int)(i / kChunk);
  const int p = (int)(i - (int64_t)c * kChunk);
  const uint32_t id = key >> kChunkBits;
  const uint32_t q_lo = id << kChunkBits, q_hi = (id + 1) << kChunkBits;  // id < 2^21 - 1: no overflow
  int64_t lo = 0, hi = 0, rank = p;
  for (int o0 = 0; o0 < a.nchunks; o0 += kRankBatch) {
    int pl[kRankBatch], ph[kRankBatch];
#pragma unroll
    for (int b = 0; b < kRankBatch; ++b) pl[b] = ph[b] = 0;
#pragma unroll
    for (int step = kChunk >> 1; step > 0; step >>= 1) {
#pragma unroll
      for (int b = 0; b < kRankBatch; ++b) {
        const int o = o0 + b < a.nchunks ? o0 + b : a.nchunks - 1;  // clamped: results of o >= nchunks unused
        const uint32_t* v = a.keys_chunk + (int64_t)o * kChunk;
        if (v[pl[b] + step - 1] < q_lo) pl[b] += step;
        if (v[ph[b] + step - 1] < q_hi) ph[b] += step;
      }
    }
#pragma unroll
    for (int b = 0; b < kRankBatch; ++b) {
      const int o = o0 + b;
      if (o >= a.nchunks) break;
      const uint32_t* v = a.keys_chunk + (int64_t)o * kChunk;
      const int cl = pl[b] + (v[pl[b]] < q_lo ? 1 : 0);
      const int ch = ph[b] + (v[ph[b]] < q_hi ? 1 : 0);
      lo += cl;
      hi += ch;
      if (o < c) rank += ch;
      else if (o > c) rank += cl;
    }
  }
  if (rank >= a.T) return;  // impossible (ranks are a permutation); bounds the stores regardless
  a.sid[rank] = id;
  a.stok[rank] = (uint32_t)((int64_t)c * kChunk + (key & (kChunk - 1)));
  a.run_lo[rank] = (int32_t)lo;
  a.run_hi[rank] = (int32_t)hi;
  if (rank == lo) atomicOr(a.bitmap + (id >> 5), 1u << (id & 31));
}

// Workspace reads in K3/K4 are clamped to their valid ranges, so even a
// corrupted workspace cannot steer a load or store out of bounds.
__device__ __forceinline__ int64_t token_of(const EmbBwdArgs& a, int64_t r) {
  const int64_t t = (int64_t)a.stok[r];
  return t < a.T ? t : 0;
}
__device__ __forceinline__ int64_t row_of(const EmbBwdArgs& a, int64_t r) { return (int64_t)a.sid[r]; }
__device__ __forceinline__ int clamp_pos(int v, int n_valid) { return v < 0 ? 0 : (v > n_valid ? n_valid : v); }

// Where a finished piece [p0, p1) of the run [lo, hi) inside window [w0, w1) goes.
// `row` is the run's id (sid[lo]), read only when the run lies in the window.
__device__ __forceinline__ void emit_piece_row(const EmbBwdArgs& a, int64_t w, int64_t w0, int64_t w1, int lo, int hi,
                                               int64_t c, const f32x4& acc, int64_t row) {
  if (lo >= w0 && hi <= w1) {
    if (row < a.V) store_out4(a, row, c, acc);
  } else {
    const int slot = lo < w0 ? 0 : 1;  // 0: continues from an earlier window; 1: run starts here
    *reinterpret_cast<f32x4*>(a.pieces + (2 * w + slot) * a.D + c) = acc;
  }
}
__device__ __forceinline__ void emit_piece1(const EmbBwdArgs& a, int64_t w, int64_t w0, int64_t w1, int lo, int hi,
                                            int64_t c, float acc) {
  if (lo >= w0 && hi <= w1) {
    const int64_t row = row_of(a, lo);
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
    // Lane i < np holds position w0 + i's token, run bounds and id, fetched
    // in one batch and read as scalars (readlane) by the loop: a window of
    // many short runs would otherwise wait for one dependent load of its
    // bounds (and one of its id) per run.
    const int np = (int)(w1 - w0);  // 1..kWin
    const int lane = threadIdx.x & 63;
    const int64_t pl = w0 + (lane < np ? lane : np - 1);
    const int tok_l = (int)token_of(a, pl);
    const int lo_l = clamp_pos(a.run_lo[pl], n_valid);
    const int hi_l = clamp_pos(a.run_hi[pl], n_valid);
    const int id_l = (int)a.sid[pl];
    int lo = (int)w0, hi = (int)w0;  // hi == w0: a run starts at the first position
    float cnt = 1.f;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < np; k0 += U) {
      u32x2 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool have = k0 + u < np;
        const int64_t t = have ? (int64_t)__builtin_amdgcn_readlane(tok_l, k0 + u) : 0;
        v[u] = (have && on) ? ld8_stream(a.grad + t * a.grs + col) : u32x2{0u, 0u};
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int k = k0 + u;
        const int r = (int)w0 + k;
        if (k < np) {
          if (r == hi) {  // a new run starts at r
            lo = min(__builtin_amdgcn_readlane(lo_l, k), r);
            hi = max(__builtin_amdgcn_readlane(hi_l, k), r + 1);
            cnt = (float)(hi - lo);
            acc = f32x4{0.f, 0.f, 0.f, 0.f};
          }
          f32x4 f = {bf_lo(v[u][0]), bf_hi(v[u][0]), bf_lo(v[u][1]), bf_hi(v[u][1])};
          if (a.scale) f = f32x4{f[0] / cnt, f[1] / cnt, f[2] / cnt, f[3] / cnt};
          acc += f;
          if (r + 1 == hi || r + 1 == (int)w1) {
            // the run's id: lane lo - w0 when the run starts in this window (a final row)
            const int64_t row = lo >= w0 ? (int64_t)(uint32_t)__builtin_amdgcn_readlane(id_l, lo - (int)w0) : 0;
            if (on) emit_piece_row(a, w, w0, w0 + kWin, lo, hi, col, acc, row);
          }
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

// Blocks [0, n_win_blocks) are window blocks, one per (window, 1024-column
// chunk); they come first in the grid so the heavy runs start early.  Every
// later block is one zero block of the launch's (conditional) share.
template <bool VEC>
__global__ __launch_bounds__(kThreads) void emb_dense(EmbBwdArgs a, int64_t n_win_blocks, ZeroShare z) {
  const int64_t nq = (a.D + kColStep - 1) / kColStep;
  const int64_t b = blockIdx.x;
  if (b < n_win_blocks) {
    const int n_valid = (int)min((int64_t)max(a.hdr->n_valid, 0), a.T);
    const int64_t w = b / nq, q = b % nq;
    if (w * kWin >= n_valid) return;
    emb_do_window<VEC>(a, w, q, n_valid);
    return;
  }
  zero_block<VEC>(a, z, b - n_win_blocks);
}

// ---- K4: runs spanning windows, pieces added in window order ---------------
// Blocks [0, comb_blocks) walk the windows grid-stride; later blocks are the
// launch's (conditional) zero share.
template <bool VEC>
__global__ __launch_bounds__(kThreads) void emb_combine(EmbBwdArgs a, int comb_blocks, ZeroShare z) {
  if ((int)blockIdx.x >= comb_blocks) {
    zero_block<VEC>(a, z, (int64_t)blockIdx.x - comb_blocks);
    return;
  }
  const int n_valid = (int)min((int64_t)max(a.hdr->n_valid, 0), a.T);
  const int64_t n_win = (n_valid + kWin - 1) / kWin;
  const int64_t nq = (a.D + kColStep - 1) / kColStep;
  for (int64_t it = blockIdx.x; it < n_win * nq; it += comb_blocks) {
    const int64_t w = it / nq, q = it % nq;
    const int64_t w0 = w * kWin, w1 = w0 + kWin;
    if (w1 >= n_valid) continue;  // the last window cannot hold a run that spans past it
    const int lo = clamp_pos(a.run_lo[w1 - 1], n_valid), hi = clamp_pos(a.run_hi[w1 - 1], n_valid);
    if (!(lo >= w0 && hi > w1)) continue;  // only the window where a spanning run starts combines it
    const int64_t wl = (hi - 1) / kWin;   // window holding the run's last position
    const int64_t row = row_of(a, lo);
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

// ---- Fused chain: RMSNorm backward -> embedding backward ------------------
// The norm's row pass walks each window's sorted positions ((id, token) order)
// instead of token order, so the rows g = dx_residual + dx of a run are summed
// into the run's fp32 accumulators as they are made -- ascending token order,
// the sums K3 forms from a stored g -- and g never reaches HBM.  Block
// b < nwin: window b (kWin positions), one row per step with the next
// position's loads in flight, in the row layout of the RMSNorm backward
// kernel for the same N (WPR waves of VPL chunks; wave w owns columns
// [w * SEG, (w + 1) * SEG)), so every row's reductions, y and g are bitwise
// those of that kernel.  Blocks [nwin, nwin + nb2): the norm rows of tokens the
// embedding skips (padding or out-of-range id), which hold no sorted
// position; their g is dropped.  Every block writes one weight-gradient
// partial row -- a fixed grouping (windows, then token ranges) -- and the
// RMSNorm finalize sums them.  Pieces of runs that span windows go to the
// same piece rows as K3's, for K4.
struct ChainArgs {
  int64_t nwin;    // window blocks
  int64_t nb2;     // norm-only blocks
  int64_t tpb2;    // tokens per norm-only block
  float* partial;  // [ceil(N / 16)][nwin + nb2][16] fp32, or nullptr (no weight gradient)
};

constexpr int64_t kChainTokens = 128;  // tokens per norm-only block

// 8 consecutive values (fp32 or bf16) at column c of table row r; write-back
// stores (a lane's 32 fp32 bytes are two 16-byte stores that L2 merges).
__device__ __forceinline__ void store_out8(const EmbBwdArgs& a, int64_t r, int64_t c, const float* v) {
  if (a.out_bf16) {
    st16(static_cast<uint16_t*>(a.out) + r * a.D + c, pack8(v));
  } else {
    float t[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) t[j] = a.round_bf16 ? round_bf(v[j]) : v[j];
    st32f(static_cast<float*>(a.out) + r * a.D + c, t);
  }
}

// Rows in flight: RB positions of the block's window per step, one per group
// of WPR waves (rloc r takes position w0 + k RB + r).  The groups r > 0 pass
// their g rows through LDS to group 0, which adds them to the run in
// position order -- the order K3 sums a stored g in -- and emits finished
// runs.  Positions past the window's end run as a masked row (row M: its
// loads re-read row M - 1, nothing is stored), so every wave meets the row
// reduction's barriers equally often.
template <int WPR>
struct ChainShape {
  static constexpr int NW = WPR > 4 ? WPR : 4;  // waves per block
  static constexpr int RB = NW / WPR;           // positions per step
};

template <int VPL, int WPR, int NDY, bool FWD>
__global__ __launch_bounds__(ChainShape<WPR>::NW * 64) void rms_emb_window(rms::RmsBwdArgs a, EmbBwdArgs e,
                                                                           ChainArgs c) {
  constexpr int NW = ChainShape<WPR>::NW, RB = ChainShape<WPR>::RB, SEG = 512 * VPL;
  __shared__ float red[2][NW][2];
  // g chunks of groups 1..RB-1 for group 0, two steps deep
  __shared__ u32x4 gx[2][RB > 1 ? RB - 1 : 1][WPR][VPL][64];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int part = wave % WPR, rloc = wave / WPR;
  const int64_t col = (int64_t)part * SEG + lane * 8;
  float wf[VPL * 8];
  {
    u32x4 wv[VPL];
    rms::load_weight<VPL>(wv, a.w, a.w_seg_len, a.w_seg_stride, col);
#pragma unroll
    for (int i = 0; i < VPL; ++i) unpack8(wv[i], wf + i * 8);
  }
  float acc[VPL * 8];
#pragma unroll
  for (int j = 0; j < VPL * 8; ++j) acc[j] = 0.f;
  int it = 0;
  const int64_t b = blockIdx.x;
  const int64_t nwb = c.nwin;  // window blocks
  if (b < nwb) {
    const int n_valid = (int)min((int64_t)max(e.hdr->n_valid, 0), e.T);
    const int w0 = (int)(b * kWin);
    const int w1 = min(n_valid, w0 + kWin);
    const int np = w1 - w0;
    if (np > 0) {
      // Lane i < np holds position w0 + i's token, run bounds and id; the
      // loop reads them as scalars (readlane), with no dependent load.
      const int li = min(lane, np - 1);
      const int tok_l = (int)token_of(e, w0 + li);
      const int lo_l = clamp_pos(e.run_lo[w0 + li], n_valid);
      const int hi_l = clamp_pos(e.run_hi[w0 + li], n_valid);
      const int id_l = (int)e.sid[w0 + li];
      const int steps = (np + RB - 1) / RB;
      float racc[VPL * 8];
#pragma unroll
      for (int j = 0; j < VPL * 8; ++j) racc[j] = 0.f;
      int lo = w0, hi = w0;  // hi == w0: a run starts at the first position
      rms::RawRow<VPL, 1> x0, x1;
      rms::RawRow<VPL, NDY> d0, d1;
      rms::RawRow<VPL, 1> r0, r1;
      float q0, q1;
      // Position q of the window (offset from w0) into the run: group 0 only.
      auto add_pos = [&](int q, const u32x4 (&gq)[VPL]) {
        const int p = w0 + q;
        if (p == hi) {
          lo = min(__builtin_amdgcn_readlane(lo_l, q), p);
          hi = max(__builtin_amdgcn_readlane(hi_l, q), p + 1);
#pragma unroll
          for (int j = 0; j < VPL * 8; ++j) racc[j] = 0.f;
        }
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
          float f[8];
          unpack8(gq[i], f);
#pragma unroll
          for (int j = 0; j < 8; ++j) racc[i * 8 + j] += f[j];
        }
        if (p + 1 == hi || p + 1 == w1) {
          if (lo >= w0 && hi <= w0 + kWin) {
            const int64_t row = (int64_t)(uint32_t)__builtin_amdgcn_readlane(id_l, lo - w0);
            if (row < e.V)
#pragma unroll
              for (int i = 0; i < VPL; ++i) store_out8(e, row, col + i * 512, racc + i * 8);
          } else {
            float* pr = e.pieces + (2 * b + (lo < w0 ? 0 : 1)) * e.D + col;
#pragma unroll
            for (int i = 0; i < VPL; ++i) st32f(pr + i * 512, racc + i * 8);
          }
        }
      };
#define KP_POS(k) ((k) * RB + rloc)
#define KP_ROWK(k) (KP_POS(k) < np ? (int64_t)__builtin_amdgcn_readlane(tok_l, KP_POS(k)) : a.M)
#define KP_LOAD(S, k)                                                                                  \
  rms::bwd_load<VPL, 1, NDY, true, FWD>(x##S, d##S, r##S, q##S, a, rms::clamp_row(KP_ROWK(k), a.M), col); \
  __builtin_amdgcn_sched_barrier(0)
#define KP_PROC(S, k)                                                                                              \
  {                                                                                                                \
    u32x4 gv[VPL];                                                                                                 \
    rms::bwd_row<VPL, WPR, 1, NDY, true, NW, FWD, true>(a, x##S, d##S, r##S, q##S, wf, acc, red, KP_ROWK(k), col,  \
                                                        lane, wave, rloc, it, gv);                                \
    if constexpr (RB > 1) {                                                                                        \
      if (rloc > 0) {                                                                                              \
        _Pragma("unroll") for (int i = 0; i < VPL; ++i) gx[it & 1][rloc - 1][part][i][lane] = gv[i];             \
      }                                                                                                            \
      __syncthreads();                                                                                             \
    }                                                                                                              \
    if (rloc == 0) {                                                                                               \
      if ((k) * RB < np) add_pos((k) * RB, gv);                                                                    \
      _Pragma("unroll") for (int r = 1; r < RB; ++r) {                                                            \
        if ((k) * RB + r < np) {                                                                                   \
          u32x4 gr[VPL];                                                                                           \
          _Pragma("unroll") for (int i = 0; i < VPL; ++i) gr[i] = gx[it & 1][r - 1][part][i][lane];              \
          add_pos((k) * RB + r, gr);                                                                               \
        }                                                                                                          \
      }                                                                                                            \
    }                                                                                                              \
    ++it;                                                                                                          \
  }
      int k = 0;
      KP_LOAD(0, 0);
      for (; k + 2 < steps; k += 2) {
        KP_LOAD(1, k + 1);
        KP_PROC(0, k);
        KP_LOAD(0, k + 2);
        KP_PROC(1, k + 1);
      }
      if (k + 1 < steps) {
        KP_LOAD(1, k + 1);
        KP_PROC(0, k);
        KP_PROC(1, k + 1);
      } else {
        KP_PROC(0, k);
      }
#undef KP_POS
#undef KP_ROWK
#undef KP_LOAD
#undef KP_PROC
    }
  } else if (b < nwb + c.nb2) {
    // Tokens [t0, t1): a row whose id K1 rejected (out of range or the
    // padding index) still belongs to the norm (y, rstd, weight gradient).
    // The ballot is the same in every wave (same ids), so the block agrees;
    // each such row is processed by the rloc 0 waves (the others run a
    // masked row to meet the barriers).
    const int64_t t0 = (b - nwb) * c.tpb2;
    const int64_t t1 = min(e.T, t0 + c.tpb2);
    for (int64_t tb = t0; tb < t1; tb += 64) {
      const int64_t t = tb + lane;
      bool skipped = false;
      if (t < t1) {
        const int64_t id = load_index(e.idx, e.ib, t);
        skipped = !(id >= 0 && id < e.V) || id == e.padding_idx;
      }
      uint64_t m = __ballot(skipped);
      while (m != 0) {
        const int64_t row = rloc == 0 ? tb + __builtin_ctzll(m) : a.M;
        m &= m - 1;
        rms::RawRow<VPL, 1> xr;
        rms::RawRow<VPL, NDY> dr;
        rms::RawRow<VPL, 1> rr;
        float rq;
        rms::bwd_load<VPL, 1, NDY, true, FWD>(xr, dr, rr, rq, a, rms::clamp_row(row, a.M), col);
        u32x4 gv[VPL];
        rms::bwd_row<VPL, WPR, 1, NDY, true, NW, FWD, true>(a, xr, dr, rr, rq, wf, acc, red, row, col, lane, wave,
                                                            rloc, it, gv);
        ++it;
      }
    }
  }
  // One partial row per block: the RB row groups' column sums combined in a
  // fixed order (rloc 0 + rloc 1 + ...) through LDS, then stored by rloc 0.
  if (c.partial != nullptr) {
    if constexpr (RB > 1) {
      __shared__ float comb[RB - 1][WPR][SEG];
      if (rloc > 0) {
#pragma unroll
        for (int j = 0; j < VPL * 8; j += 4)
          *reinterpret_cast<f32x4*>(&comb[rloc - 1][part][(j / 8) * 512 + lane * 8 + (j % 8)]) =
              f32x4{acc[j], acc[j + 1], acc[j + 2], acc[j + 3]};
      }
      __syncthreads();
      if (rloc == 0) {
#pragma unroll
        for (int r = 0; r < RB - 1; ++r)
#pragma unroll
          for (int j = 0; j < VPL * 8; ++j) acc[j] += comb[r][part][(j / 8) * 512 + lane * 8 + (j % 8)];
      }
    }
    if (rloc == 0) {
      const int64_t P = nwb + c.nb2;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        float* pp = c.partial + rms::part_index(col + i * 512, b, P);  // 8 columns inside one 16-column chunk
        *reinterpret_cast<f32x4*>(pp) = f32x4{acc[i * 8], acc[i * 8 + 1], acc[i * 8 + 2], acc[i * 8 + 3]};
        *reinterpret_cast<f32x4*>(pp + 4) = f32x4{acc[i * 8 + 4], acc[i * 8 + 5], acc[i * 8 + 6], acc[i * 8 + 7]};
      }
    }
  }
}

typedef void (*ChainKernel)(rms::RmsBwdArgs, EmbBwdArgs, ChainArgs);

template <int VPL, int WPR>
ChainKernel chain_kernel_for(int n_dy, bool fwd) {
  switch (n_dy * 2 + (fwd ? 1 : 0)) {
    case 2: return rms_emb_window<VPL, WPR, 1, false>;
    case 3: return rms_emb_window<VPL, WPR, 1, true>;
    case 4: return rms_emb_window<VPL, WPR, 2, false>;
    case 5: return rms_emb_window<VPL, WPR, 2, true>;
    case 6: return rms_emb_window<VPL, WPR, 3, false>;
    case 7: return rms_emb_window<VPL, WPR, 3, true>;
  }
  return nullptr;
}
// Row widths with a fused kernel and their row layout: the RMSNorm
// backward's default shape for that N (VPL chunks x WPR waves per row).
// *nw gets the block's waves, *rb its rows per step.
ChainKernel chain_kernel(int64_t N, int n_dy, bool fwd, int* nw, int* rb) {
  switch (N) {
    case 2048: *nw = ChainShape<1>::NW; *rb = ChainShape<1>::RB; return chain_kernel_for<4, 1>(n_dy, fwd);
    case 4096: *nw = ChainShape<2>::NW; *rb = ChainShape<2>::RB; return chain_kernel_for<4, 2>(n_dy, fwd);
    case 8192: *nw = ChainShape<8>::NW; *rb = ChainShape<8>::RB; return chain_kernel_for<2, 8>(n_dy, fwd);
  }
  return nullptr;
}

// ------------------------------------------------------------- workspace
struct Layout {
  size_t hdr, keys_chunk, chunk_valid, sid, stok, run_lo, run_hi, bitmap, pieces, total;
  int64_t nchunks;
  int64_t nwin;
};

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

Layout make_layout(int64_t T, int64_t V, int64_t D) {
  Layout L{};
  L.nchunks = ceil_div(T > 0 ? T : 1, kChunk);
  L.nwin = ceil_div(T, kWin);
  size_t o = 0;
  L.hdr = o;
  o = align256(o + sizeof(EmbHeader));
  L.keys_chunk = o;
  o = align256(o + (size_t)L.nchunks * kChunk * 4);
  L.chunk_valid = o;
  o = align256(o + (size_t)L.nchunks * 4);
  L.sid = o;
  o = align256(o + (size_t)T * 4);
  L.stok = o;
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

// Zero-fill share of each latency-chain launch, in MiB of output rows (K1,
// K2: unconditional; K4: conditional), at least as long to stream as the
// launch's own chain (~13-17 us each at the C3 configuration).  Measured on
// MI355X at C3 (whole call): 96/96/64 MiB 357.1 us, 128/128/96 356.1 us,
// 160/160/128 357.6 us, 256/256/192 360.9 us -- once the chains are hidden
// the pipeline is bound by HBM alone.  Tuning knobs: KP_EMB_ZERO_MB_SORT /
// _RANK / _COMBINE.
int64_t share_rows(const char* env, int64_t dflt_mb, int64_t row_bytes, int64_t cap_rows) {
  static_assert(sizeof(long long) == 8, "");
  const char* e = getenv(env);
  const int64_t mb = e ? atoll(e) : dflt_mb;
  const int64_t rows = mb <= 0 ? 0 : ((mb << 20) + row_bytes - 1) / row_bytes;
  return rows < cap_rows ? rows : cap_rows;
}

// Workspace of the fused chain: the embedding backward's layout, then the
// weight-gradient partial rows of its window and norm-only blocks.
struct ChainLayout {
  Layout emb;
  int64_t nwin, nb2;
  size_t partial, total;
};
ChainLayout make_chain_layout(int64_t T, int64_t V, int64_t D) {
  ChainLayout L{};
  L.emb = make_layout(T, V, D);
  L.nwin = ceil_div(T, kWin);
  L.nb2 = ceil_div(T, kChainTokens);
  L.partial = L.emb.total;
  L.total = align256(L.partial + (size_t)(L.nwin + L.nb2) * (size_t)(ceil_div(D, rms::kPartChunk) * rms::kPartChunk) *
                                     sizeof(float));
  return L;
}

bool rows16(const void* p, int64_t stride) { return aligned16(p) && (stride & 7) == 0; }

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
  hipStream_t s = as_stream(stream);
  if (vec) {  // one token per wave: the grid covers T
    if (blocks_needed > 0x7fffffff) return fail(KP_EUNSUPPORTED, "%s: T = %lld tokens exceeds one launch", who, (long long)T);
    if (index_bytes == 8) KP_LAUNCH_DOMINANT(emb_fwd_vec<8>, dim3((unsigned)blocks_needed), dim3(kThreads), 0, s, a);
    else KP_LAUNCH_DOMINANT(emb_fwd_vec<4>, dim3((unsigned)blocks_needed), dim3(kThreads), 0, s, a);
  } else {
    const int64_t cap = (int64_t)cu_count() * 16;
    const int grid = (int)(blocks_needed < cap ? blocks_needed : cap);
    KP_LAUNCH_DOMINANT(emb_fwd_scalar, dim3(grid), dim3(kThreads), 0, s, a);
  }
  return check_launch(who);
}

size_t kp_embedding_bwd_workspace_size(int64_t T, int64_t V, int64_t D) {
  if (T < 0 || V <= 0 || D <= 0) return 0;
  return make_layout(T, V < kMaxVocab ? V : kMaxVocab, D).total;  // one slab's bitmap (see the entry point)
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
  if (T > 0x7fffffffLL)
    return fail(KP_EUNSUPPORTED, "%s: T=%lld outside this build's sort (T < 2^31)", who, (long long)T);
  // The sort keys hold an id below 2^21 (kMaxVocab), so a larger vocabulary
  // runs as one pass of the whole pipeline per slab of kMaxVocab rows: each
  // pass sorts the ids of its slab (relative to the slab), writes the slab's
  // rows (dense sums and zero fill) and ignores every other token.  The
  // workspace holds one slab's bitmap; the passes reuse it in stream order.
  const int64_t vs_max = V < kMaxVocab ? V : kMaxVocab;
  const Layout L = make_layout(T, vs_max, D);
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
  a.V = vs_max;
  a.D = D;
  a.padding_idx = padding_idx;
  a.id_lo = 0;
  a.v_all = V;
  a.scale = scale_grad_by_freq ? 1 : 0;
  a.out = grad_table;
  a.out_bf16 = out_dtype == KP_DTYPE_BF16;
  a.round_bf16 = out_round_bf16 ? 1 : 0;
  a.nchunks = (int)L.nchunks;
  a.err = error_flag;
  a.hdr = reinterpret_cast<EmbHeader*>(ws + L.hdr);
  a.keys_chunk = reinterpret_cast<uint32_t*>(ws + L.keys_chunk);
  a.chunk_valid = reinterpret_cast<int32_t*>(ws + L.chunk_valid);
  a.sid = reinterpret_cast<uint32_t*>(ws + L.sid);
  a.stok = reinterpret_cast<uint32_t*>(ws + L.stok);
  a.run_lo = reinterpret_cast<int32_t*>(ws + L.run_lo);
  a.run_hi = reinterpret_cast<int32_t*>(ws + L.run_hi);
  a.bitmap = reinterpret_cast<uint32_t*>(ws + L.bitmap);
  a.pieces = reinterpret_cast<float*>(ws + L.pieces);

  const bool vec = (D % 4) == 0 && aligned16(grad_table) &&
                   (T == 0 || ((reinterpret_cast<uintptr_t>(grad) & 7u) == 0 && grad_row_stride % 4 == 0));
  hipStream_t s = as_stream(stream);
  const int64_t nq = ceil_div(D, kColStep);
  const int64_t row_bytes = D * (out_dtype == KP_DTYPE_BF16 ? 2 : 4);
  const int64_t nwin_blocks = L.nwin * nq;
  const int64_t total_keys = L.nchunks * kChunk;
  const int64_t rank_blocks = ceil_div(total_keys, kThreads);
  const int comb_blocks = cu_count() * 4;
  for (int64_t lo = 0; lo < V; lo += kMaxVocab) {
    const int64_t Vs = V - lo < kMaxVocab ? V - lo : kMaxVocab;  // this pass's slab [lo, lo + Vs)
    const bool first = lo == 0, last = lo + Vs >= V;
    a.id_lo = lo;
    a.V = Vs;
    a.out = static_cast<uint8_t*>(grad_table) + lo * row_bytes;
    // Zero-fill shares, taken from the top of the slab down (high ids are
    // the rarely touched ones under the usual frequency-ordered vocabularies):
    // K1 [Vs - z1, Vs), K2 [Vs - z1 - z2, Vs - z1), K4 [r3, Vs - z1 - z2), K3 [0, r3).
    const int64_t z1 = share_rows("KP_EMB_ZERO_MB_SORT", 128, row_bytes, Vs / 4);
    const int64_t z2 = share_rows("KP_EMB_ZERO_MB_RANK", 128, row_bytes, Vs / 4);
    const int64_t z4 = share_rows("KP_EMB_ZERO_MB_COMBINE", 96, row_bytes, Vs / 4);
    const ZeroShare zs1{Vs - z1, Vs, 0};
    const ZeroShare zs2{Vs - z1 - z2, Vs - z1, 0};
    const ZeroShare zs4{Vs - z1 - z2 - z4, Vs - z1 - z2, 1};
    const ZeroShare zs3{0, Vs - z1 - z2 - z4, 1};
    const int64_t g1 = L.nchunks + z1 * nq, g2 = rank_blocks + z2 * nq, g3 = nwin_blocks + zs3.hi * nq,
                  g4 = comb_blocks + z4 * nq;
    if (g1 > 0x7fffffffLL || g2 > 0x7fffffffLL || g3 > 0x7fffffffLL || g4 > 0x7fffffffLL)
      return fail(KP_EUNSUPPORTED, "%s: V * D too large for one launch", who);
    // With the timing hook set, the events span the whole pipeline (the first
    // K1's start to the last K4's end): its zero fill is spread over all four
    // launches.
    int st;
    if (vec) KP_LAUNCH_SPAN(first, false, emb_sort_chunks<true>, dim3((unsigned)g1), dim3(kThreads), 0, s, a, zs1);
    else KP_LAUNCH_SPAN(first, false, emb_sort_chunks<false>, dim3((unsigned)g1), dim3(kThreads), 0, s, a, zs1);
    if ((st = check_launch(who)) != KP_OK) return st;
    if (vec) hipLaunchKernelGGL(emb_rank<true>, dim3((unsigned)g2), dim3(kThreads), 0, s, a, (int)rank_blocks, zs2);
    else hipLaunchKernelGGL(emb_rank<false>, dim3((unsigned)g2), dim3(kThreads), 0, s, a, (int)rank_blocks, zs2);
    if ((st = check_launch(who)) != KP_OK) return st;
    if (vec) hipLaunchKernelGGL(emb_dense<true>, dim3((unsigned)g3), dim3(kThreads), 0, s, a, nwin_blocks, zs3);
    else hipLaunchKernelGGL(emb_dense<false>, dim3((unsigned)g3), dim3(kThreads), 0, s, a, nwin_blocks, zs3);
    if ((st = check_launch(who)) != KP_OK) return st;
    if (vec)
      KP_LAUNCH_SPAN(false, last, emb_combine<true>, dim3((unsigned)g4), dim3(kThreads), 0, s, a, comb_blocks, zs4);
    else
      KP_LAUNCH_SPAN(false, last, emb_combine<false>, dim3((unsigned)g4), dim3(kThreads), 0, s, a, comb_blocks, zs4);
    if ((st = check_launch(who)) != KP_OK) return st;
  }
  return KP_OK;
}

size_t kp_rmsnorm_embedding_bwd_workspace_size(int64_t M, int64_t N, int64_t V) {
  if (M < 0 || N <= 0 || V <= 0) return 0;
  return make_chain_layout(M, V, N).total;
}

int kp_rmsnorm_embedding_bwd_bf16(const void* const* dy_terms, const int64_t* dy_strides, int n_dy, const void* x,
                                  int64_t x_stride, const float* rstd, const void* weight, int64_t w_seg_len,
                                  int64_t w_seg_stride, const void* dx_residual, int64_t dxr_stride, void* y,
                                  int64_t y_stride, float* rstd_out, float* dw_f32, void* dw_bf16,
                                  int dw_f32_round_bf16, int64_t M, int64_t N, float eps, const void* indices,
                                  int index_bytes, int64_t V, int64_t padding_idx, void* grad_table, int out_dtype,
                                  int out_round_bf16, void* workspace, size_t workspace_bytes, int32_t* error_flag,
                                  void* stream) {
  static const char* who = "kp_rmsnorm_embedding_bwd_bf16";
  if (M < 0 || N <= 0 || V <= 0) return fail(KP_EINVAL, "%s: need M >= 0, N > 0, V > 0", who);
  if (dy_terms == nullptr || dy_strides == nullptr || n_dy < 1 || n_dy > 3)
    return fail(KP_EINVAL, "%s: dy needs 1..3 terms", who);
  if (grad_table == nullptr) return fail(KP_EINVAL, "%s: grad_table is NULL", who);
  if (M > 0) {
    for (int i = 0; i < n_dy; ++i)
      if (dy_terms[i] == nullptr || dy_strides[i] < 0) return fail(KP_EINVAL, "%s: dy term %d is NULL or has a negative stride", who, i);
    if (x == nullptr || x_stride < 0 || dx_residual == nullptr || dxr_stride < 0 || indices == nullptr)
      return fail(KP_EINVAL, "%s: NULL x, dx_residual or indices (or a negative stride)", who);
  }
  if (index_bytes != 4 && index_bytes != 8) return fail(KP_EINVAL, "%s: index_bytes must be 4 or 8", who);
  if (out_dtype != KP_DTYPE_F32 && out_dtype != KP_DTYPE_BF16) return fail(KP_EINVAL, "%s: bad out_dtype", who);
  const bool want_dw = dw_f32 != nullptr || dw_bf16 != nullptr;
  if (want_dw && weight == nullptr) return fail(KP_EINVAL, "%s: a weight gradient needs a weight", who);
  if (weight != nullptr && (w_seg_len <= 0 || w_seg_stride < 0))
    return fail(KP_EINVAL, "%s: weight segment length must be > 0", who);
  if (rstd != nullptr && (y != nullptr || rstd_out != nullptr))
    return fail(KP_EINVAL, "%s: y / rstd_out are the forward's outputs: pass rstd = NULL to compute them", who);
  if (y != nullptr && y_stride < 0) return fail(KP_EINVAL, "%s: negative y stride", who);
  // The fused row pass: N = 2048, 4096 or 8192, 16-byte rows, one x term,
  // the residual epilogue, the sort's limits.  Anything else: KP_EUNSUPPORTED
  // (the caller runs the norm and then kp_embedding_bwd_bf16).
  const bool fwd = y != nullptr || rstd_out != nullptr;
  int nw = 4, rb = 1;  // rb: rows per step, documented by the kernel's shape
  const ChainKernel kern = chain_kernel(N, n_dy, fwd, &nw, &rb);
  (void)rb;
  bool ok = kern != nullptr && V <= kMaxVocab && M <= 0x7fffffffLL && rows16(x, x_stride) &&
            rows16(dx_residual, dxr_stride) && (y == nullptr || rows16(y, y_stride)) &&
            (weight == nullptr || (aligned16(weight) && (w_seg_len & 7) == 0 && (w_seg_stride & 7) == 0)) &&
            aligned16(grad_table);
  for (int i = 0; ok && i < n_dy; ++i) ok = rows16(dy_terms[i], dy_strides[i]);
  if (!ok)
    return fail(KP_EUNSUPPORTED, "%s: no fused row pass for this shape or layout (N=%lld, %d dy terms, V=%lld)", who,
                (long long)N, n_dy, (long long)V);
  const ChainLayout CL = make_chain_layout(M, V, N);
  if (workspace == nullptr || workspace_bytes < CL.total || !aligned16(workspace))
    return fail(KP_EWORKSPACE, "%s: workspace needs %zu bytes, 16-byte aligned (got %zu)", who, CL.total,
                workspace_bytes);
  const Layout& L = CL.emb;
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  EmbBwdArgs e{};
  e.grad = nullptr;
  e.grs = N;
  e.idx = indices;
  e.ib = index_bytes;
  e.T = M;
  e.V = V;
  e.D = N;
  e.padding_idx = padding_idx;
  e.id_lo = 0;
  e.v_all = V;
  e.scale = 0;
  e.out = grad_table;
  e.out_bf16 = out_dtype == KP_DTYPE_BF16;
  e.round_bf16 = out_round_bf16 ? 1 : 0;
  e.nchunks = (int)L.nchunks;
  e.err = error_flag;
  e.hdr = reinterpret_cast<EmbHeader*>(ws + L.hdr);
  e.keys_chunk = reinterpret_cast<uint32_t*>(ws + L.keys_chunk);
  e.chunk_valid = reinterpret_cast<int32_t*>(ws + L.chunk_valid);
  e.sid = reinterpret_cast<uint32_t*>(ws + L.sid);
  e.stok = reinterpret_cast<uint32_t*>(ws + L.stok);
  e.run_lo = reinterpret_cast<int32_t*>(ws + L.run_lo);
  e.run_hi = reinterpret_cast<int32_t*>(ws + L.run_hi);
  e.bitmap = reinterpret_cast<uint32_t*>(ws + L.bitmap);
  e.pieces = reinterpret_cast<float*>(ws + L.pieces);

  rms::RmsBwdArgs a{};
  for (int i = 0; i < n_dy; ++i) {
    a.dy[i] = static_cast<const uint16_t*>(dy_terms[i]);
    a.dys[i] = dy_strides[i];
  }
  a.n_dy = n_dy;
  a.x[0] = static_cast<const uint16_t*>(x);
  a.xs[0] = x_stride;
  a.n_x = 1;
  a.rstd = rstd;
  a.w = static_cast<const uint16_t*>(weight);
  a.w_seg_len = weight ? w_seg_len : N;
  a.w_seg_stride = weight ? w_seg_stride : N;
  a.dxr = static_cast<const uint16_t*>(dx_residual);
  a.dxrs = dxr_stride;
  a.y = static_cast<uint16_t*>(y);
  a.ys = y_stride;
  a.rstd_out = rstd_out;
  a.M = M;
  a.N = N;
  a.eps = eps;
  ChainArgs c{CL.nwin, CL.nb2, kChainTokens, want_dw ? reinterpret_cast<float*>(ws + CL.partial) : nullptr};

  hipStream_t s = as_stream(stream);
  const int64_t nq = ceil_div(N, kColStep);
  const int64_t row_bytes = N * (out_dtype == KP_DTYPE_BF16 ? 2 : 4);
  // Zero fill: K1 and K2 carry unconditional shares from the top of the
  // vocabulary and K4 a conditional one, as in kp_embedding_bwd_bf16; the
  // rest of the untouched rows go to K3's zero blocks, launched with no
  // window blocks after the fused row pass (whose registers would hold zero
  // blocks sharing its launch to a few per CU).
  const int64_t z1 = share_rows("KP_EMB_ZERO_MB_SORT", 128, row_bytes, V / 4);
  const int64_t z2 = share_rows("KP_EMB_ZERO_MB_RANK", 128, row_bytes, V / 4);
  const int64_t z4 = share_rows("KP_EMB_ZERO_MB_COMBINE", 96, row_bytes, V / 4);
  const ZeroShare zs1{V - z1, V, 0};
  const ZeroShare zs2{V - z1 - z2, V - z1, 0};
  const ZeroShare zs4{V - z1 - z2 - z4, V - z1 - z2, 1};
  const ZeroShare zs3{0, V - z1 - z2 - z4, 1};
  const int64_t total_keys = L.nchunks * kChunk;
  const int64_t rank_blocks = ceil_div(total_keys, kThreads);
  const int comb_blocks = cu_count() * 4;
  const int64_t g1 = L.nchunks + z1 * nq, g2 = rank_blocks + z2 * nq, g3 = zs3.hi * nq, g4 = comb_blocks + z4 * nq;
  if (g1 > 0x7fffffffLL || g2 > 0x7fffffffLL || g3 > 0x7fffffffLL || g4 > 0x7fffffffLL)
    return fail(KP_EUNSUPPORTED, "%s: V * N too large for one launch", who);
  int st;
  KP_LAUNCH_SPAN(true, false, emb_sort_chunks<true>, dim3((unsigned)g1), dim3(kThreads), 0, s, e, zs1);
  if ((st = check_launch(who)) != KP_OK) return st;
  hipLaunchKernelGGL(emb_rank<true>, dim3((unsigned)g2), dim3(kThreads), 0, s, e, (int)rank_blocks, zs2);
  if ((st = check_launch(who)) != KP_OK) return st;
  const int64_t nblocks = CL.nwin + CL.nb2;  // window blocks, then norm-only blocks
  if (nblocks > 0) {
    hipLaunchKernelGGL(kern, dim3((unsigned)nblocks), dim3(nw * 64), 0, s, a, e, c);
    if ((st = check_launch(who)) != KP_OK) return st;
  }
  if (g3 > 0) {
    hipLaunchKernelGGL(emb_dense<true>, dim3((unsigned)g3), dim3(kThreads), 0, s, e, (int64_t)0, zs3);
    if ((st = check_launch(who)) != KP_OK) return st;
  }
  KP_LAUNCH_SPAN(false, true, emb_combine<true>, dim3((unsigned)g4), dim3(kThreads), 0, s, e, comb_blocks, zs4);
  if ((st = check_launch(who)) != KP_OK) return st;
  // The weight gradient: the partial rows in block order (none when M == 0:
  // zeros).
  if (want_dw)
    return rms_dw_finalize_launch(c.partial, (int)nblocks, N, dw_f32, static_cast<uint16_t*>(dw_bf16),
                                  dw_f32_round_bf16, s, who);
  return KP_OK;
}

}  // extern "C"
