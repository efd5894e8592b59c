// RMSNorm row kernels for gfx950: argument blocks, device helpers and the
// vectorized forward / backward kernel templates, shared by kp_rmsnorm.hip
// (dispatch, generic kernels, C ABI) and the instantiation units
// kp_rms_fwd.hip and kp_rms_bwd_<VPL>.hip.
//
// Layout: row-major bf16 [M, N], unit stride along N.  A row is processed by
// WPR wave64s, each owning a contiguous segment of 512*VPL columns; lane l of
// a wave holds the 8-element chunks at column offsets (v*64 + l)*8, v < VPL,
// so every load/store instruction of the wave moves 1 KiB of consecutive
// bytes.  Row sums are wave DPP trees (kp::wave_sum); the WPR > 1 case
// combines the per-wave sums through 32 bytes of LDS in a fixed order.
//
// Backward weight gradient: each block accumulates its rows' dy * xhat
// contributions in registers (per lane, per column), combines its waves in
// LDS in wave order and writes one fp32 partial row; a second small kernel
// sums the partial rows in a fixed order.  No float atomics anywhere, so
// results are bitwise reproducible for a given device and shape.
#pragma once

#include "kp_common.hpp"

namespace kp {
namespace rms {

constexpr int kThreads = 256;  // 4 waves per block

struct RmsFwdArgs {
  const uint16_t* x[3];
  int64_t xs[3];
  int n_x;
  // Gather variant: row r of term 0 is x[0] row idx[r] (idx_bytes 4 or 8);
  // an id outside [0, idx_rows) reads row 0 in its place, gives a zero row and sets *err.
  const void* idx;
  int idx_bytes;
  int64_t idx_rows;
  int32_t* err;
  const uint16_t* w;
  int64_t w_seg_len, w_seg_stride;
  uint16_t* h;
  int64_t hs;
  uint16_t* y;
  int64_t ys;
  float* rstd;
  int64_t M, N;
  float eps;
};

struct RmsBwdArgs {
  const uint16_t* dy[3];
  int64_t dys[3];
  int n_dy;
  const uint16_t* x[3];
  int64_t xs[3];
  int n_x;
  const float* rstd;
  const uint16_t* w;
  int64_t w_seg_len, w_seg_stride;
  const uint16_t* dxr;
  int64_t dxrs;
  uint16_t* dx;
  int64_t dxs;
  float* partial;  // [gridDim.x, N] fp32, or nullptr when no weight gradient is wanted
  // Forward outputs of the fused forward + backward kernels (FWD): the
  // normalised row y = bf16(x * rstd * w), the summed x terms h (n_x > 1;
  // may be NULL) and rstd (may be NULL), all from the rstd the backward uses.
  uint16_t* y;
  int64_t ys;
  uint16_t* h;
  int64_t hs;
  float* rstd_out;
  int64_t M, N;
  float eps;
  // Block timeline (kp_debug_block_trace): 4 words per block for blocks below
  // trace_blocks, or nullptr.
  unsigned long long* trace;
  int trace_blocks;
};

// Weight-gradient partials are stored column-chunk-major, [ceil(N/16)][P][16]
// fp32 (P = row blocks): a lane's 8 columns land as 32 contiguous bytes, and
// the finalize -- one block per 16-column chunk, N / 16 blocks, at least one
// per CU for N >= 4096 -- reads each chunk of all P rows contiguously.
constexpr int kPartChunk = 16;
__host__ __device__ __forceinline__ int64_t part_index(int64_t c, int64_t p, int64_t P) {
  return ((c / kPartChunk) * P + p) * kPartChunk + (c % kPartChunk);
}

__device__ __forceinline__ int64_t w_index(int64_t c, int64_t seg_len, int64_t seg_stride) {
  if (c < seg_len) return c;  // first segment, i.e. every column of a contiguous weight: no division
  if (((uint64_t)c | (uint64_t)seg_len) < 0x80000000ull) {  // 32-bit divide (a 64-bit one is ~100 instructions)
    const uint32_t q = (uint32_t)c / (uint32_t)seg_len;
    return (int64_t)q * seg_stride + (c - (int64_t)q * seg_len);
  }
  return (c / seg_len) * seg_stride + (c % seg_len);
}

// Row groups of block b in a grid of G blocks walking groups b, b + G, ...
// (b < G <= ngroups): ngroups fits 32 bits for any tensor that fits in
// memory, so the divide is a 32-bit one.
__device__ __forceinline__ int64_t block_trips(int64_t ngroups, int64_t b, int64_t G) {
  if (ngroups <= 0x7fffffffLL) return (int64_t)((uint32_t)(ngroups - 1 - b) / (uint32_t)G) + 1;
  return (ngroups - 1 - b) / G + 1;
}

// Raw (not yet summed) 16-byte chunks of up to NT row terms.  Rows are
// software-pipelined: the next row's raw terms are requested before the
// current row's stores, because vmcnt counts loads and stores in issue order
// and a wait on a load issued after a store would also wait for that store.
//
// Row loads are never predicated.  The row loops run an exact per-block trip
// count, so a row past the end occurs only in the last row group when M is
// not a multiple of the rows per group; it is read as row M - 1 and its
// results are discarded.  A load under a branch makes the compiler's
// wait-count merge at the join assume nothing is known about the loads in
// flight and emit vmcnt(0), which would also wait for the prefetched row.
// A scheduling barrier follows every prefetch so that the machine scheduler
// cannot hoist the current row's arithmetic (and its waits) above it.
template <int VPL, int NT>
struct RawRow {
  u32x4 v[NT][VPL];
};

__device__ __forceinline__ int64_t clamp_row(int64_t row, int64_t M) { return row < M ? row : M - 1; }

template <int VPL, int NT>
__device__ __forceinline__ void load_raw(RawRow<VPL, NT>& r, const uint16_t* const (&base)[3],
                                         const int64_t (&strides)[3], int64_t row, int64_t col) {
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const uint16_t* p = base[t] + row * strides[t] + col;
#pragma unroll
    for (int i = 0; i < VPL; ++i) r.v[t][i] = ld16_stream(p + i * 512);
  }
}

// The same with cacheable loads, for gathered rows: Zipf-repeated ids re-read
// the same table rows, which L2 / MALL then serve (at C3 the non-temporal
// loads above took the fused gather + norm 42.3 us, these 34.1 us).
template <int VPL, int NT>
__device__ __forceinline__ void load_raw_cached(RawRow<VPL, NT>& r, const uint16_t* const (&base)[3],
                                                const int64_t (&strides)[3], int64_t row, int64_t col) {
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const uint16_t* p = base[t] + row * strides[t] + col;
#pragma unroll
    for (int i = 0; i < VPL; ++i) r.v[t][i] = ld16(p + i * 512);
  }
}

// bf16 running sum of the terms, each add rounded as an eager bf16 add.Tensor.
template <int VPL, int NT>
__device__ __forceinline__ void sum_raw(u32x4 (&out)[VPL], const RawRow<VPL, NT>& r) {
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    u32x4 acc = r.v[0][i];
#pragma unroll
    for (int t = 1; t < NT; ++t) acc = add_bf8(acc, r.v[t][i]);
    out[i] = acc;
  }
}

template <int VPL>
__device__ __forceinline__ void load_weight(u32x4 (&wv)[VPL], const uint16_t* w, int64_t seg_len, int64_t seg_stride,
                                            int64_t col) {
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    if (w) {
      wv[i] = ld16(w + w_index(col + i * 512, seg_len, seg_stride));
    } else {
      wv[i] = u32x4{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};  // bf16 1.0
    }
  }
}

// ------------------------------------------------------------------ forward
// One row (this wave's column segment of it): bf16 term sum, sum of squares,
// cross-wave combine, y = bf16(h * rstd * w), optional h and rstd stores.
// The summed row is unpacked to fp32 once for both passes and the weight
// stays in fp32 registers for the whole kernel (see bwd_row).
template <int VPL, int WPR, int NX, bool GATHER>
__device__ __forceinline__ void fwd_row(const RmsFwdArgs& a, const RawRow<VPL, NX>& cur, bool id_ok,
                                        const float (&wf)[VPL * 8], float (&red)[2][4], int64_t row, int64_t col,
                                        int lane, int wave, int part, int rloc, int it) {
  const bool valid = row < a.M;
  u32x4 hv[VPL];
  sum_raw<VPL, NX>(hv, cur);
  if constexpr (GATHER) {
    if (!id_ok) {
#pragma unroll
      for (int i = 0; i < VPL; ++i) hv[i] = u32x4{0u, 0u, 0u, 0u};
      if (valid && part == 0 && lane == 0 && a.err) *a.err = 1;
    }
  }
  float hf[VPL * 8];
#pragma unroll
  for (int i = 0; i < VPL; ++i) unpack8(hv[i], hf + i * 8);
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < VPL * 8; ++j) ss = fmaf(hf[j], hf[j], ss);
  ss = wave_sum(ss);
  if constexpr (WPR > 1) {
    if (lane == 0) red[it & 1][wave] = ss;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int p = 0; p < WPR; ++p) t += red[it & 1][rloc * WPR + p];
    ss = t;
  }
  const float r = 1.0f / sqrtf(ss / (float)a.N + a.eps);
  if (valid) {
    uint16_t* yrow = a.y + row * a.ys + col;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (hf[i * 8 + e] * r) * wf[i * 8 + e];
      st16_stream(yrow + i * 512, pack8(o));
    }
    if ((NX > 1 || GATHER) && a.h != nullptr) {
      uint16_t* hrow = a.h + row * a.hs + col;
#pragma unroll
      for (int i = 0; i < VPL; ++i) st16_stream(hrow + i * 512, hv[i]);
    }
    if (a.rstd != nullptr && part == 0 && lane == 0) a.rstd[row] = r;
  }
}

// Blocks walk the row groups grid-stride (measured faster on gfx950 than
// contiguous per-block ranges for these row loops) with one row group of loads
// in flight ahead of the one being reduced.  The two register slots are
// separate named variables, and the loop is unrolled two steps per pass so
// that no slot is ever copied: an array of slots indexed by the step ends up
// in scratch memory, and a slot copy makes the wave wait for the prefetch.
// Gathered rows: lane j of a wave holds the id of the wave's row at step
// kb + j (kb a multiple of 64), fetched by one vector load per 64 steps; a
// step reads its id with readlane.  Read inside the row loop instead, the id
// was a vector load (the loop's stores might alias it) whose wait drained the
// other slot's prefetched row loads as well.
__device__ __forceinline__ int64_t gather_fetch(const RmsFwdArgs& a, int64_t kb, int64_t nb, int64_t b, int64_t G,
                                                int RB, int rloc, int lane) {
  const int64_t k = kb + lane < nb ? kb + lane : nb - 1;
  const int64_t row = clamp_row((b + k * G) * RB + rloc, a.M);
  return a.idx_bytes == 8 ? static_cast<const int64_t*>(a.idx)[row]
                          : (int64_t) static_cast<const int32_t*>(a.idx)[row];
}
// The source row of step k: the id when in [0, idx_rows), else row 0 (always
// readable) with ok = false.
__device__ __forceinline__ int64_t gather_src(const RmsFwdArgs& a, int64_t idl, int64_t k, bool& ok) {
  const int j = (int)(k & 63);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)idl, j);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)idl >> 32), j);
  const int64_t id = (int64_t)(((uint64_t)hi << 32) | lo);
  ok = id >= 0 && id < a.idx_rows;
  return ok ? id : 0;
}

template <int VPL, int WPR, int NX, bool GATHER>
__global__ __launch_bounds__(kThreads) void rms_fwd_vec(RmsFwdArgs a) {
  constexpr int RB = 4 / WPR;
  constexpr int SEG = 512 * VPL;
  __shared__ float red[2][4];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int part = wave % WPR, rloc = wave / WPR;
  const int64_t col = (int64_t)part * SEG + lane * 8;

  // Rows of 4 waves run one block per row (a one-shot grid, three blocks per
  // CU): a new block waits ~1024 cycles before its loads, which paces the
  // refill of a CU's slots.  Measured at [16384, 8192], two x terms, on one
  // box: 171.0 us against 172.4 us without the pause, 174.2 us with half of
  // it, 171.4 us with twice it.
  if constexpr (WPR == 4) __builtin_amdgcn_s_sleep(16);
  float wf[VPL * 8];
  {
    u32x4 wv[VPL];
    load_weight<VPL>(wv, a.w, a.w_seg_len, a.w_seg_stride, col);
#pragma unroll
    for (int i = 0; i < VPL; ++i) unpack8(wv[i], wf + i * 8);
  }

  const int64_t ngroups = ceil_div_dev(a.M, RB);
  const int64_t G = gridDim.x;
  RawRow<VPL, NX> s0, s1;
  bool s0ok = true, s1ok = true;
  int it = 0;
#define KP_ROW(g) ((g) * RB + rloc)
#define KP_LOAD(S, g, kk)                                                                             \
  {                                                                                                   \
    int64_t src_ = clamp_row(KP_ROW(g), a.M);                                                         \
    if constexpr (GATHER) {                                                                           \
      if ((kk) > 0 && ((kk) & 63) == 0) idl = gather_fetch(a, (kk), nb, blockIdx.x, G, RB, rloc, lane); \
      src_ = gather_src(a, idl, (kk), S##ok);                                                         \
    }                                                                                                 \
    if constexpr (GATHER) load_raw_cached<VPL, NX>(S, a.x, a.xs, src_, col);                          \
    else load_raw<VPL, NX>(S, a.x, a.xs, src_, col);                                                  \
  }                                                                                                   \
  __builtin_amdgcn_sched_barrier(0)
#define KP_PROC(S, g)                                                                               \
  fwd_row<VPL, WPR, NX, GATHER>(a, S, S##ok, wf, red, KP_ROW(g), col, lane, wave, part, rloc, it); \
  ++it
  // Exact trip count: the grid never exceeds the row-group count, so every
  // block owns nb >= 1 groups and nothing is prefetched past its last one.
  const int64_t nb = block_trips(ngroups, blockIdx.x, G);
  int64_t idl = 0;
  if constexpr (GATHER) idl = gather_fetch(a, 0, nb, blockIdx.x, G, RB, rloc, lane);
  int64_t g = blockIdx.x, k = 0;
  KP_LOAD(s0, g, 0);
  for (; k + 2 < nb; k += 2, g += 2 * G) {
    KP_LOAD(s1, g + G, k + 1);
    KP_PROC(s0, g);
    KP_LOAD(s0, g + 2 * G, k + 2);
    KP_PROC(s1, g + G);
  }
  if (k + 1 < nb) {
    KP_LOAD(s1, g + G, k + 1);
    KP_PROC(s0, g);
    KP_PROC(s1, g + G);
  } else {
    KP_PROC(s0, g);
  }
#undef KP_ROW
#undef KP_LOAD
#undef KP_PROC
}

// ----------------------------------------------------------------- backward
// LDS image of one wave's per-column accumulators, same column layout as the row.
template <int VPL>
__device__ __forceinline__ void stash_acc(float* buf, int lane, const float (&acc)[VPL * 8]) {
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    *reinterpret_cast<f32x4*>(buf + i * 512 + lane * 8) = f32x4{acc[i * 8], acc[i * 8 + 1], acc[i * 8 + 2], acc[i * 8 + 3]};
    *reinterpret_cast<f32x4*>(buf + i * 512 + lane * 8 + 4) =
        f32x4{acc[i * 8 + 4], acc[i * 8 + 5], acc[i * 8 + 6], acc[i * 8 + 7]};
  }
}
template <int VPL>
__device__ __forceinline__ void add_acc(const float* buf, int lane, float (&acc)[VPL * 8]) {
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const f32x4 u = *reinterpret_cast<const f32x4*>(buf + i * 512 + lane * 8);
    const f32x4 v = *reinterpret_cast<const f32x4*>(buf + i * 512 + lane * 8 + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc[i * 8 + e] += u[e];
      acc[i * 8 + 4 + e] += v[e];
    }
  }
}

// Loads of one row group of the backward: x and dy terms, the residual
// gradient (RES) and the given rstd.  `row` is already clamped to M - 1 and
// nothing is predicated (see load_raw); without a given rstd the 4-byte load
// reads the row's own first x word instead (an L1 hit, never used).
template <int VPL, int NX, int NDY, bool RES, bool FWD>
__device__ __forceinline__ void bwd_load(RawRow<VPL, NX>& xr, RawRow<VPL, NDY>& dr, RawRow<VPL, 1>& rr, float& rq,
                                         const RmsBwdArgs& a, int64_t row, int64_t col) {
  load_raw<VPL, NX>(xr, a.x, a.xs, row, col);
  load_raw<VPL, NDY>(dr, a.dy, a.dys, row, col);
  if constexpr (RES) {
    const uint16_t* rrow = a.dxr + row * a.dxrs + col;
#pragma unroll
    for (int i = 0; i < VPL; ++i) rr.v[0][i] = ld16_stream(rrow + i * 512);
  }
  const float* rp = (!FWD && a.rstd != nullptr) ? a.rstd + row : reinterpret_cast<const float*>(a.x[0] + row * a.xs[0]);
  rq = *rp;
}

// One row of the backward: dx (with the residual epilogue) and this row's
// contribution dy * xhat to the per-column weight-gradient accumulators.
// The row's x and dy are unpacked to fp32 once and kept across both passes,
// and the weight stays in fp32 registers for the whole kernel: unpacking
// them again in the second pass (to save registers) made the loop ~16 VALU
// instructions per element against ~10 now, and the backward grids run one
// wave per SIMD, so the registers are free.
//
// FWD (fused forward + backward): rstd is recomputed from x here (never
// loaded), and the forward's outputs are stored from it as well -- y =
// bf16(xhat * w), the same expression as the forward kernel, h when there are
// several x terms, rstd -- so the chain's x is read once for both passes.
//
// KEEP: the row's dx (with the residual epilogue) is handed back in gout[]
// (the same packed bf16 chunks the store would write) instead of stored, for
// a consumer in the same kernel (the embedding backward of the chain).
template <int VPL, int WPR, int NX, int NDY, bool RES, int NW, bool FWD, bool KEEP = false, bool UNCOND = false>
__device__ __forceinline__ void bwd_row(const RmsBwdArgs& a, const RawRow<VPL, NX>& xr, const RawRow<VPL, NDY>& dr,
                                        const RawRow<VPL, 1>& rr, float rq, const float (&wf)[VPL * 8],
                                        float (&acc)[VPL * 8], float (&red)[2][NW][2], int64_t row, int64_t col,
                                        int lane, int wave, int rloc, int it, u32x4* gout = nullptr) {
  const bool valid = row < a.M;
  const float inv_n = 1.0f / (float)a.N;
  const bool have_rstd = !FWD && a.rstd != nullptr;
  float xf[VPL * 8], df[VPL * 8];
  u32x4 xv[VPL];
  {
    u32x4 dv[VPL];
    sum_raw<VPL, NX>(xv, xr);
    sum_raw<VPL, NDY>(dv, dr);
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      unpack8(xv[i], xf + i * 8);
      unpack8(dv[i], df + i * 8);
    }
  }
  // sum(x * g) and, when rstd is not supplied, sum(x^2), in one sweep.
  float sxg = 0.f, ss = 0.f;
#pragma unroll
  for (int j = 0; j < VPL * 8; ++j) {
    sxg = fmaf(xf[j], df[j] * wf[j], sxg);
    ss = fmaf(xf[j], xf[j], ss);
  }
  sxg = wave_sum(sxg);
  if (!have_rstd) ss = wave_sum(ss);
  if constexpr (WPR > 1) {
    if (lane == 0) {
      red[it & 1][wave][0] = sxg;
      red[it & 1][wave][1] = ss;
    }
    __syncthreads();
    float t0 = 0.f, t1 = 0.f;
#pragma unroll
    for (int p = 0; p < WPR; ++p) {
      t0 += red[it & 1][rloc * WPR + p][0];
      t1 += red[it & 1][rloc * WPR + p][1];
    }
    sxg = t0;
    ss = t1;
  }
  const float r = have_rstd ? rq : 1.0f / sqrtf(ss / (float)a.N + a.eps);
  // sum(xhat * g) = r * sum(x * g);  dx = (g - xhat * sum/N) * r
  const float cN = (r * sxg) * inv_n;
  if constexpr (UNCOND && !FWD && !KEEP) {
    // The stores are not under a branch (see rms_bwd_vec): this form only
    // runs rows below M.
    uint16_t* dxrow = a.dx + row * a.dxs + col;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int j = i * 8 + e;
        const float xh = xf[j] * r;
        const float gg = df[j] * wf[j];
        o[e] = (gg - xh * cN) * r;
        acc[j] = fmaf(df[j], xh, acc[j]);
      }
      u32x4 ov = pack8(o);
      if constexpr (RES) ov = add_bf8(rr.v[0][i], ov);
      st16_stream(dxrow + i * 512, ov);
    }
    return;
  }
  if (valid) {
    if constexpr (FWD) {
      uint16_t* yrow = a.y + row * a.ys + col;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = (xf[i * 8 + e] * r) * wf[i * 8 + e];
        st16_stream(yrow + i * 512, pack8(o));
      }
      if constexpr (NX > 1) {
        if (a.h != nullptr) {
          uint16_t* hrow = a.h + row * a.hs + col;
#pragma unroll
          for (int i = 0; i < VPL; ++i) st16_stream(hrow + i * 512, xv[i]);
        }
      }
      if (a.rstd_out != nullptr && wave % WPR == 0 && lane == 0) a.rstd_out[row] = r;
    }
    uint16_t* dxrow = KEEP ? nullptr : a.dx + row * a.dxs + col;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int j = i * 8 + e;
        const float xh = xf[j] * r;
        const float gg = df[j] * wf[j];
        o[e] = (gg - xh * cN) * r;
        acc[j] = fmaf(df[j], xh, acc[j]);
      }
      u32x4 ov = pack8(o);
      if constexpr (RES) ov = add_bf8(rr.v[0][i], ov);
      if constexpr (KEEP) {
        gout[i] = ov;
      } else {
        st16_stream(dxrow + i * 512, ov);
      }
    }
  }
}

// Grid-stride over row groups with one group of loads in flight, in two named
// register slots (see rms_fwd_vec).  NW waves per block (4 or 8): RB = NW / WPR
// rows per block step; every block owns one weight-gradient partial row.
// The block's timeline record (kp_debug_block_trace): start, rows done,
// partial row stored (constant 100 MHz clock), XCC id; written by thread 0.
__device__ __forceinline__ void trace_block(const RmsBwdArgs& a, unsigned long long t_start,
                                            unsigned long long t_rows) {
  __builtin_amdgcn_s_waitcnt(0);
  const unsigned long long t_end = __builtin_amdgcn_s_memrealtime();
  if (threadIdx.x == 0 && (int)blockIdx.x < a.trace_blocks) {
    unsigned xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    unsigned long long* d = a.trace + (size_t)blockIdx.x * 4;
    d[0] = t_start;
    d[1] = t_rows;
    d[2] = t_end;
    d[3] = xcc;
  }
}

template <int VPL, int WPR, int NX, int NDY, bool RES, int NW, bool FWD>
__global__ __launch_bounds__(NW * 64) void rms_bwd_vec(RmsBwdArgs a) {
  constexpr int RB = NW / WPR;
  constexpr bool kExact = NW == 4 && !FWD;  // exact wait counts (see the row loop)
  constexpr int SEG = 512 * VPL;
  extern __shared__ float smem[];  // [RB / 2][WPR][SEG] weight-gradient combine (only when a.partial)
  __shared__ float red[2][NW][2];
  const unsigned long long t_start = a.trace != nullptr ? __builtin_amdgcn_s_memrealtime() : 0ull;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int part = wave % WPR, rloc = wave / WPR;
  const int64_t col = (int64_t)part * SEG + lane * 8;

  float wf[VPL * 8];
  {
    u32x4 wv[VPL];
    load_weight<VPL>(wv, a.w, a.w_seg_len, a.w_seg_stride, col);
#pragma unroll
    for (int i = 0; i < VPL; ++i) unpack8(wv[i], wf + i * 8);
  }

  float acc[VPL * 8];
#pragma unroll
  for (int i = 0; i < VPL * 8; ++i) acc[i] = 0.f;

  const int64_t ngroups = ceil_div_dev(a.M, RB);
  const int64_t G = gridDim.x;
  RawRow<VPL, NX> x0, x1;
  RawRow<VPL, NDY> d0, d1;
  RawRow<VPL, 1> r0, r1;
  float q0, q1;
  int it = 0;
#define KP_ROW(g) ((g) * RB + rloc)
#define KP_LOAD(S, g)                                                                       \
  bwd_load<VPL, NX, NDY, RES, FWD>(x##S, d##S, r##S, q##S, a, clamp_row(KP_ROW(g), a.M), col); \
  __builtin_amdgcn_sched_barrier(0)
#define KP_PROC(S, g)                                                                                             \
  bwd_row<VPL, WPR, NX, NDY, RES, NW, FWD, false, kExact>(a, x##S, d##S, r##S, q##S, wf, acc, red, KP_ROW(g), col, \
                                                          lane, wave, rloc, it);                                     \
  ++it
  int64_t g = blockIdx.x, k = 0;
  if constexpr (kExact) {
    // The loop walks the full row groups only, stores unbranched (every row
    // < M), and is entered after the first group's stores, so that both paths
    // into its header (from the prologue and from the loop's end) hold the
    // same loads and stores in flight: every wait for a group's loads is
    // exact instead of also waiting for the previous group's stores (c2
    // kernel 34.7-34.8 -> 34.5-34.6 us).  A last group with rows past M is
    // its owner's last group anyway and runs after the loop with guarded
    // stores, so dw keeps its order and no row is written by a wave that did
    // not read it (dx may alias its inputs).  The 8-wave shapes (N = 8192)
    // keep the other form: there the store waits pace the 3-read loop (c5b
    // 174.7 against 180.9 us exact).
    const int64_t nfull = a.M / RB;
    const int64_t nb = (int64_t)blockIdx.x < nfull ? block_trips(nfull, blockIdx.x, G) : 0;
    if (nb >= 2) {
      KP_LOAD(0, g);
      KP_LOAD(1, g + G);
      KP_PROC(0, g);
      for (; k + 3 < nb; k += 2, g += 2 * G) {
        KP_LOAD(0, g + 2 * G);
        KP_PROC(1, g + G);
        KP_LOAD(1, g + 3 * G);
        KP_PROC(0, g + 2 * G);
      }
      if (k + 2 < nb) {
        KP_LOAD(0, g + 2 * G);
        KP_PROC(1, g + G);
        KP_PROC(0, g + 2 * G);
      } else {
        KP_PROC(1, g + G);
      }
    } else if (nb == 1) {
      KP_LOAD(0, g);
      KP_PROC(0, g);
    }
    if (nfull < ngroups && (ngroups - 1) % G == (int64_t)blockIdx.x) {
      const int64_t gl = ngroups - 1;
      KP_LOAD(0, gl);
      bwd_row<VPL, WPR, NX, NDY, RES, NW, FWD>(a, x0, d0, r0, q0, wf, acc, red, KP_ROW(gl), col, lane, wave, rloc, it);
      ++it;
    }
  } else {
    // Exact trip count (see rms_fwd_vec): nb >= 1 groups per block.
    const int64_t nb = block_trips(ngroups, blockIdx.x, G);
    KP_LOAD(0, g);
    for (; k + 2 < nb; k += 2, g += 2 * G) {
      KP_LOAD(1, g + G);
      KP_PROC(0, g);
      KP_LOAD(0, g + 2 * G);
      KP_PROC(1, g + G);
    }
    if (k + 1 < nb) {
      KP_LOAD(1, g + G);
      KP_PROC(0, g);
      KP_PROC(1, g + G);
    } else {
      KP_PROC(0, g);
    }
  }
#undef KP_ROW
#undef KP_LOAD
#undef KP_PROC
  unsigned long long t_rows = 0;
  if (a.trace != nullptr) {
    __builtin_amdgcn_s_waitcnt(0);
    t_rows = __builtin_amdgcn_s_memrealtime();
  }

  if (a.partial == nullptr) {
    if (a.trace != nullptr) trace_block(a, t_start, t_rows);
    return;
  }
  // Combine the column partials of the RB waves that share a column segment
  // with a fixed pairwise tree (level `step`: rloc r += rloc r + step), through
  // [RB / 2][WPR][SEG] floats of LDS, then write one partial row per block.
#pragma unroll
  for (int step = RB / 2; step >= 1; step /= 2) {
    if (rloc >= step && rloc < 2 * step) stash_acc<VPL>(smem + ((rloc - step) * WPR + part) * SEG, lane, acc);
    __syncthreads();
    if (rloc < step) add_acc<VPL>(smem + (rloc * WPR + part) * SEG, lane, acc);
    __syncthreads();
  }
  if (rloc == 0) {
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      // 8 consecutive columns, 8-aligned: inside one 16-column chunk
      float* pp = a.partial + part_index(col + i * 512, blockIdx.x, gridDim.x);
      *reinterpret_cast<f32x4*>(pp) = f32x4{acc[i * 8], acc[i * 8 + 1], acc[i * 8 + 2], acc[i * 8 + 3]};
      *reinterpret_cast<f32x4*>(pp + 4) = f32x4{acc[i * 8 + 4], acc[i * 8 + 5], acc[i * 8 + 6], acc[i * 8 + 7]};
    }
  }
  if (a.trace != nullptr) trace_block(a, t_start, t_rows);
}


typedef void (*FwdKernel)(RmsFwdArgs);
typedef void (*BwdKernel)(RmsBwdArgs);

// Kernel instantiations live in several translation units so that they
// compile in parallel: kp_rms_fwd.hip holds every forward shape, and
// kp_rms_bwd_<VPL>.hip the backward shapes with VPL chunks per lane.
// Each getter returns nullptr for a shape or term combination it lacks.
FwdKernel fwd_kernel(int vpl, int wpr, int nx);
// Gather variants (one term, row ids): kp_rms_fwd_gather.hip.
FwdKernel fwd_gather_kernel(int vpl, int wpr);
// fwd = true selects the fused forward + backward variant (FWD).
BwdKernel bwd_kernel_vpl1(int wpr, int nx, int ndy, bool res, bool fwd);
BwdKernel bwd_kernel_vpl2(int wpr, int nx, int ndy, bool res, bool fwd);
BwdKernel bwd_kernel_vpl3(int wpr, int nx, int ndy, bool res, bool fwd);
BwdKernel bwd_kernel_vpl4(int wpr, int nx, int ndy, bool res, bool fwd);
BwdKernel bwd_kernel_vpl5(int wpr, int nx, int ndy, bool res, bool fwd);
BwdKernel bwd_kernel_vpl68(int vpl, int wpr, int nx, int ndy, bool res, bool fwd);

template <int VPL, int WPR>
FwdKernel fwd_for_terms(int nx) {
  switch (nx) {
    case 1: return rms_fwd_vec<VPL, WPR, 1, false>;
    case 2: return rms_fwd_vec<VPL, WPR, 2, false>;
    case 3: return rms_fwd_vec<VPL, WPR, 3, false>;
  }
  return nullptr;
}
// Term combinations of the backward fast path (x terms, dy terms, residual
// epilogue) -- the ones the configurations and reference fragments use;
// others run the generic kernel.
// The fused forward + backward variants cover the chain fragments' terms:
// (1 x, 1..3 dy, +- residual) and (2 x, 2 dy, residual).  NW waves per block
// (4, or 8 for the 8-waves-per-row shape of N = 8192).
template <int VPL, int WPR, int NW = kThreads / 64>
BwdKernel bwd_for_terms(int nx, int ndy, bool res, bool fwd) {
  if (fwd) {
    if (!res) {
      if (nx == 1 && ndy == 1) return rms_bwd_vec<VPL, WPR, 1, 1, false, NW, true>;
    } else {
      if (nx == 1 && ndy == 1) return rms_bwd_vec<VPL, WPR, 1, 1, true, NW, true>;
      if (nx == 1 && ndy == 2) return rms_bwd_vec<VPL, WPR, 1, 2, true, NW, true>;
      if (nx == 1 && ndy == 3) return rms_bwd_vec<VPL, WPR, 1, 3, true, NW, true>;
      if (nx == 2 && ndy == 2) return rms_bwd_vec<VPL, WPR, 2, 2, true, NW, true>;
    }
    return nullptr;
  }
  if (!res) {
    if (nx == 1 && ndy == 1) return rms_bwd_vec<VPL, WPR, 1, 1, false, NW, false>;
    if (nx == 1 && ndy == 2) return rms_bwd_vec<VPL, WPR, 1, 2, false, NW, false>;
    if (nx == 1 && ndy == 3) return rms_bwd_vec<VPL, WPR, 1, 3, false, NW, false>;
    if (nx == 2 && ndy == 1) return rms_bwd_vec<VPL, WPR, 2, 1, false, NW, false>;
    if (nx == 3 && ndy == 1) return rms_bwd_vec<VPL, WPR, 3, 1, false, NW, false>;
    if (nx == 2 && ndy == 2) return rms_bwd_vec<VPL, WPR, 2, 2, false, NW, false>;
  } else {
    if (nx == 1 && ndy == 1) return rms_bwd_vec<VPL, WPR, 1, 1, true, NW, false>;
    if (nx == 1 && ndy == 2) return rms_bwd_vec<VPL, WPR, 1, 2, true, NW, false>;
    if (nx == 1 && ndy == 3) return rms_bwd_vec<VPL, WPR, 1, 3, true, NW, false>;
    if (nx == 2 && ndy == 2) return rms_bwd_vec<VPL, WPR, 2, 2, true, NW, false>;
  }
  return nullptr;
}

}  // namespace rms
}  // namespace kp
