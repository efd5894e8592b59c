// RMSNorm forward / backward for gfx950.
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
#include <stdlib.h>

#include "kp_common.hpp"
#include "kp_internal.hpp"

namespace kp {
namespace {

constexpr int kThreads = 256;  // 4 waves per block

struct RmsFwdArgs {
  const uint16_t* x[3];
  int64_t xs[3];
  int n_x;
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
  int64_t M, N;
  float eps;
};

// Weight-gradient partials are stored column-chunk-major, [ceil(N/32)][P][32]
// fp32 (P = row blocks): a block's partial row lands as full 128-byte lines
// and the finalize reads each 32-column chunk of all P rows contiguously.
constexpr int kPartChunk = 32;
__host__ __device__ __forceinline__ int64_t part_index(int64_t c, int64_t p, int64_t P) {
  return ((c / kPartChunk) * P + p) * kPartChunk + (c % kPartChunk);
}

__device__ __forceinline__ int64_t w_index(int64_t c, int64_t seg_len, int64_t seg_stride) {
  return (c / seg_len) * seg_stride + (c % seg_len);
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
template <int VPL, int WPR, int NX>
__device__ __forceinline__ void fwd_row(const RmsFwdArgs& a, const RawRow<VPL, NX>& cur, u32x4 (&wv)[VPL],
                                        float (&red)[2][4], int64_t row, int64_t col, int lane, int wave, int part,
                                        int rloc, int it) {
  const bool valid = row < a.M;
  u32x4 hv[VPL];
  sum_raw<VPL, NX>(hv, cur);
#pragma unroll
  for (int i = 0; i < VPL; ++i) reg_barrier(wv[i]);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    float f[8];
    unpack8(hv[i], f);
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = fmaf(f[e], f[e], ss);
  }
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
#pragma unroll
  for (int i = 0; i < VPL; ++i) reg_barrier(hv[i]);
  if (valid) {
    uint16_t* yrow = a.y + row * a.ys + col;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      float f[8], wf[8], o[8];
      unpack8(hv[i], f);
      unpack8(wv[i], wf);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (f[e] * r) * wf[e];
      st16_stream(yrow + i * 512, pack8(o));
    }
    if (NX > 1 && a.h != nullptr) {
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
template <int VPL, int WPR, int NX>
__global__ __launch_bounds__(kThreads) void rms_fwd_vec(RmsFwdArgs a) {
  constexpr int RB = 4 / WPR;
  constexpr int SEG = 512 * VPL;
  __shared__ float red[2][4];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int part = wave % WPR, rloc = wave / WPR;
  const int64_t col = (int64_t)part * SEG + lane * 8;

  u32x4 wv[VPL];
  load_weight<VPL>(wv, a.w, a.w_seg_len, a.w_seg_stride, col);

  const int64_t ngroups = ceil_div_dev(a.M, RB);
  const int64_t G = gridDim.x;
  RawRow<VPL, NX> s0, s1;
  int it = 0;
#define KP_ROW(g) ((g) * RB + rloc)
#define KP_LOAD(S, g)                                              \
  load_raw<VPL, NX>(S, a.x, a.xs, clamp_row(KP_ROW(g), a.M), col); \
  __builtin_amdgcn_sched_barrier(0)
#define KP_PROC(S, g)                                                               \
  fwd_row<VPL, WPR, NX>(a, S, wv, red, KP_ROW(g), col, lane, wave, part, rloc, it); \
  ++it
  // Exact trip count: the grid never exceeds the row-group count, so every
  // block owns nb >= 1 groups and nothing is prefetched past its last one.
  const int64_t nb = (ngroups - 1 - blockIdx.x) / G + 1;
  int64_t g = blockIdx.x, k = 0;
  KP_LOAD(s0, g);
  for (; k + 2 < nb; k += 2, g += 2 * G) {
    KP_LOAD(s1, g + G);
    KP_PROC(s0, g);
    KP_LOAD(s0, g + 2 * G);
    KP_PROC(s1, g + G);
  }
  if (k + 1 < nb) {
    KP_LOAD(s1, g + G);
    KP_PROC(s0, g);
    KP_PROC(s1, g + G);
  } else {
    KP_PROC(s0, g);
  }
#undef KP_ROW
#undef KP_LOAD
#undef KP_PROC
}

// Any N, any alignment: one block per row, scalar accesses, two passes.
__device__ __forceinline__ float term_sum_scalar(const uint16_t* const* base, const int64_t* strides, int n,
                                                 int64_t row, int64_t c) {
  float v = bf_to_f(base[0][row * strides[0] + c]);
  if (n > 1) v = round_bf(v + bf_to_f(base[1][row * strides[1] + c]));
  if (n > 2) v = round_bf(v + bf_to_f(base[2][row * strides[2] + c]));
  return v;
}

__device__ __forceinline__ float block_sum(float v, float* red4) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = wave_sum(v);
  __syncthreads();  // red4 may still be read from the previous call
  if (lane == 0) red4[wave] = v;
  __syncthreads();
  return (red4[0] + red4[1]) + (red4[2] + red4[3]);
}

__global__ __launch_bounds__(kThreads) void rms_fwd_generic(RmsFwdArgs a) {
  __shared__ float red[4];
  for (int64_t row = blockIdx.x; row < a.M; row += gridDim.x) {
    float ss = 0.f;
    for (int64_t c = threadIdx.x; c < a.N; c += kThreads) {
      const float v = term_sum_scalar(a.x, a.xs, a.n_x, row, c);
      ss = fmaf(v, v, ss);
    }
    ss = block_sum(ss, red);
    const float r = 1.0f / sqrtf(ss / (float)a.N + a.eps);
    for (int64_t c = threadIdx.x; c < a.N; c += kThreads) {
      const float v = term_sum_scalar(a.x, a.xs, a.n_x, row, c);
      const float wf = a.w ? bf_to_f(a.w[w_index(c, a.w_seg_len, a.w_seg_stride)]) : 1.0f;
      a.y[row * a.ys + c] = f_to_bf((v * r) * wf);
      if (a.h != nullptr && a.n_x > 1) a.h[row * a.hs + c] = f_to_bf(v);
    }
    if (a.rstd != nullptr && threadIdx.x == 0) a.rstd[row] = r;
  }
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
template <int VPL, int NX, int NDY, bool RES>
__device__ __forceinline__ void bwd_load(RawRow<VPL, NX>& xr, RawRow<VPL, NDY>& dr, RawRow<VPL, 1>& rr, float& rq,
                                         const RmsBwdArgs& a, int64_t row, int64_t col) {
  load_raw<VPL, NX>(xr, a.x, a.xs, row, col);
  load_raw<VPL, NDY>(dr, a.dy, a.dys, row, col);
  if constexpr (RES) {
    const uint16_t* rrow = a.dxr + row * a.dxrs + col;
#pragma unroll
    for (int i = 0; i < VPL; ++i) rr.v[0][i] = ld16_stream(rrow + i * 512);
  }
  const float* rp = a.rstd != nullptr ? a.rstd + row : reinterpret_cast<const float*>(a.x[0] + row * a.xs[0]);
  rq = *rp;
}

// One row of the backward: dx (with the residual epilogue) and this row's
// contribution dy * xhat to the per-column weight-gradient accumulators.
template <int VPL, int WPR, int NX, int NDY, bool RES, int NW>
__device__ __forceinline__ void bwd_row(const RmsBwdArgs& a, const RawRow<VPL, NX>& xr, const RawRow<VPL, NDY>& dr,
                                        const RawRow<VPL, 1>& rr, float rq, u32x4 (&wv)[VPL], float (&acc)[VPL * 8],
                                        float (&red)[2][NW][2], int64_t row, int64_t col, int lane, int wave, int rloc,
                                        int it) {
  const bool valid = row < a.M;
  const float inv_n = 1.0f / (float)a.N;
  u32x4 xv[VPL], dv[VPL];
  sum_raw<VPL, NX>(xv, xr);
  sum_raw<VPL, NDY>(dv, dr);
#pragma unroll
  for (int i = 0; i < VPL; ++i) reg_barrier(wv[i]);
  // sum(x * g) and, when rstd is not supplied, sum(x^2), in one sweep.
  float sxg = 0.f, ss = 0.f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    float xf[8], df[8], wf[8];
    unpack8(xv[i], xf);
    unpack8(dv[i], df);
    unpack8(wv[i], wf);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      sxg = fmaf(xf[e], df[e] * wf[e], sxg);
      ss = fmaf(xf[e], xf[e], ss);
    }
  }
  sxg = wave_sum(sxg);
  if (a.rstd == nullptr) ss = wave_sum(ss);
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
  const float r = (a.rstd != nullptr) ? rq : 1.0f / sqrtf(ss / (float)a.N + a.eps);
  // sum(xhat * g) = r * sum(x * g);  dx = (g - xhat * sum/N) * r
  const float cN = (r * sxg) * inv_n;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    reg_barrier(xv[i]);
    reg_barrier(dv[i]);
    reg_barrier(wv[i]);
  }
  if (valid) {
    uint16_t* dxrow = a.dx + row * a.dxs + col;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      float xf[8], df[8], wf[8], o[8];
      unpack8(xv[i], xf);
      unpack8(dv[i], df);
      unpack8(wv[i], wf);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float xh = xf[e] * r;
        const float gg = df[e] * wf[e];
        o[e] = (gg - xh * cN) * r;
        acc[i * 8 + e] = fmaf(df[e], xh, acc[i * 8 + e]);
      }
      u32x4 ov = pack8(o);
      if constexpr (RES) ov = add_bf8(rr.v[0][i], ov);
      st16_stream(dxrow + i * 512, ov);
    }
  }
}

// Grid-stride over row groups with one group of loads in flight, in two named
// register slots (see rms_fwd_vec).  NW waves per block (4 or 8): RB = NW / WPR
// rows per block step; every block owns one weight-gradient partial row.
template <int VPL, int WPR, int NX, int NDY, bool RES, int NW>
__global__ __launch_bounds__(NW * 64) void rms_bwd_vec(RmsBwdArgs a) {
  constexpr int RB = NW / WPR;
  constexpr int SEG = 512 * VPL;
  extern __shared__ float smem[];  // [RB / 2][WPR][SEG] weight-gradient combine (only when a.partial)
  __shared__ float red[2][NW][2];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int part = wave % WPR, rloc = wave / WPR;
  const int64_t col = (int64_t)part * SEG + lane * 8;

  u32x4 wv[VPL];
  load_weight<VPL>(wv, a.w, a.w_seg_len, a.w_seg_stride, col);

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
  bwd_load<VPL, NX, NDY, RES>(x##S, d##S, r##S, q##S, a, clamp_row(KP_ROW(g), a.M), col); \
  __builtin_amdgcn_sched_barrier(0)
#define KP_PROC(S, g)                                                                                               \
  bwd_row<VPL, WPR, NX, NDY, RES, NW>(a, x##S, d##S, r##S, q##S, wv, acc, red, KP_ROW(g), col, lane, wave, rloc, it); \
  ++it
  // Exact trip count (see rms_fwd_vec): nb >= 1 groups per block.
  const int64_t nb = (ngroups - 1 - blockIdx.x) / G + 1;
  int64_t g = blockIdx.x, k = 0;
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
#undef KP_ROW
#undef KP_LOAD
#undef KP_PROC

  if (a.partial == nullptr) return;
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
      // 8 consecutive columns, 8-aligned: inside one 32-column chunk
      float* pp = a.partial + part_index(col + i * 512, blockIdx.x, gridDim.x);
      *reinterpret_cast<f32x4*>(pp) = f32x4{acc[i * 8], acc[i * 8 + 1], acc[i * 8 + 2], acc[i * 8 + 3]};
      *reinterpret_cast<f32x4*>(pp + 4) = f32x4{acc[i * 8 + 4], acc[i * 8 + 5], acc[i * 8 + 6], acc[i * 8 + 7]};
    }
  }
}

// Any N, any alignment: one block per row, scalar accesses.  The block's
// weight-gradient partial row lives directly in `partial` (read-modify-write,
// owned by this block only; same chunked layout as the vector kernel).
__global__ __launch_bounds__(kThreads) void rms_bwd_generic(RmsBwdArgs a) {
  __shared__ float red[4];
  float* part = a.partial;
  const int64_t P = gridDim.x;
  if (part)
    for (int64_t c = threadIdx.x; c < a.N; c += kThreads) part[part_index(c, blockIdx.x, P)] = 0.f;
  const float inv_n = 1.0f / (float)a.N;
  for (int64_t row = blockIdx.x; row < a.M; row += gridDim.x) {
    float sxg = 0.f, ss = 0.f;
    for (int64_t c = threadIdx.x; c < a.N; c += kThreads) {
      const float xf = term_sum_scalar(a.x, a.xs, a.n_x, row, c);
      const float df = term_sum_scalar(a.dy, a.dys, a.n_dy, row, c);
      const float wf = a.w ? bf_to_f(a.w[w_index(c, a.w_seg_len, a.w_seg_stride)]) : 1.0f;
      sxg = fmaf(xf, df * wf, sxg);
      ss = fmaf(xf, xf, ss);
    }
    sxg = block_sum(sxg, red);
    float r;
    if (a.rstd != nullptr) {
      r = a.rstd[row];
    } else {
      ss = block_sum(ss, red);
      r = 1.0f / sqrtf(ss / (float)a.N + a.eps);
    }
    const float cN = (r * sxg) * inv_n;
    for (int64_t c = threadIdx.x; c < a.N; c += kThreads) {
      const float xf = term_sum_scalar(a.x, a.xs, a.n_x, row, c);
      const float df = term_sum_scalar(a.dy, a.dys, a.n_dy, row, c);
      const float wf = a.w ? bf_to_f(a.w[w_index(c, a.w_seg_len, a.w_seg_stride)]) : 1.0f;
      const float xh = xf * r;
      float o = round_bf((df * wf - xh * cN) * r);
      if (a.dxr) o = bf_to_f(a.dxr[row * a.dxrs + c]) + o;
      a.dx[row * a.dxs + c] = f_to_bf(o);
      if (part) {
        float& pc = part[part_index(c, blockIdx.x, P)];
        pc = fmaf(df, xh, pc);
      }
    }
  }
}

// dw[c] = sum_{p < P} partial[p, c].  A block owns one 32-column chunk, whose
// P partial rows are contiguous ([P][32] fp32).  Thread (r, q) sums columns
// 4q..4q+3 over rows r, r + 32, r + 64, ... in row order; the 32 row-group
// sums are then added in group order.  Loads go out in batches of 8 rows.
constexpr int kFinGroups = kThreads / (kPartChunk / 4);  // 32

__global__ __launch_bounds__(kThreads) void rms_dw_finalize(const float* __restrict__ partial, int P, int64_t N,
                                                            float* dw_f32, uint16_t* dw_bf16, int round_f32) {
  __shared__ float s[kFinGroups][kPartChunk + 1];
  const int q = threadIdx.x & 7, r = threadIdx.x >> 3;
  const int64_t c0 = (int64_t)blockIdx.x * kPartChunk;
  const float* base = partial + (int64_t)blockIdx.x * P * kPartChunk;
  const int ncol = (int)(N - c0 < kPartChunk ? N - c0 : kPartChunk);
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  if (ncol == kPartChunk) {
    int p = r;
    for (; p + 7 * kFinGroups < P; p += 8 * kFinGroups) {
      f32x4 v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k)
        v[k] = *reinterpret_cast<const f32x4*>(base + (int64_t)(p + k * kFinGroups) * kPartChunk + q * 4);
#pragma unroll
      for (int k = 0; k < 8; ++k) acc += v[k];
    }
    for (; p < P; p += kFinGroups) acc += *reinterpret_cast<const f32x4*>(base + (int64_t)p * kPartChunk + q * 4);
  } else {
    for (int k = 0; k < 4; ++k) {
      if (q * 4 + k < ncol) {
        float t = 0.f;
        for (int p = r; p < P; p += kFinGroups) t += base[(int64_t)p * kPartChunk + q * 4 + k];
        acc[k] = t;
      }
    }
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) s[r][q * 4 + k] = acc[k];
  __syncthreads();
  if (threadIdx.x < ncol) {
    float t = s[0][threadIdx.x];
    for (int g = 1; g < kFinGroups; ++g) t += s[g][threadIdx.x];
    const int64_t c = c0 + threadIdx.x;
    if (dw_bf16) dw_bf16[c] = f_to_bf(t);
    if (dw_f32) dw_f32[c] = round_f32 ? round_bf(t) : t;
  }
}

// ------------------------------------------------------------------- dispatch
// Fast path shape: N = 512 * VPL * WPR with WPR in {1, 2, 4}.  Fewer chunks
// per lane (VPL <= 4, at most ~120 VGPRs) keep 4 waves per SIMD resident; a
// wider row is split over more waves instead.  VPL up to 8 is the fallback.
int env_int(const char* name, int dflt, int lo, int hi) {
  const char* e = getenv(name);
  const int v = e ? atoi(e) : dflt;
  return (v >= lo && v <= hi) ? v : dflt;
}
// Row blocks per CU for the pipelined row kernels: enough blocks that the
// row loads in flight per CU (waves x 2 slots x bytes per wave slot) come to
// about `target` bytes.  Measured on MI355X (kernel time, 4-wave blocks): the
// forward is best near 128 KiB per CU ([4096, 4096]: 2 blocks 12.8 us, 1 block
// 15.0 us); the backward near 64-96 KiB ([8192, 4096]: 1 block 36.7 us, 2
// blocks 37.7 us, 3 blocks 42.2 us; [16384, 8192] with 3 input streams: 1
// block 177 us, 2 blocks 187 us) -- more loads in flight only add DRAM
// contention there, and fewer blocks also mean fewer weight-gradient partials.
int auto_bpc(int waves_per_block, int64_t wave_slot_bytes, int64_t target, int max_bpc) {
  const int64_t per_block = (int64_t)waves_per_block * 2 * wave_slot_bytes;
  const int v = (int)((target + per_block / 2) / per_block);
  return v < 1 ? 1 : (v > max_bpc ? max_bpc : v);
}
// Launch-shape tuning knobs (read once): KP_RMS_FWD_BPC / KP_RMS_BWD_BPC, row
// blocks per CU for the forward / backward grids (0 or unset: auto_bpc).
int fwd_bpc(int64_t wave_slot_bytes) {
  static const int v = env_int("KP_RMS_FWD_BPC", 0, 0, 64);
  return v ? v : auto_bpc(4, wave_slot_bytes, 128 * 1024, 8);
}
// Backward block shape: KP_RMS_BWD_WAVES waves per block (4 or 8).
int bwd_waves() {
  static const int v = env_int("KP_RMS_BWD_WAVES", 4, 4, 8) == 8 ? 8 : 4;
  return v;
}
// At most 4 blocks per CU: the workspace holds one partial row per block.
int bwd_bpc(int64_t wave_slot_bytes) {
  static const int v = env_int("KP_RMS_BWD_BPC", 0, 0, 4);
  return v ? v : auto_bpc(bwd_waves(), wave_slot_bytes, 64 * 1024, 4);
}

// Fast-path row shapes: N = 512 * VPL * WPR, at most 5 16-byte chunks per
// lane (pipelined kernels stay well under 256 VGPRs); wider rows are split
// over 2 or 4 waves.  KP_RMS_WPR_MIN (tuning knob) asks for at least that
// many waves per row where a shape exists.
int wpr_min() {
  static const int v = env_int("KP_RMS_WPR_MIN", 1, 1, 4);
  return v;
}
// Measured defaults (MI355X): the forward keeps a whole row in one wave up
// to 8 chunks per lane (N <= 4096; no cross-wave barrier), the backward --
// which also holds per-column weight-gradient accumulators -- at most 5.
// KP_RMS_VPL_MAX (tuning knob) overrides both.
int vpl_max(bool forward, int64_t N) {
  static const int v = env_int("KP_RMS_VPL_MAX", 0, 1, 8);
  if (v) return v;
  return (forward && N <= 4096) ? 8 : 5;
}
bool shape_ok(int vpl, int wpr) {
  switch (vpl * 10 + wpr) {
    case 11: case 21: case 31: case 41: case 51:
    case 12: case 22: case 32: case 42: case 52:
    case 14: case 24: case 34: case 44:
    case 61: case 81: case 82: return true;
  }
  return false;
}
bool pick_vec(int64_t N, bool forward, int* vpl, int* wpr) {
  if (N <= 0 || N % 512 != 0) return false;
  const int64_t k = N / 512;
  for (int pass = 0; pass < 2; ++pass) {
    for (int w : {1, 2, 4}) {
      if (pass == 0 && w < wpr_min()) continue;
      if (k % w == 0 && k / w <= vpl_max(forward, N) && shape_ok((int)(k / w), w)) {
        *vpl = (int)(k / w);
        *wpr = w;
        return true;
      }
    }
  }
  return false;
}

typedef void (*FwdKernel)(RmsFwdArgs);
typedef void (*BwdKernel)(RmsBwdArgs);

template <int VPL, int WPR>
FwdKernel fwd_for_terms(int nx) {
  switch (nx) {
    case 1: return rms_fwd_vec<VPL, WPR, 1>;
    case 2: return rms_fwd_vec<VPL, WPR, 2>;
    case 3: return rms_fwd_vec<VPL, WPR, 3>;
  }
  return nullptr;
}
// Term combinations of the backward fast path (x terms, dy terms, residual
// epilogue) -- the ones the configurations and reference fragments use;
// others run the generic kernel.
template <int VPL, int WPR, int NW>
BwdKernel bwd_for_terms_nw(int nx, int ndy, bool res) {
  if (!res) {
    if (nx == 1 && ndy == 1) return rms_bwd_vec<VPL, WPR, 1, 1, false, NW>;
    if (nx == 1 && ndy == 2) return rms_bwd_vec<VPL, WPR, 1, 2, false, NW>;
    if (nx == 1 && ndy == 3) return rms_bwd_vec<VPL, WPR, 1, 3, false, NW>;
    if (nx == 2 && ndy == 1) return rms_bwd_vec<VPL, WPR, 2, 1, false, NW>;
    if (nx == 3 && ndy == 1) return rms_bwd_vec<VPL, WPR, 3, 1, false, NW>;
    if (nx == 2 && ndy == 2) return rms_bwd_vec<VPL, WPR, 2, 2, false, NW>;
  } else {
    if (nx == 1 && ndy == 1) return rms_bwd_vec<VPL, WPR, 1, 1, true, NW>;
    if (nx == 1 && ndy == 2) return rms_bwd_vec<VPL, WPR, 1, 2, true, NW>;
    if (nx == 1 && ndy == 3) return rms_bwd_vec<VPL, WPR, 1, 3, true, NW>;
  }
  return nullptr;
}
template <int VPL, int WPR>
BwdKernel bwd_for_terms(int nx, int ndy, bool res, int nw) {
  return nw == 8 ? bwd_for_terms_nw<VPL, WPR, 8>(nx, ndy, res) : bwd_for_terms_nw<VPL, WPR, 4>(nx, ndy, res);
}
#define KP_SHAPE_SWITCH(FN, ...)                      \
  switch (vpl * 10 + wpr) {                           \
    case 11: return FN<1, 1>(__VA_ARGS__);            \
    case 21: return FN<2, 1>(__VA_ARGS__);            \
    case 31: return FN<3, 1>(__VA_ARGS__);            \
    case 41: return FN<4, 1>(__VA_ARGS__);            \
    case 51: return FN<5, 1>(__VA_ARGS__);            \
    case 12: return FN<1, 2>(__VA_ARGS__);            \
    case 22: return FN<2, 2>(__VA_ARGS__);            \
    case 32: return FN<3, 2>(__VA_ARGS__);            \
    case 42: return FN<4, 2>(__VA_ARGS__);            \
    case 52: return FN<5, 2>(__VA_ARGS__);            \
    case 14: return FN<1, 4>(__VA_ARGS__);            \
    case 24: return FN<2, 4>(__VA_ARGS__);            \
    case 34: return FN<3, 4>(__VA_ARGS__);            \
    case 44: return FN<4, 4>(__VA_ARGS__);            \
    case 61: return FN<6, 1>(__VA_ARGS__);            \
    case 81: return FN<8, 1>(__VA_ARGS__);            \
    case 82: return FN<8, 2>(__VA_ARGS__);            \
  }                                                   \
  return nullptr;
FwdKernel fwd_kernel(int vpl, int wpr, int nx) { KP_SHAPE_SWITCH(fwd_for_terms, nx) }
BwdKernel bwd_kernel(int vpl, int wpr, int nx, int ndy, bool res, int nw) {
  KP_SHAPE_SWITCH(bwd_for_terms, nx, ndy, res, nw)
}
#undef KP_SHAPE_SWITCH

bool rows_vec_ok(const void* const* p, const int64_t* s, int n) {
  for (int i = 0; i < n; ++i)
    if (!aligned16(p[i]) || (s[i] & 7) != 0) return false;
  return true;
}

// Term pointers may be NULL only when there are no rows (empty tensors).
int check_terms(const char* who, const char* name, const void* const* p, const int64_t* s, int n, int64_t M) {
  if (p == nullptr || s == nullptr || n < 1 || n > 3) return fail(KP_EINVAL, "%s: %s needs 1..3 terms", who, name);
  for (int i = 0; i < n; ++i) {
    if (p[i] == nullptr && M > 0) return fail(KP_EINVAL, "%s: %s term %d is NULL", who, name, i);
    if (s[i] < 0) return fail(KP_EINVAL, "%s: %s term %d has a negative row stride", who, name, i);
  }
  return KP_OK;
}

// Row blocks for the backward: a fixed number per CU so that the partial row
// count (and hence the summation order) depends only on device and shape.
int bwd_blocks(int64_t M, int rows_per_block_step, int bpc) {
  const int64_t groups = ceil_div(M, rows_per_block_step);
  const int64_t want = (int64_t)cu_count() * bpc;
  return (int)(groups < want ? (groups > 0 ? groups : 1) : want);
}

}  // namespace
}  // namespace kp

using namespace kp;

extern "C" {

int kp_rmsnorm_fwd_bf16(const void* const* x_terms, const int64_t* x_strides, int n_x, const void* weight,
                        int64_t w_seg_len, int64_t w_seg_stride, void* h_out, int64_t h_stride, void* y,
                        int64_t y_stride, float* rstd, int64_t M, int64_t N, float eps, void* stream) {
  static const char* who = "kp_rmsnorm_fwd_bf16";
  int st = check_terms(who, "x", x_terms, x_strides, n_x, M);
  if (st != KP_OK) return st;
  if (M < 0 || N <= 0) return fail(KP_EINVAL, "%s: need M >= 0 and N > 0 (M=%lld N=%lld)", who, (long long)M, (long long)N);
  if ((y == nullptr && M > 0) || y_stride < 0) return fail(KP_EINVAL, "%s: y is NULL or has a negative stride", who);
  if (weight != nullptr && (w_seg_len <= 0 || w_seg_stride < 0))
    return fail(KP_EINVAL, "%s: weight segment length must be > 0", who);
  if (M == 0) return KP_OK;

  RmsFwdArgs a{};
  for (int i = 0; i < n_x; ++i) {
    a.x[i] = static_cast<const uint16_t*>(x_terms[i]);
    a.xs[i] = x_strides[i];
  }
  a.n_x = n_x;
  a.w = static_cast<const uint16_t*>(weight);
  a.w_seg_len = weight ? w_seg_len : N;
  a.w_seg_stride = weight ? w_seg_stride : N;
  a.h = static_cast<uint16_t*>(h_out);
  a.hs = h_stride;
  a.y = static_cast<uint16_t*>(y);
  a.ys = y_stride;
  a.rstd = rstd;
  a.M = M;
  a.N = N;
  a.eps = eps;

  int vpl = 0, wpr = 0;
  bool vec = pick_vec(N, true, &vpl, &wpr) && rows_vec_ok(x_terms, x_strides, n_x) && aligned16(y) && (y_stride & 7) == 0;
  if (vec && h_out) vec = aligned16(h_out) && (h_stride & 7) == 0;
  if (vec && weight) vec = aligned16(weight) && (w_seg_len & 7) == 0 && (w_seg_stride & 7) == 0;
  const FwdKernel fk = vec ? fwd_kernel(vpl, wpr, n_x) : nullptr;
  vec = vec && fk != nullptr;
  hipStream_t s = as_stream(stream);
  if (vec) {
    const int rb = 4 / wpr;
    const int64_t groups = ceil_div(M, rb);
    const int64_t cap = (int64_t)cu_count() * fwd_bpc((int64_t)n_x * vpl * 1024);
    const int grid = (int)(groups < cap ? groups : cap);
    void* args[] = {&a};
    launch_dominant_raw(reinterpret_cast<const void*>(fk), dim3(grid), dim3(kThreads), args, 0, s);
  } else {
    const int64_t cap = (int64_t)cu_count() * 8;
    const int grid = (int)(M < cap ? M : cap);
    KP_LAUNCH_DOMINANT(rms_fwd_generic, dim3(grid), dim3(kThreads), 0, s, a);
  }
  return check_launch(who);
}

size_t kp_rmsnorm_bwd_workspace_size(int64_t M, int64_t N) {
  if (M <= 0 || N <= 0) return 16;
  // Partial rows: at most one per row block; the block count never exceeds 4 per
  // CU.  Rows are padded to whole 32-column chunks.
  const int64_t blocks = (int64_t)cu_count() * 4;
  const int64_t rows = M < blocks ? M : blocks;
  return (size_t)(rows * ceil_div(N, kPartChunk) * kPartChunk * (int64_t)sizeof(float));
}

int kp_rmsnorm_bwd_bf16(const void* const* dy_terms, const int64_t* dy_strides, int n_dy, const void* const* x_terms,
                        const int64_t* x_strides, int n_x, const float* rstd, const void* weight, int64_t w_seg_len,
                        int64_t w_seg_stride, const void* dx_residual, int64_t dxr_stride, void* dx,
                        int64_t dx_stride, float* dw_f32, void* dw_bf16, int dw_f32_round_bf16, int64_t M, int64_t N,
                        float eps, void* workspace, size_t workspace_bytes, void* stream) {
  static const char* who = "kp_rmsnorm_bwd_bf16";
  int st = check_terms(who, "dy", dy_terms, dy_strides, n_dy, M);
  if (st != KP_OK) return st;
  st = check_terms(who, "x", x_terms, x_strides, n_x, M);
  if (st != KP_OK) return st;
  if (M < 0 || N <= 0) return fail(KP_EINVAL, "%s: need M >= 0 and N > 0 (M=%lld N=%lld)", who, (long long)M, (long long)N);
  if ((dx == nullptr && M > 0) || dx_stride < 0) return fail(KP_EINVAL, "%s: dx is NULL or has a negative stride", who);
  if (dx_residual != nullptr && dxr_stride < 0) return fail(KP_EINVAL, "%s: negative dx_residual stride", who);
  const bool want_dw = dw_f32 != nullptr || dw_bf16 != nullptr;
  if (want_dw && weight == nullptr) return fail(KP_EINVAL, "%s: a weight gradient needs a weight", who);
  if (weight != nullptr && (w_seg_len <= 0 || w_seg_stride < 0))
    return fail(KP_EINVAL, "%s: weight segment length must be > 0", who);
  const size_t need = kp_rmsnorm_bwd_workspace_size(M, N);
  if (want_dw && M > 0 && (workspace == nullptr || workspace_bytes < need || !aligned16(workspace)))
    return fail(KP_EWORKSPACE, "%s: workspace needs %zu bytes, 16-byte aligned (got %zu)", who, need, workspace_bytes);

  hipStream_t s = as_stream(stream);
  RmsBwdArgs a{};
  for (int i = 0; i < n_dy; ++i) {
    a.dy[i] = static_cast<const uint16_t*>(dy_terms[i]);
    a.dys[i] = dy_strides[i];
  }
  a.n_dy = n_dy;
  for (int i = 0; i < n_x; ++i) {
    a.x[i] = static_cast<const uint16_t*>(x_terms[i]);
    a.xs[i] = x_strides[i];
  }
  a.n_x = n_x;
  a.rstd = rstd;
  a.w = static_cast<const uint16_t*>(weight);
  a.w_seg_len = weight ? w_seg_len : N;
  a.w_seg_stride = weight ? w_seg_stride : N;
  a.dxr = static_cast<const uint16_t*>(dx_residual);
  a.dxrs = dxr_stride;
  a.dx = static_cast<uint16_t*>(dx);
  a.dxs = dx_stride;
  a.partial = want_dw ? static_cast<float*>(workspace) : nullptr;
  a.M = M;
  a.N = N;
  a.eps = eps;

  int blocks = 0;
  if (M > 0) {
    int vpl = 0, wpr = 0;
    bool vec = pick_vec(N, false, &vpl, &wpr) && rows_vec_ok(x_terms, x_strides, n_x) &&
               rows_vec_ok(dy_terms, dy_strides, n_dy) && aligned16(dx) && (dx_stride & 7) == 0;
    if (vec && dx_residual) vec = aligned16(dx_residual) && (dxr_stride & 7) == 0;
    if (vec && weight) vec = aligned16(weight) && (w_seg_len & 7) == 0 && (w_seg_stride & 7) == 0;
    int nw = bwd_waves();
    // 8-wave blocks need (8 / wpr / 2) * wpr * SEG floats of combine LDS; stay within 48 KiB.
    if (vec && nw == 8 && (size_t)(8 / wpr / 2) * wpr * 512 * vpl * sizeof(float) > 48 * 1024) nw = 4;
    const BwdKernel bk = vec ? bwd_kernel(vpl, wpr, n_x, n_dy, dx_residual != nullptr, nw) : nullptr;
    vec = vec && bk != nullptr;
    if (vec) {
      const int rb = nw / wpr;
      blocks = bwd_blocks(M, rb, bwd_bpc((int64_t)(n_x + n_dy + (dx_residual ? 1 : 0)) * vpl * 1024));
      const size_t lds = (want_dw && rb >= 2) ? (size_t)(rb / 2) * wpr * 512 * vpl * sizeof(float) : 0;
      void* args[] = {&a};
      launch_dominant_raw(reinterpret_cast<const void*>(bk), dim3(blocks), dim3(nw * 64), args, lds, s);
    } else {
      blocks = bwd_blocks(M, 1, 2);  // generic kernel: one row per block step, 2 blocks per CU
      KP_LAUNCH_DOMINANT(rms_bwd_generic, dim3(blocks), dim3(kThreads), 0, s, a);
    }
    st = check_launch(who);
    if (st != KP_OK) return st;
  }
  if (want_dw) {
    hipLaunchKernelGGL(rms_dw_finalize, dim3((unsigned)ceil_div(N, kPartChunk)), dim3(kThreads), 0, s,
                       static_cast<const float*>(workspace), blocks, N, dw_f32, static_cast<uint16_t*>(dw_bf16),
                       dw_f32_round_bf16);
    st = check_launch(who);
  }
  return st;
}

}  // extern "C"
