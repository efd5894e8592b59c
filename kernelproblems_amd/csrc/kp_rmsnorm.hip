// RMSNorm forward / backward for gfx950: dispatch, the generic (any shape,
// any alignment) kernels, the weight-gradient finalize and the C ABI.  The
// vectorized row kernels are in kp_rmsnorm_kernels.hpp.
#include <stdlib.h>

#include <mutex>

#include "kp_internal.hpp"
#include "kp_rmsnorm_kernels.hpp"

namespace kp {
namespace {

using namespace rms;

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

// dw[c] = sum_{p < P} partial[p, c].  A block owns one 16-column chunk, whose
// P partial rows are contiguous ([P][16] fp32).  Thread (r, q) sums columns
// 4q..4q+3 over rows r, r + 64, r + 128, ... in row order (loads in batches
// of 4 rows: P = 256 is one batch); the 64 row-group sums of a column are
// then added as 16 sums of 4 consecutive groups, and those 16 in order.  The
// order is fixed, so the result is bitwise reproducible.
constexpr int kFinGroups = kThreads / (kPartChunk / 4);  // 64
constexpr int kFinPairs = kThreads / kPartChunk;         // 16

__global__ __launch_bounds__(kThreads) void rms_dw_finalize(const float* __restrict__ partial, int P, int64_t N,
                                                            float* dw_f32, uint16_t* dw_bf16, int round_f32) {
  __shared__ float s[kFinGroups][kPartChunk + 1];
  __shared__ float s2[kFinPairs][kPartChunk + 1];
  const int q = threadIdx.x & 3, r = threadIdx.x >> 2;
  const int64_t c0 = (int64_t)blockIdx.x * kPartChunk;
  const float* base = partial + (int64_t)blockIdx.x * P * kPartChunk;
  const int ncol = (int)(N - c0 < kPartChunk ? N - c0 : kPartChunk);
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  if (ncol == kPartChunk) {
    int p = r;
    for (; p + 3 * kFinGroups < P; p += 4 * kFinGroups) {
      f32x4 v[4];
#pragma unroll
      for (int k = 0; k < 4; ++k)
        v[k] = *reinterpret_cast<const f32x4*>(base + (int64_t)(p + k * kFinGroups) * kPartChunk + q * 4);
#pragma unroll
      for (int k = 0; k < 4; ++k) acc += v[k];
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
  {
    const int c = threadIdx.x & (kPartChunk - 1), g = threadIdx.x / kPartChunk;  // g < 16
    s2[g][c] = ((s[4 * g][c] + s[4 * g + 1][c]) + s[4 * g + 2][c]) + s[4 * g + 3][c];
  }
  __syncthreads();
  if (threadIdx.x < ncol) {
    float t = s2[0][threadIdx.x];
#pragma unroll
    for (int g = 1; g < kFinPairs; ++g) t += s2[g][threadIdx.x];
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
// At most 4 blocks per CU: the workspace holds one partial row per block.
int bwd_bpc(int waves_per_block, int64_t wave_slot_bytes) {
  static const int v = env_int("KP_RMS_BWD_BPC", 0, 0, 4);
  return v ? v : auto_bpc(waves_per_block, wave_slot_bytes, 64 * 1024, 4);
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

// Forward row shape for M rows: pick_vec's, except that rows of 4096 go to one
// block of 4 waves each (the one-shot grid of one row per block) from
// KP_RMS_FWD_BLOCK_ROWS (default 8192) rows on.  Measured on MI355X per call
// (one wave per row -> one block per row): M = 4096 12.1 -> 13.5 us (c1),
// 6144 18.9 both, 8192 25.0 -> 23.9, 12288 35.7 -> 34.0, 16384 46.3 -> 44.4,
// 32768 90.9 -> 86.3.  0 turns the rule off (tuning knob).
bool pick_fwd(int64_t M, int64_t N, int* vpl, int* wpr) {
  if (!pick_vec(N, true, vpl, wpr)) return false;
  static const int64_t from = env_int("KP_RMS_FWD_BLOCK_ROWS", 8192, 0, 1 << 30);
  static const bool knobs = getenv("KP_RMS_VPL_MAX") != nullptr || getenv("KP_RMS_WPR_MIN") != nullptr;
  if (!knobs && from > 0 && M >= from && N == 4096 && shape_ok(2, 4)) {
    *vpl = 2;
    *wpr = 4;
  }
  return true;
}

// Backward row shape: N = 8192 runs 8 waves per row with 2 chunks per lane in
// 8-wave blocks (one row per block step; measured on MI355X at [16384, 8192]
// with two x terms: 171.5 us against 175.5 us for 4 waves x 4 chunks in
// 4-wave blocks, whose grid-wide row pass is otherwise the same).  Every other
// width takes pick_vec's shape in 4-wave blocks.  *nw = waves per block.
bool pick_bwd(int64_t N, int* vpl, int* wpr, int* nw) {
  static const bool knobs = getenv("KP_RMS_VPL_MAX") != nullptr || getenv("KP_RMS_WPR_MIN") != nullptr;
  if (N == 8192 && !knobs) {
    *vpl = 2;
    *wpr = 8;
    *nw = 8;
    return true;
  }
  *nw = kThreads / 64;
  return pick_vec(N, false, vpl, wpr);
}

// Backward kernel for a fast-path shape, from its instantiation unit (fwd:
// the fused forward + backward variant).
BwdKernel bwd_kernel(int vpl, int wpr, int nx, int ndy, bool res, bool fwd) {
  switch (vpl) {
    case 1: return bwd_kernel_vpl1(wpr, nx, ndy, res, fwd);
    case 2: return bwd_kernel_vpl2(wpr, nx, ndy, res, fwd);
    case 3: return bwd_kernel_vpl3(wpr, nx, ndy, res, fwd);
    case 4: return bwd_kernel_vpl4(wpr, nx, ndy, res, fwd);
    case 5: return bwd_kernel_vpl5(wpr, nx, ndy, res, fwd);
    case 6:
    case 8: return bwd_kernel_vpl68(vpl, wpr, nx, ndy, res, fwd);
  }
  return nullptr;
}

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


// Forward outputs of the fused forward + backward (kp_rmsnorm_fwd_bwd_bf16).
struct FwdOut {
  uint16_t* y;
  int64_t ys;
  uint16_t* h;
  int64_t hs;
  float* rstd;
};

size_t bwd_workspace_size(int64_t M, int64_t N) {
  if (M <= 0 || N <= 0) return 16;
  // Partial rows: at most one per row block; the block count never exceeds 4 per
  // CU.  Rows are padded to whole 16-column chunks (kPartChunk).
  const int64_t blocks = (int64_t)cu_count() * 4;
  const int64_t rows = M < blocks ? M : blocks;
  return (size_t)(rows * ceil_div(N, kPartChunk) * kPartChunk * (int64_t)sizeof(float));
}
// The fused forward + backward also keeps room for an fp32 rstd per row after
// the partial rows (used only by its two-launch fallback).
size_t fwd_bwd_workspace_size(int64_t M, int64_t N) {
  if (M <= 0 || N <= 0) return 16;
  return ((bwd_workspace_size(M, N) + 255) & ~(size_t)255) + (size_t)M * sizeof(float);
}

// Launch plan of a backward row pass: the kernel and its block count (each
// block writes one weight-gradient partial row).
struct BwdPlan {
  BwdKernel vec;   // vectorized kernel, or nullptr for rms_bwd_generic
  int wpr;         // waves per row of the vectorized kernel
  int threads;     // threads per block
  int blocks;      // row blocks = partial rows
  size_t lds;      // dynamic LDS of the vectorized kernel
};

BwdPlan plan_bwd(const void* const* dy_terms, const int64_t* dy_strides, int n_dy, const void* const* x_terms,
                 const int64_t* x_strides, int n_x, const void* weight, int64_t w_seg_len, int64_t w_seg_stride,
                 const void* dx_residual, int64_t dxr_stride, const void* dx, int64_t dx_stride, bool want_dw,
                 const FwdOut* fo, int64_t M, int64_t N) {
  BwdPlan p{nullptr, 1, kThreads, 0, 0};
  if (M <= 0) return p;
  int vpl = 0, wpr = 0, nw = kThreads / 64;
  bool vec = pick_bwd(N, &vpl, &wpr, &nw) && rows_vec_ok(x_terms, x_strides, n_x) &&
             rows_vec_ok(dy_terms, dy_strides, n_dy) && aligned16(dx) && (dx_stride & 7) == 0;
  if (vec && dx_residual) vec = aligned16(dx_residual) && (dxr_stride & 7) == 0;
  if (vec && weight) vec = aligned16(weight) && (w_seg_len & 7) == 0 && (w_seg_stride & 7) == 0;
  if (vec && fo)
    vec = aligned16(fo->y) && (fo->ys & 7) == 0 && (fo->h == nullptr || (aligned16(fo->h) && (fo->hs & 7) == 0));
  p.vec = vec ? bwd_kernel(vpl, wpr, n_x, n_dy, dx_residual != nullptr, fo != nullptr) : nullptr;
  if (p.vec != nullptr) {
    const int rb = nw / wpr;
    p.wpr = wpr;
    p.threads = nw * 64;
    p.blocks = bwd_blocks(M, rb, bwd_bpc(nw, (int64_t)(n_x + n_dy + (dx_residual ? 1 : 0)) * vpl * 1024));
    p.lds = (want_dw && rb >= 2) ? (size_t)(rb / 2) * wpr * 512 * vpl * sizeof(float) : 0;
  } else {
    p.blocks = bwd_blocks(M, 1, 2);  // generic kernel: one row per block step, 2 blocks per CU
  }
  return p;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Bytes of the partial rows a plan writes.
size_t partial_bytes(const BwdPlan& p, int64_t N) {
  return (size_t)p.blocks * (size_t)(ceil_div(N, kPartChunk) * kPartChunk) * sizeof(float);
}

// The RMSNorm backward (fo == nullptr) and the fused forward + backward
// (fo != nullptr: rstd is recomputed and y / h / rstd are written by the same
// row pass).  Shapes or term combinations without a fused kernel run the
// forward kernel and then the backward with the rstd it wrote (workspace
// bytes past the partial rows hold it when the caller wants no rstd).  The
// workspace must hold the partial rows the launch plan writes (the *_size
// functions return an upper bound of that).
int rms_bwd_impl(const char* who, const void* const* dy_terms, const int64_t* dy_strides, int n_dy,
                 const void* const* x_terms, const int64_t* x_strides, int n_x, const float* rstd, const void* weight,
                 int64_t w_seg_len, int64_t w_seg_stride, const void* dx_residual, int64_t dxr_stride, void* dx,
                 int64_t dx_stride, float* dw_f32, void* dw_bf16, int dw_f32_round_bf16, int64_t M, int64_t N,
                 float eps, void* workspace, size_t workspace_bytes, const FwdOut* fo, void* stream) {
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

  // The pass: the fused kernel when there is one, else (fo only) the forward
  // kernel followed by the plain backward.
  BwdPlan plan = plan_bwd(dy_terms, dy_strides, n_dy, x_terms, x_strides, n_x, weight, w_seg_len, w_seg_stride,
                          dx_residual, dxr_stride, dx, dx_stride, want_dw, fo, M, N);
  const bool two_launch = fo != nullptr && M > 0 && plan.vec == nullptr;
  if (two_launch)
    plan = plan_bwd(dy_terms, dy_strides, n_dy, x_terms, x_strides, n_x, weight, w_seg_len, w_seg_stride,
                    dx_residual, dxr_stride, dx, dx_stride, want_dw, nullptr, M, N);
  const size_t part = want_dw ? partial_bytes(plan, N) : 0;
  const bool rstd_in_ws = two_launch && fo->rstd == nullptr;
  const size_t need = rstd_in_ws ? align256(part) + (size_t)M * sizeof(float) : part;
  if (need > 0 && (workspace == nullptr || workspace_bytes < need || !aligned16(workspace)))
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
  a.trace = block_trace_buf();
  a.trace_blocks = a.trace ? block_trace_blocks() : 0;
  a.M = M;
  a.N = N;
  a.eps = eps;

  if (M > 0) {
    if (two_launch) {
      float* r = rstd_in_ws ? reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + align256(part)) : fo->rstd;
      st = kp_rmsnorm_fwd_bf16(x_terms, x_strides, n_x, weight, w_seg_len, w_seg_stride, n_x > 1 ? fo->h : nullptr,
                               fo->hs, fo->y, fo->ys, r, M, N, eps, stream);
      if (st != KP_OK) return st;
      a.rstd = r;
    } else if (fo != nullptr) {
      a.y = fo->y;
      a.ys = fo->ys;
      a.h = n_x > 1 ? fo->h : nullptr;
      a.hs = fo->hs;
      a.rstd_out = fo->rstd;
      a.rstd = nullptr;
    }
    if (plan.vec != nullptr) {
      void* args[] = {&a};
      launch_dominant_raw(reinterpret_cast<const void*>(plan.vec), dim3(plan.blocks), dim3(plan.threads), args,
                          plan.lds, s);
    } else {
      KP_LAUNCH_DOMINANT(rms_bwd_generic, dim3(plan.blocks), dim3(kThreads), 0, s, a);
    }
    st = check_launch(who);
    if (st != KP_OK) return st;
  }
  if (want_dw) {
    hipLaunchKernelGGL(rms_dw_finalize, dim3((unsigned)ceil_div(N, kPartChunk)), dim3(kThreads), 0, s,
                       static_cast<const float*>(workspace), plan.blocks, N, dw_f32, static_cast<uint16_t*>(dw_bf16),
                       dw_f32_round_bf16);
    st = check_launch(who);
  }
  return st;
}

// ------------------------------------------------------------ allocation-free
// kp_rmsnorm_bwd_bf16_noalloc keeps the weight-gradient partial rows in a
// fixed device array instead of a caller workspace: one copy per GPU, held
// until the process ends, shared by every call on that GPU.  Nothing in it
// needs clearing: each call's row blocks write their whole partial rows
// before the finalize reads them.  The array's name is a host-side stand-in
// in host code, never a device address: the per-device set-up looks the
// address up once (that device current) with hipGetSymbolAddress, and
// launches take that pointer.
//
// Overlap guard: the set-up also creates one event per device, recorded on
// the calling stream after each call's launches.  A call on a different
// stream from the previous call on that GPU first asks whether that event
// has completed; while it has not, the call returns KP_EBUSY and launches
// nothing (two unordered calls would race on the array).  Calls on one
// stream are ordered by the stream and pass straight through.  A stream
// under graph capture is not guarded (an event query there would end the
// capture): a captured call records nothing and checks nothing.
constexpr size_t kScratchBytes = (size_t)8 << 20;  // 256 row blocks x 8192 fp32 columns
__device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxScratchDevices = 64;
struct ScratchState {
  void* ptr = nullptr;         // device address of this GPU's copy of `scratch`
  hipEvent_t done = nullptr;   // recorded after the previous uncaptured call's launches
  hipStream_t last = nullptr;  // that call's stream
  bool used = false;
};
std::mutex g_scratch_mu;  // guards g_scratch and serialises guarded calls (check, launch, record)
ScratchState g_scratch[kMaxScratchDevices];

// Per-device set-up (first call on the device, that device current).
// Caller holds g_scratch_mu.
int scratch_state(const char* who, ScratchState** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDevices)
    return fail(KP_EHIP, "%s: no current HIP device (or device %d beyond %d)", who, dev, kMaxScratchDevices);
  ScratchState& st = g_scratch[dev];
  if (st.ptr == nullptr) {
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(KP_EHIP, "%s: hipGetSymbolAddress(scratch) on device %d: %s", who, dev, hipGetErrorString(e));
    hipEvent_t ev = nullptr;
    e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e != hipSuccess) return fail(KP_EHIP, "%s: hipEventCreateWithFlags on device %d: %s", who, dev, hipGetErrorString(e));
    st.ptr = p;
    st.done = ev;
  }
  *out = &st;
  return KP_OK;
}
}  // namespace

int rms_dw_finalize_launch(const float* partial, int P, int64_t N, float* dw_f32, uint16_t* dw_bf16, int round_f32,
                           hipStream_t s, const char* who) {
  hipLaunchKernelGGL(rms_dw_finalize, dim3((unsigned)ceil_div(N, kPartChunk)), dim3(kThreads), 0, s, partial, P, N,
                     dw_f32, dw_bf16, round_f32);
  return check_launch(who);
}

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
  bool vec = pick_fwd(M, N, &vpl, &wpr) && rows_vec_ok(x_terms, x_strides, n_x) && aligned16(y) && (y_stride & 7) == 0;
  if (vec && h_out) vec = aligned16(h_out) && (h_stride & 7) == 0;
  if (vec && weight) vec = aligned16(weight) && (w_seg_len & 7) == 0 && (w_seg_stride & 7) == 0;
  const FwdKernel fk = vec ? fwd_kernel(vpl, wpr, n_x) : nullptr;
  vec = vec && fk != nullptr;
  hipStream_t s = as_stream(stream);
  if (vec) {
    const int rb = 4 / wpr;
    const int64_t groups = ceil_div(M, rb);
    // Rows of 4 waves (one row per block): one block per row, no persistent
    // walk -- measured on MI355X at [16384, 8192] with two x terms: 170.5 us
    // against 185 us for 2 pipelined blocks per CU.  Shorter rows (1 or 2
    // waves) keep the pipelined grid ([4096, 4096]: 12.5 us against 13.8 us
    // for one block per 4 rows).
    const int64_t cap = wpr == 4 ? groups : (int64_t)cu_count() * fwd_bpc((int64_t)n_x * vpl * 1024);
    if (groups > INT32_MAX) return fail(KP_EUNSUPPORTED, "%s: too many rows for one launch", who);
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

int kp_embedding_rmsnorm_fwd_bf16(const void* table, int64_t V, int64_t table_row_stride, const void* indices,
                                  int index_bytes, int64_t T, const void* weight, int64_t w_seg_len,
                                  int64_t w_seg_stride, void* h_out, int64_t h_stride, void* y, int64_t y_stride,
                                  float* rstd, int64_t N, float eps, int32_t* error_flag, void* stream) {
  static const char* who = "kp_embedding_rmsnorm_fwd_bf16";
  if (T < 0 || N <= 0 || V <= 0) return fail(KP_EINVAL, "%s: need T >= 0, N > 0, V > 0", who);
  if (index_bytes != 4 && index_bytes != 8) return fail(KP_EINVAL, "%s: index_bytes must be 4 or 8", who);
  if (T > 0 && (table == nullptr || indices == nullptr || y == nullptr))
    return fail(KP_EINVAL, "%s: table, indices and y are required", who);
  if (table_row_stride < N || y_stride < 0 || (h_out != nullptr && h_stride < 0))
    return fail(KP_EINVAL, "%s: bad row stride", who);
  if (weight != nullptr && (w_seg_len <= 0 || w_seg_stride < 0))
    return fail(KP_EINVAL, "%s: weight segment length must be > 0", who);
  if (T == 0) return KP_OK;

  RmsFwdArgs a{};
  a.x[0] = static_cast<const uint16_t*>(table);
  a.xs[0] = table_row_stride;
  a.n_x = 1;
  a.idx = indices;
  a.idx_bytes = index_bytes;
  a.idx_rows = V;
  a.err = error_flag;
  a.w = static_cast<const uint16_t*>(weight);
  a.w_seg_len = weight ? w_seg_len : N;
  a.w_seg_stride = weight ? w_seg_stride : N;
  a.h = static_cast<uint16_t*>(h_out);
  a.hs = h_stride;
  a.y = static_cast<uint16_t*>(y);
  a.ys = y_stride;
  a.rstd = rstd;
  a.M = T;
  a.N = N;
  a.eps = eps;

  int vpl = 0, wpr = 0;
  // one wave per row whatever T: the gather's row-per-block form measured
  // 39.3 against 34.2 us at C3 (cache-served table rows favour the
  // persistent pipelined grid)
  bool vec = pick_vec(N, true, &vpl, &wpr) && aligned16(table) && (table_row_stride & 7) == 0 && aligned16(y) &&
             (y_stride & 7) == 0;
  if (vec && h_out) vec = aligned16(h_out) && (h_stride & 7) == 0;
  if (vec && weight) vec = aligned16(weight) && (w_seg_len & 7) == 0 && (w_seg_stride & 7) == 0;
  const FwdKernel fk = vec ? fwd_gather_kernel(vpl, wpr) : nullptr;
  if (fk == nullptr)
    return fail(KP_EUNSUPPORTED, "%s: row shape / alignment without a fused kernel (N=%lld)", who, (long long)N);
  const int rb = 4 / wpr;
  const int64_t groups = ceil_div(T, rb);
  // one block per row for rows of 4 waves, as in kp_rmsnorm_fwd_bf16
  const int64_t cap = wpr == 4 ? groups : (int64_t)cu_count() * fwd_bpc((int64_t)vpl * 1024);
  if (groups > INT32_MAX) return fail(KP_EUNSUPPORTED, "%s: too many rows for one launch", who);
  const int grid = (int)(groups < cap ? groups : cap);
  void* args[] = {&a};
  launch_dominant_raw(reinterpret_cast<const void*>(fk), dim3(grid), dim3(kThreads), args, 0, as_stream(stream));
  return check_launch(who);
}

size_t kp_rmsnorm_bwd_workspace_size(int64_t M, int64_t N) { return bwd_workspace_size(M, N); }

size_t kp_rmsnorm_fwd_bwd_workspace_size(int64_t M, int64_t N) { return fwd_bwd_workspace_size(M, N); }

int kp_rmsnorm_bwd_bf16(const void* const* dy_terms, const int64_t* dy_strides, int n_dy, const void* const* x_terms,
                        const int64_t* x_strides, int n_x, const float* rstd, const void* weight, int64_t w_seg_len,
                        int64_t w_seg_stride, const void* dx_residual, int64_t dxr_stride, void* dx,
                        int64_t dx_stride, float* dw_f32, void* dw_bf16, int dw_f32_round_bf16, int64_t M, int64_t N,
                        float eps, void* workspace, size_t workspace_bytes, void* stream) {
  return rms_bwd_impl("kp_rmsnorm_bwd_bf16", dy_terms, dy_strides, n_dy, x_terms, x_strides, n_x, rstd, weight,
                      w_seg_len, w_seg_stride, dx_residual, dxr_stride, dx, dx_stride, dw_f32, dw_bf16,
                      dw_f32_round_bf16, M, N, eps, workspace, workspace_bytes, nullptr, stream);
}

size_t kp_rmsnorm_bwd_noalloc_max_bytes(void) { return kScratchBytes; }

int kp_rmsnorm_bwd_bf16_noalloc(const void* const* dy_terms, const int64_t* dy_strides, int n_dy,
                                const void* const* x_terms, const int64_t* x_strides, int n_x, const float* rstd,
                                const void* weight, int64_t w_seg_len, int64_t w_seg_stride, const void* dx_residual,
                                int64_t dxr_stride, void* dx, int64_t dx_stride, float* dw_f32, void* dw_bf16,
                                int dw_f32_round_bf16, int64_t M, int64_t N, float eps, void* stream) {
  static const char* who = "kp_rmsnorm_bwd_bf16_noalloc";
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  ScratchState* ss = nullptr;
  int st = scratch_state(who, &ss);
  if (st != KP_OK) return st;
  hipStream_t s = as_stream(stream);
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(s, &cap);
  if (e != hipSuccess) return fail(KP_EHIP, "%s: hipStreamIsCapturing: %s", who, hipGetErrorString(e));
  const bool guarded = cap == hipStreamCaptureStatusNone;
  if (guarded && ss->used && s != ss->last) {
    e = hipEventQuery(ss->done);
    if (e == hipErrorNotReady)
      return fail(KP_EBUSY,
                  "%s: the previous call on this GPU (another stream) has not finished; calls on different "
                  "streams share the static scratch and must be ordered by the caller",
                  who);
    if (e != hipSuccess) return fail(KP_EHIP, "%s: hipEventQuery: %s", who, hipGetErrorString(e));
  }
  st = rms_bwd_impl(who, dy_terms, dy_strides, n_dy, x_terms, x_strides, n_x, rstd, weight, w_seg_len, w_seg_stride,
                    dx_residual, dxr_stride, dx, dx_stride, dw_f32, dw_bf16, dw_f32_round_bf16, M, N, eps, ss->ptr,
                    kScratchBytes, nullptr, stream);
  if (st == KP_EWORKSPACE)  // rejected before any launch
    return fail(KP_EUNSUPPORTED,
                "%s: M=%lld, N=%lld needs more weight-gradient partial rows than its %zu bytes of static scratch "
                "hold (one fp32 row of N per row block); use kp_rmsnorm_bwd_bf16 with a workspace",
                who, (long long)M, (long long)N, kScratchBytes);
  if (st != KP_OK || !guarded) return st;
  e = hipEventRecord(ss->done, s);
  if (e != hipSuccess) return fail(KP_EHIP, "%s: hipEventRecord: %s", who, hipGetErrorString(e));
  ss->last = s;
  ss->used = true;
  return KP_OK;
}

int kp_rmsnorm_fwd_bwd_bf16(const void* const* dy_terms, const int64_t* dy_strides, int n_dy,
                            const void* const* x_terms, const int64_t* x_strides, int n_x, const void* weight,
                            int64_t w_seg_len, int64_t w_seg_stride, void* h_out, int64_t h_stride, void* y,
                            int64_t y_stride, float* rstd_out, const void* dx_residual, int64_t dxr_stride, void* dx,
                            int64_t dx_stride, float* dw_f32, void* dw_bf16, int dw_f32_round_bf16, int64_t M,
                            int64_t N, float eps, void* workspace, size_t workspace_bytes, void* stream) {
  static const char* who = "kp_rmsnorm_fwd_bwd_bf16";
  if ((y == nullptr && M > 0) || y_stride < 0 || (h_out != nullptr && h_stride < 0))
    return fail(KP_EINVAL, "%s: y is NULL or a forward output has a negative stride", who);
  FwdOut fo{static_cast<uint16_t*>(y), y_stride, static_cast<uint16_t*>(h_out), h_stride, rstd_out};
  return rms_bwd_impl(who, dy_terms, dy_strides, n_dy, x_terms, x_strides, n_x, nullptr, weight, w_seg_len,
                      w_seg_stride, dx_residual, dxr_stride, dx, dx_stride, dw_f32, dw_bf16, dw_f32_round_bf16, M, N,
                      eps, workspace, workspace_bytes, &fo, stream);
}

}  // extern "C"
