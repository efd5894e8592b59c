// Cross-entropy loss over a vocabulary for gfx950: the _log_softmax +
// nll_loss region at the end of a Llama step, forward and backward.
//
// Forward (sum reduction, ignore_index):
//   lse_i  = max_j x_ij + log(sum_j exp(x_ij - max_j x_ij))     x = fp32(bf16 logits)
//   loss   = scale * sum_{i: t_i != ignore} (lse_i - x_{i, t_i}),  total_weight = #{i: t_i != ignore}
// The log-softmax matrix itself is never materialised: each logits row is
// read once (HBM read-bound) with a running reference exponent and a sum of
// exponentials per lane, one wave per row.  Per-row losses land in a workspace and a
// second one-block launch sums them in a fixed order in fp64 (deterministic,
// no atomics).
//
// Backward, given the saved fp32 log-softmax L and the upstream gradient g of
// the summed loss:
//   out_ij = bf16( grad_ij - exp(L_ij) * s_i ),   grad_ij = (j == t_i) ? -g : 0,  s_i = sum_j grad_ij
// (nll_loss_backward then _log_softmax_backward_data, fp32, then _to_copy):
// a streaming kernel, 4 bytes read and 2 written per element, evaluated in
// the same fp32 operations as torch's kernels (expf, this order).
//
// Forward and backward straight from the bf16 logits (the whole region when
// the log-softmax is not needed elsewhere): one block per row holds the row
// in registers, so each logit is read once and each gradient written once.
#include <math.h>

#include "kp_common.hpp"
#include "kp_internal.hpp"

namespace kp {
namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kThreads = 256;
constexpr int kWavesPerBlock = kThreads / kWave;

__device__ __forceinline__ int64_t target_at(const void* t, int bytes, int64_t i) {
  return bytes == 8 ? static_cast<const int64_t*>(t)[i] : (int64_t) static_cast<const int32_t*>(t)[i];
}

// ------------------------------------------------------------------ forward
struct FwdArgs {
  const uint16_t* logits;
  int64_t rs;  // row stride, elements
  int64_t M, V;
  const void* targets;
  int tbytes;
  int64_t ignore;
  double* row_loss;   // [M]: lse_i - x_{i,t_i}, 0 for ignored rows
  int32_t* row_valid;  // [M]: 1 when the row counts
  float* lse_out;     // optional [M]
  int32_t* err;       // optional flag: a target outside [0, V) and not ignore_index
};

// A lane's running state is (R, s): R an fp32 reference exponent in log2
// units (the running max times L, L = log2 e rounded to fp32, rounded to
// fp32) and s = sum_j 2^(x_j L - R), each exponent argument formed by one
// fma, so it is rounded once relative to its own size.  The row's
// log2(sum_j 2^(x_j L)) is R + log2(s), and lse = (R + log2 s) / L in fp64:
// dividing by the same L the exponents used makes the dominant term exact,
// so neither R's rounding (~2e-3 in log2 units at |max| ~ 3e4) nor L's
// (L = log2 e (1 - 1.3e-8)) scales with the logits' magnitude; what remains
// is ~1.3e-8 log(V) plus the fp32 sums.

// (R, s) folded with 8 more values.
__device__ __forceinline__ void online8(float& R, float& s, const float* v) {
  const float cm = fmaxf(fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3])), fmaxf(fmaxf(v[4], v[5]), fmaxf(v[6], v[7])));
  const float rn = fmaxf(R, cm * kLog2e);  // rounding to fp32 is monotone: max commutes with it
  if (rn == -INFINITY) return;             // nothing but -inf so far: (R, s) stays (-inf, 0)
  s *= (R == rn) ? 1.0f : __builtin_amdgcn_exp2f(R - rn);
  float c = 0.0f, d = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; i += 2) {
    c += __builtin_amdgcn_exp2f(__builtin_fmaf(v[i], kLog2e, -rn));
    d += __builtin_amdgcn_exp2f(__builtin_fmaf(v[i + 1], kLog2e, -rn));
  }
  s += c + d;
  R = rn;
}

// (R1, s1) + (R2, s2) of two lanes' states.
__device__ __forceinline__ void combine(float& R, float& s, float R2, float s2) {
  const float rn = fmaxf(R, R2);
  if (rn == -INFINITY) return;
  const float a = (R == rn) ? s : s * __builtin_amdgcn_exp2f(R - rn);
  const float b = (R2 == rn) ? s2 : s2 * __builtin_amdgcn_exp2f(R2 - rn);
  R = rn;
  s = a + b;
}

template <int CTRL>
__device__ __forceinline__ void combine_dpp(float& R, float& s) {
  combine(R, s, dpp_f<CTRL>(R), dpp_f<CTRL>(s));
}

// The row's target and the raw bf16 logit at it, requested by the row's wave
// before its data loads: the target is then a scalar load ahead of any store,
// and the logit's wait, at the end of the row, does not sit behind the row's
// stores (loaded after them, the two formed a chain of full waits on the
// kernel's last wave generation).  An id outside [0, V) reads column 0.
struct FwdTarget {
  int64_t t;
  uint16_t xt;
};
__device__ __forceinline__ FwdTarget row_target(const FwdArgs& a, int64_t row) {
  const int64_t t = target_at(a.targets, a.tbytes, row);
  const bool in = t >= 0 && t < a.V;
  return FwdTarget{t, a.logits[row * a.rs + (in ? t : 0)]};
}

// Row-wave epilogue: reduce the lanes' states, then lane 0 writes the row's loss.
__device__ __forceinline__ void finish_row(const FwdArgs& a, int64_t row, FwdTarget rt, float R, float s) {
  combine_dpp<0xB1>(R, s);   // quad_perm [1,0,3,2]
  combine_dpp<0x4E>(R, s);   // quad_perm [2,3,0,1]
  combine_dpp<0x141>(R, s);  // row_half_mirror
  combine_dpp<0x140>(R, s);  // row_mirror
  float r0 = readlane_f(R, 0), s0 = readlane_f(s, 0);
  combine(r0, s0, readlane_f(R, 16), readlane_f(s, 16));
  float r1 = readlane_f(R, 32), s1 = readlane_f(s, 32);
  combine(r1, s1, readlane_f(R, 48), readlane_f(s, 48));
  combine(r0, s0, r1, s1);
  if ((threadIdx.x & (kWave - 1)) != 0) return;
  const double lse = ((double)r0 + log2((double)s0)) / (double)kLog2e;
  if (a.lse_out) a.lse_out[row] = (float)lse;
  const int64_t t = rt.t;
  int valid = t != a.ignore;
  if (valid && (t < 0 || t >= a.V)) {
    valid = 0;
    if (a.err) a.err[0] = 1;
  }
  a.row_loss[row] = valid ? lse - (double)bf_to_f(rt.xt) : 0.0;
  a.row_valid[row] = valid;
}

constexpr int kUnroll = 4;        // 16-byte chunks per lane per step (4 KiB per wave in flight)
constexpr float kStepMax = 0x1p64f;  // a step's sum of 2^(x log2 e - R) above this (or NaN) takes the exact path

// One step of a lane over kUnroll chunks.  Fast path: every exponential is
// taken against the lane's reference R as it stands, so there is no
// per-chunk max and no rescale; R only moves when a value exceeds it by more
// than 64 in log2 units (the step's sum passes 2^64), on the lane's first
// step (R = -inf makes every term +inf), or on inf / NaN input -- then the
// lane redoes the step exactly with online8, which moves R to the running
// max.  A stale (smaller) R only scales the lane's sum, which the (R, s)
// combines take into account.
template <bool TAIL>
__device__ __forceinline__ void fwd_step(const u32x4* p, int64_t c0, int64_t cpr, int lane, float& R, float& s) {
  u32x4 v[kUnroll];
  bool ok[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t c = c0 + u * kWave + lane;
    ok[u] = !TAIL || c < cpr;
    v[u] = ld16_stream(p + (ok[u] ? c : 0));
  }
  float f[kUnroll][8];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    unpack8(v[u], f[u]);
    if (TAIL && !ok[u]) {
#pragma unroll
      for (int i = 0; i < 8; ++i) f[u][i] = -INFINITY;
    }
  }
  float part[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int u = 0; u < kUnroll; ++u)
#pragma unroll
    for (int i = 0; i < 8; ++i) part[i & 3] += __builtin_amdgcn_exp2f(__builtin_fmaf(f[u][i], kLog2e, -R));
  const float step = (part[0] + part[1]) + (part[2] + part[3]);
  if (step <= kStepMax) {
    s += step;
  } else {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) online8(R, s, f[u]);
  }
}

// One wave per row, rows 16-byte granular (V % 8 == 0, aligned): lane l reads
// chunks (k * 64 + l), k = 0, 1, ... of the row, kUnroll per step, all loads
// of a step issued together.  Full steps carry no masks; the tail step's
// chunks past the row end read the row's first chunk and count as -inf.
__global__ __launch_bounds__(kThreads) void xent_fwd_vec(FwdArgs a) {
  const int64_t row = (int64_t)blockIdx.x * kWavesPerBlock + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  if (row >= a.M) return;
  const FwdTarget rt = row_target(a, row);
  const int lane = threadIdx.x & (kWave - 1);
  const u32x4* p = reinterpret_cast<const u32x4*>(a.logits + row * a.rs);
  const int64_t cpr = a.V / 8;
  constexpr int64_t kStep = (int64_t)kUnroll * kWave;
  const int64_t full = cpr / kStep * kStep;
  float R = -INFINITY, s = 0.0f;
  for (int64_t c0 = 0; c0 < full; c0 += kStep) fwd_step<false>(p, c0, cpr, lane, R, s);
  if (full < cpr) fwd_step<true>(p, full, cpr, lane, R, s);
  finish_row(a, row, rt, R, s);
}

// Any row stride / alignment / V: lane l reads elements l, l + 64, ...
__global__ __launch_bounds__(kThreads) void xent_fwd_scalar(FwdArgs a) {
  const int64_t row = (int64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (row >= a.M) return;
  const FwdTarget rt = row_target(a, row);
  const int lane = threadIdx.x & (kWave - 1);
  const uint16_t* p = a.logits + row * a.rs;
  float R = -INFINITY, s = 0.0f;
  for (int64_t j0 = 0; j0 < a.V; j0 += 8 * kWave) {
    float f[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t j = j0 + i * kWave + lane;
      f[i] = j < a.V ? bf_to_f(p[j]) : -INFINITY;
    }
    online8(R, s, f);
  }
  finish_row(a, row, rt, R, s);
}

// One block: loss = scale * sum(row_loss), total_weight = sum(row_valid), in a
// fixed order (thread t sums rows t, t + 1024, ... in fp64, then a tree).
constexpr int kFinThreads = 1024;
__global__ __launch_bounds__(kFinThreads) void xent_fwd_finish(const double* row_loss, const int32_t* row_valid,
                                                                int64_t M, double scale, float* loss, float* total_weight) {
  __shared__ double ls[kFinThreads];
  __shared__ int64_t cs[kFinThreads];
  double acc = 0.0;
  int64_t cnt = 0;
  for (int64_t i = threadIdx.x; i < M; i += kFinThreads) {
    acc += row_loss[i];
    cnt += row_valid[i];
  }
  ls[threadIdx.x] = acc;
  cs[threadIdx.x] = cnt;
  __syncthreads();
  for (int w = kFinThreads / 2; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) {
      ls[threadIdx.x] += ls[threadIdx.x + w];
      cs[threadIdx.x] += cs[threadIdx.x + w];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    loss[0] = (float)(ls[0] * scale);
    total_weight[0] = (float)cs[0];
  }
}

// ------------------------------------------------------------------ backward
struct BwdArgs {
  const float* lsm;
  int64_t rs;  // row stride of lsm, elements
  uint16_t* out;
  int64_t ors;  // row stride of out, elements
  int64_t M, V;
  const void* targets;
  int tbytes;
  int64_t ignore;
  float g;
  int32_t* err;
  int bpr;  // blocks per row (vector path)
};

// The row's target column and s_i = sum_j grad_ij (-g, or 0 for an ignored /
// out-of-range target).  Out-of-range targets raise the flag once per row.
__device__ __forceinline__ int64_t row_target(const BwdArgs& a, int64_t row, bool first, float& sum) {
  const int64_t t = target_at(a.targets, a.tbytes, row);
  const bool in_range = t >= 0 && t < a.V;
  if (t != a.ignore && !in_range && first && a.err) a.err[0] = 1;
  const bool valid = t != a.ignore && in_range;
  sum = valid ? -a.g : 0.0f;
  return valid ? t : -1;
}

// grad - expf(L) * s, as _log_softmax_backward_data evaluates it in fp32.
__device__ __forceinline__ float xent_grad(float l, bool is_target, float g, float sum) {
  const float grad = is_target ? -g : 0.0f;
  return grad - expf(l) * sum;
}

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Rows of V = 4k elements, lsm rows 16-byte and out rows 8-byte aligned.  A
// block covers 2048 consecutive elements of one row (block b: row b / bpr,
// float4 groups [(b % bpr) * 512, +512)); wave w takes groups
// [w * 128, +128) as two 1 KiB load instructions (lane l: groups l and
// 64 + l) and writes each group's 4 bf16 as one 8-byte store.  Measured on
// MI355X for this 4-byte-read / 2-byte-write stream: one group per lane per
// instruction beats 2-4 (1086-1144 us at [8192, 128256] against 996 us), and
// lanes holding 8 consecutive elements (two loads 32 bytes apart, one
// 16-byte store) ran at 1144 us.
constexpr int64_t kBwdBlockGroups = (int64_t)kThreads * 2;  // float4 groups per block

__global__ __launch_bounds__(kThreads) void xent_bwd_vec(BwdArgs a) {
  const int64_t row = (int64_t)((int)blockIdx.x / a.bpr);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & (kWave - 1);
  const int64_t g0 = (int64_t)((int)blockIdx.x - (int)row * a.bpr) * kBwdBlockGroups + (int64_t)wave * 128;
  const int64_t gpr = a.V / 4;
  const f32x4* p = reinterpret_cast<const f32x4*>(a.lsm + row * a.rs);
  u32x2* q = reinterpret_cast<u32x2*>(a.out + row * a.ors);
  f32x4 v[2];
  int64_t gi[2];
  bool ok[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    gi[h] = g0 + h * kWave + lane;
    ok[h] = gi[h] < gpr;
    v[h] = __builtin_nontemporal_load(p + (ok[h] ? gi[h] : 0));
  }
  // The row's target after the data loads: its scalar load (lgkmcnt) is
  // waited for independently of the data (vmcnt), whereas ahead of them it
  // held every block's data loads back by a chain of scalar round trips.
  __builtin_amdgcn_sched_barrier(0);
  float sum;
  const int64_t t = row_target(a, row, g0 == 0 && lane == 0, sum);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const bool has = (t >> 2) == gi[h];  // t = -1 for rows without a target column
    float o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = xent_grad(v[h][i], has && (t & 3) == i, a.g, sum);
    const u32x2 r = {pack_bf2(o[0], o[1]), pack_bf2(o[2], o[3])};
    if (ok[h]) __builtin_nontemporal_store(r, q + gi[h]);
  }
}

__global__ __launch_bounds__(kThreads) void xent_bwd_scalar(BwdArgs a) {
  const int64_t total = a.M * a.V;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total; i += (int64_t)gridDim.x * kThreads) {
    const int64_t r = i / a.V, j = i - r * a.V;
    float sum;
    const int64_t t = row_target(a, r, j == 0, sum);
    a.out[r * a.ors + j] = f_to_bf(xent_grad(a.lsm[r * a.rs + j], j == t, a.g, sum));
  }
}

// ------------------------------------------------------------------ forward + backward from the logits
// out_ij = bf16( grad_ij - exp(x_ij - lse_i) * s_i ) straight from the bf16
// logits (the _log_softmax -> nll_loss_forward -> nll_loss_backward ->
// _log_softmax_backward_data region with the fp32 log-softmax never stored),
// optionally with the forward's loss.  A row needs its lse before its first
// gradient, so a whole row is held on chip: one 1024-thread block per row,
// thread t holding chunks t + 1024 k (k < KC) in registers -- 16 chunks
// (64 VGPRs) cover V <= 131072, e.g. the 128256-entry vocabulary (256 KB of
// bf16 per row).  Each element is read once and written once: 4 bytes per
// element instead of the 6 of a forward pass followed by a pass that re-reads
// the logits.  The lse comes from the same (R, s) states as the forward
// (exponents by one fma against R = fl(max L)), combined across the block.
struct FbArgs {
  const uint16_t* logits;
  int64_t rs;  // row stride, elements
  uint16_t* out;
  int64_t ors;  // row stride of out, elements
  int64_t M, V;
  const void* targets;
  int tbytes;
  int64_t ignore;
  float g;             // upstream gradient of the summed loss
  double* row_loss;    // optional [M] (loss requested)
  int32_t* row_valid;  // optional [M]
  int32_t* err;
};

constexpr int kFbThreads = 1024;
constexpr int kFbMaxChunks = 16;  // 16-byte chunks per thread held in registers

// The row's combined (R, s), identical in every thread of the block: lanes
// fold by DPP and readlane, waves through LDS in a fixed order.
template <int NWAVES>
__device__ __forceinline__ void block_combine(float& R, float& s, float* lds) {
  combine_dpp<0xB1>(R, s);
  combine_dpp<0x4E>(R, s);
  combine_dpp<0x141>(R, s);
  combine_dpp<0x140>(R, s);
  float r0 = readlane_f(R, 0), s0 = readlane_f(s, 0);
  combine(r0, s0, readlane_f(R, 16), readlane_f(s, 16));
  float r1 = readlane_f(R, 32), s1 = readlane_f(s, 32);
  combine(r1, s1, readlane_f(R, 48), readlane_f(s, 48));
  combine(r0, s0, r1, s1);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & (kWave - 1)) == 0) {
    lds[w] = r0;
    lds[NWAVES + w] = s0;
  }
  __syncthreads();
  R = lds[0];
  s = lds[NWAVES];
#pragma unroll
  for (int i = 1; i < NWAVES; ++i) combine(R, s, lds[i], lds[NWAVES + i]);
}

struct RowTarget {
  int64_t t;     // target column, -1 when the row has none
  float sum;     // s_i = sum_j grad_ij: -g, or 0
  bool valid;
};

__device__ __forceinline__ RowTarget fb_target_of(const FbArgs& a, int64_t t) {
  const bool in_range = t >= 0 && t < a.V;
  const bool valid = t != a.ignore && in_range;
  if (t != a.ignore && !in_range && threadIdx.x == 0 && a.err) a.err[0] = 1;
  return RowTarget{valid ? t : -1, valid ? -a.g : 0.0f, valid};
}
__device__ __forceinline__ RowTarget fb_target(const FbArgs& a, int64_t row) {
  return fb_target_of(a, target_at(a.targets, a.tbytes, row));
}

// Thread 0 records the row's loss lse - x_t (x_t loaded before any store of
// the row, so out may alias the logits).  lse = (R + log2 s) / L with the
// fp32 log2 s of the gradient (|log2 s| < 18 for V < 2^17: within 2^-24 x 18
// of exact), summed and divided in fp64.
__device__ __forceinline__ void fb_row_loss(const FbArgs& a, int64_t row, const RowTarget& rt, float R, float lg,
                                            float xt) {
  if (a.row_loss == nullptr || threadIdx.x != 0) return;
  const double lse = ((double)R + (double)lg) / (double)kLog2e;
  a.row_loss[row] = rt.valid ? lse - (double)xt : 0.0;
  a.row_valid[row] = rt.valid;
}

// p = exp(x - lse) = 2^((x L - R) - log2 s): the fma is rounded relative to
// x L - R (small for the large p), and log2 s is subtracted afterwards, so
// p near 1 (a confident row's target, where grad - p sum cancels) carries
// fp32 relative error rather than an absolute error of ulp(R).
__device__ __forceinline__ float fb_grad(float x, float R, float lg, bool is_target, float g, float sum) {
  const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(x, kLog2e, -R) - lg);
  const float grad = is_target ? -g : 0.0f;
  return grad - p * sum;
}

// An empty asm that takes the packed chunks as in/out operands: the values
// unpacked in one pass cannot be reused in the next, so only the 4 x KC
// packed registers stay live across passes (reusing the 8 x KC unpacked
// floats needs twice the registers and spills at KC = 16).
template <int KC>
__device__ __forceinline__ void keep_packed(u32x4* v) {
#pragma unroll
  for (int k = 0; k < KC; ++k) asm volatile("" : "+v"(v[k]));
}

// Rows are addressed through raw buffer descriptors: the row base and length
// sit in SGPRs and each access takes a single 32-bit offset VGPR, where a
// 64-bit address takes two (32 per row at KC = 16, which spill).  The range
// check of the descriptor covers the VGPR offset: a load past the row end
// returns zeros and a store past it is dropped, so chunks beyond the row get
// the offset 0x80000000 (out of range for any row) instead of a branch, and
// a descriptor of length 0 fetches nothing.  Word 3 0x00020000 is the
// raw-buffer setting of the gfx9 family (32-bit data format).
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int kBufNT = 2;               // cache policy: non-temporal
constexpr uint32_t kOutOfRange = 0x80000000u;

__device__ __forceinline__ rsrc_t row_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// Byte offset of chunk k of thread tid, or kOutOfRange past the row.
__device__ __forceinline__ uint32_t fb_off(int tid, int k, int64_t cpr) {
  const int64_t c = tid + (int64_t)k * kFbThreads;
  return c < cpr ? (uint32_t)c * 16u : kOutOfRange;
}

// All KC loads of a row, issued together.
template <int KC>
__device__ __forceinline__ void fb_load_row(rsrc_t r, int tid, int64_t cpr, u32x4* v) {
#pragma unroll
  for (int k = 0; k < KC; ++k) v[k] = __builtin_amdgcn_raw_buffer_load_b128(r, fb_off(tid, k, cpr), 0, kBufNT);
}

// Target of `row` (int32 or int64 ids) by two 4-byte buffer loads and no
// branch: a load under a branch makes the wait-count pass drain every
// outstanding load and store at the join, i.e. the whole previous row's
// stores and this row's loads.  For int32 ids the high word may fall past
// the array, where the descriptor's range check returns 0.
__device__ __forceinline__ void fb_target_load(const FbArgs& a, int64_t row, uint32_t& lo, uint32_t& hi) {
  const rsrc_t r = row_rsrc(a.targets, (uint32_t)(a.M * a.tbytes));
  const uint32_t off = (uint32_t)(row * a.tbytes);
  lo = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
  hi = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, off + 4u, 0, 0);
}
// The words pass through an empty asm first, so that the compiler neither
// sinks the high word's load into a branch nor reads the words before the
// row's own loads are issued.
__device__ __forceinline__ int64_t fb_target_value(const FbArgs& a, uint32_t lo, uint32_t hi) {
  asm volatile("" : "+v"(lo), "+v"(hi));
  return a.tbytes == 8 ? (int64_t)(((uint64_t)hi << 32) | lo) : (int64_t)(int32_t)lo;
}

// Persistent: one block per CU walks rows blockIdx.x, + gridDim.x, ...; the
// next row's loads are issued as soon as the previous row's stores are, so
// the store stream of one row overlaps the load stream of the next (754 us
// against 791 us for one fresh block per row at [8192, 128256]).  Issuing
// the next row's chunk k right after row r's chunk k is unpacked, interleaved
// with row r's stores, measured slower (808 us).  The LDS slots of the block
// reduction alternate between rows (a slow wave may still read row r's slots
// while a fast one writes row r + 1's).
template <int KC>
__global__ __launch_bounds__(kFbThreads) void xent_fwd_bwd_vec(FbArgs a) {
  constexpr int kWaves = kFbThreads / kWave;
  __shared__ float red[2][2 * kWaves];
  const int64_t cpr = a.V / 8;
  const uint32_t row_bytes = (uint32_t)a.V * 2u;
  u32x4 v[KC];
  int parity = 0;
  for (int64_t row = blockIdx.x; row < a.M; row += gridDim.x, parity ^= 1) {
    // the thread index passes through an empty asm each row, so the chunk
    // offsets derived from it are recomputed where they are used instead of
    // being hoisted out of the loop (16 more live VGPRs)
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    // the row's target is requested ahead of its data: vmcnt counts in issue
    // order, so waiting for the target afterwards does not wait for the row
    uint32_t t_lo, t_hi;
    fb_target_load(a, row, t_lo, t_hi);
    __builtin_amdgcn_sched_barrier(0);
    fb_load_row<KC>(row_rsrc(a.logits + row * a.rs, row_bytes), tid, cpr, v);
    __builtin_amdgcn_sched_barrier(0);
    const rsrc_t ro = row_rsrc(a.out + row * a.ors, row_bytes);
    const RowTarget rt = fb_target_of(a, fb_target_value(a, t_lo, t_hi));
    // x_t for the row loss, loaded by every lane without a branch (an invalid
    // target reads out of range: 0) and consumed only before the block
    // combine, so its wait is not a wait for the whole row; thread 0 uses it
    uint16_t xtb = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(
        row_rsrc(a.logits + row * a.rs, row_bytes), rt.valid ? (uint32_t)rt.t * 2u : kOutOfRange, 0, 0);
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < KC; ++k) {
      if (tid + (int64_t)k * kFbThreads < cpr) {
        float f[8];
        unpack8(v[k], f);
#pragma unroll
        for (int i = 0; i < 8; ++i) m = fmaxf(m, f[i]);
      }
    }
    keep_packed<KC>(v);
    float R = m * kLog2e, s = 0.0f;
    if (R != -INFINITY) {
      float part[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int k = 0; k < KC; ++k) {
        if (tid + (int64_t)k * kFbThreads < cpr) {
          float f[8];
          unpack8(v[k], f);
#pragma unroll
          for (int i = 0; i < 8; ++i) part[i & 3] += __builtin_amdgcn_exp2f(__builtin_fmaf(f[i], kLog2e, -R));
        }
      }
      s = (part[0] + part[1]) + (part[2] + part[3]);
    }
    asm volatile("" : "+v"(xtb));  // x_t has arrived before the barrier: other waves may overwrite it after
    const float xt = (a.row_loss != nullptr && tid == 0 && rt.valid) ? bf_to_f(xtb) : 0.0f;
    block_combine<kWaves>(R, s, red[parity]);
    const float lg = log2f(s);
    fb_row_loss(a, row, rt, R, lg, xt);
    keep_packed<KC>(v);
    const int64_t tc = rt.t >> 3;  // -1 >> 3 = -1: no chunk matches
    const int ti = (int)(rt.t & 7);
    asm volatile("" : "+v"(tid));  // the store offsets are recomputed here, not kept from the loads
#pragma unroll
    for (int k = 0; k < KC; ++k) {
      const int64_t c = tid + (int64_t)k * kFbThreads;
      float f[8], o[8];
      unpack8(v[k], f);
      const uint32_t off = fb_off(tid, k, cpr);
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = fb_grad(f[i], R, lg, c == tc && i == ti, a.g, rt.sum);
      __builtin_amdgcn_raw_buffer_store_b128(pack8(o), ro, off, 0, kBufNT);
    }
  }
}

// Any V, stride or alignment: 256 threads per row, two passes over the row
// (the second re-reads it); each element is read before it is written by the
// same thread, so out may alias the logits here too.
__global__ __launch_bounds__(kThreads) void xent_fwd_bwd_scalar(FbArgs a) {
  __shared__ float red[2 * kWavesPerBlock];
  const int64_t row = blockIdx.x;
  const uint16_t* x = a.logits + row * a.rs;
  uint16_t* o = a.out + row * a.ors;
  const RowTarget rt = fb_target(a, row);
  const float xt = (a.row_loss != nullptr && threadIdx.x == 0 && rt.valid) ? bf_to_f(x[rt.t]) : 0.0f;
  float R = -INFINITY, s = 0.0f;
  for (int64_t j0 = 0; j0 < a.V; j0 += 8 * kThreads) {
    float f[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t j = j0 + i * kThreads + threadIdx.x;
      f[i] = j < a.V ? bf_to_f(x[j]) : -INFINITY;
    }
    online8(R, s, f);
  }
  asm volatile("" ::"v"(xt));  // x_t has arrived before the barrier: other waves may overwrite it after
  block_combine<kWavesPerBlock>(R, s, red);
  const float lg = log2f(s);
  fb_row_loss(a, row, rt, R, lg, xt);
  for (int64_t j = threadIdx.x; j < a.V; j += kThreads)
    o[j] = f_to_bf(fb_grad(bf_to_f(x[j]), R, lg, j == rt.t, a.g, rt.sum));
}

const void* fwd_bwd_vec_kernel(int kc) {
  switch (kc) {
    case 1: return reinterpret_cast<const void*>(xent_fwd_bwd_vec<1>);
    case 2: return reinterpret_cast<const void*>(xent_fwd_bwd_vec<2>);
    case 4: return reinterpret_cast<const void*>(xent_fwd_bwd_vec<4>);
    case 8: return reinterpret_cast<const void*>(xent_fwd_bwd_vec<8>);
    default: return reinterpret_cast<const void*>(xent_fwd_bwd_vec<16>);
  }
}

bool valid_target_bytes(int b) { return b == 4 || b == 8; }

}  // namespace
}  // namespace kp

using namespace kp;

extern "C" {

size_t kp_cross_entropy_fwd_workspace_size(int64_t M) {
  if (M <= 0) return 0;
  return (size_t)M * sizeof(double) + (size_t)M * sizeof(int32_t);
}

int kp_cross_entropy_fwd_bf16(const void* logits, int64_t row_stride, int64_t M, int64_t V, const void* targets,
                              int target_bytes, int64_t ignore_index, float scale, float* loss, float* total_weight,
                              float* row_lse, int32_t* error_flag, void* workspace, size_t workspace_bytes,
                              void* stream) {
  static const char* who = "kp_cross_entropy_fwd_bf16";
  if (M < 0 || V < 1) return fail(KP_EINVAL, "%s: bad shape [%lld, %lld]", who, (long long)M, (long long)V);
  if (loss == nullptr || total_weight == nullptr) return fail(KP_EINVAL, "%s: loss / total_weight is NULL", who);
  if (!valid_target_bytes(target_bytes)) return fail(KP_EINVAL, "%s: target_bytes must be 4 or 8", who);
  if (M > 1 && row_stride < V) return fail(KP_EINVAL, "%s: row stride %lld < V", who, (long long)row_stride);
  const size_t need = kp_cross_entropy_fwd_workspace_size(M);
  if (M > 0 && (logits == nullptr || targets == nullptr)) return fail(KP_EINVAL, "%s: logits / targets NULL", who);
  if (workspace_bytes < need || (need && workspace == nullptr))
    return fail(KP_EWORKSPACE, "%s: workspace of %zu bytes needed", who, need);
  if ((reinterpret_cast<uintptr_t>(workspace) & 7) != 0) return fail(KP_EINVAL, "%s: workspace not 8-byte aligned", who);
  if (M > ((int64_t)1 << 31) * kWavesPerBlock) return fail(KP_EUNSUPPORTED, "%s: too many rows", who);
  hipStream_t st = as_stream(stream);
  FwdArgs a{};
  a.logits = static_cast<const uint16_t*>(logits);
  a.rs = row_stride;
  a.M = M;
  a.V = V;
  a.targets = targets;
  a.tbytes = target_bytes;
  a.ignore = ignore_index;
  a.row_loss = static_cast<double*>(workspace);
  a.row_valid = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + (size_t)M * sizeof(double));
  a.lse_out = row_lse;
  a.err = error_flag;
  if (M > 0) {
    const bool vec = V % 8 == 0 && aligned16(logits) && (M == 1 || row_stride % 8 == 0);
    const unsigned blocks = (unsigned)ceil_div(M, kWavesPerBlock);
    void* args[] = {&a};
    launch_dominant_raw(reinterpret_cast<const void*>(vec ? xent_fwd_vec : xent_fwd_scalar), dim3(blocks),
                        dim3(kThreads), args, 0, st);
    const int rc = check_launch(who);
    if (rc != KP_OK) return rc;
  }
  hipLaunchKernelGGL(xent_fwd_finish, dim3(1), dim3(kFinThreads), 0, st, a.row_loss, a.row_valid, M, (double)scale,
                     loss, total_weight);
  return check_launch(who);
}

int kp_cross_entropy_bwd_bf16(const float* log_softmax, int64_t lsm_row_stride, const void* targets, int target_bytes,
                              int64_t ignore_index, float grad_loss, void* grad_logits, int64_t out_row_stride,
                              int64_t M, int64_t V, int32_t* error_flag, void* stream) {
  static const char* who = "kp_cross_entropy_bwd_bf16";
  if (M < 0 || V < 1) return fail(KP_EINVAL, "%s: bad shape [%lld, %lld]", who, (long long)M, (long long)V);
  if (!valid_target_bytes(target_bytes)) return fail(KP_EINVAL, "%s: target_bytes must be 4 or 8", who);
  if (M == 0) return KP_OK;
  if (log_softmax == nullptr || targets == nullptr || grad_logits == nullptr)
    return fail(KP_EINVAL, "%s: NULL operand", who);
  if (M > 1 && (lsm_row_stride < V || out_row_stride < V)) return fail(KP_EINVAL, "%s: row stride < V", who);
  if (M > (((int64_t)1 << 62) / V)) return fail(KP_EUNSUPPORTED, "%s: too large", who);
  BwdArgs a{};
  a.lsm = log_softmax;
  a.rs = lsm_row_stride;
  a.out = static_cast<uint16_t*>(grad_logits);
  a.ors = out_row_stride;
  a.M = M;
  a.V = V;
  a.targets = targets;
  a.tbytes = target_bytes;
  a.ignore = ignore_index;
  a.g = grad_loss;
  a.err = error_flag;
  const bool vec = V % 4 == 0 && aligned16(log_softmax) && (reinterpret_cast<uintptr_t>(grad_logits) & 7) == 0 &&
                   (M == 1 || (lsm_row_stride % 4 == 0 && out_row_stride % 4 == 0));
  void* args[] = {&a};
  if (vec) {
    const int64_t bpr = ceil_div(V / 4, kBwdBlockGroups);
    if (bpr * M > 0x7fffffffLL) return fail(KP_EUNSUPPORTED, "%s: too many blocks", who);
    a.bpr = (int)bpr;
    launch_dominant_raw(reinterpret_cast<const void*>(xent_bwd_vec), dim3((unsigned)(bpr * M)), dim3(kThreads), args,
                        0, as_stream(stream));
  } else {
    const int64_t want = ceil_div(M * V, kThreads);
    const int64_t cap = (int64_t)cu_count() * 16;
    launch_dominant_raw(reinterpret_cast<const void*>(xent_bwd_scalar), dim3((unsigned)(want < cap ? want : cap)),
                        dim3(kThreads), args, 0, as_stream(stream));
  }
  return check_launch(who);
}

int kp_cross_entropy_fwd_bwd_bf16(const void* logits, int64_t row_stride, int64_t M, int64_t V, const void* targets,
                                  int target_bytes, int64_t ignore_index, float grad_loss, void* grad_logits,
                                  int64_t out_row_stride, float scale, float* loss, float* total_weight,
                                  int32_t* error_flag, void* workspace, size_t workspace_bytes, void* stream) {
  static const char* who = "kp_cross_entropy_fwd_bwd_bf16";
  if (M < 0 || V < 1) return fail(KP_EINVAL, "%s: bad shape [%lld, %lld]", who, (long long)M, (long long)V);
  if (!valid_target_bytes(target_bytes)) return fail(KP_EINVAL, "%s: target_bytes must be 4 or 8", who);
  if ((loss == nullptr) != (total_weight == nullptr))
    return fail(KP_EINVAL, "%s: loss and total_weight are both given or both NULL", who);
  const bool want_loss = loss != nullptr;
  const size_t need = want_loss ? kp_cross_entropy_fwd_workspace_size(M) : 0;
  if (workspace_bytes < need || (need && workspace == nullptr))
    return fail(KP_EWORKSPACE, "%s: workspace of %zu bytes needed", who, need);
  if (need && (reinterpret_cast<uintptr_t>(workspace) & 7) != 0)
    return fail(KP_EINVAL, "%s: workspace not 8-byte aligned", who);
  if (M > 0 && (logits == nullptr || targets == nullptr || grad_logits == nullptr))
    return fail(KP_EINVAL, "%s: NULL operand", who);
  if (M > 1 && (row_stride < V || out_row_stride < V)) return fail(KP_EINVAL, "%s: row stride < V", who);
  if (M > 0x7fffffffLL) return fail(KP_EUNSUPPORTED, "%s: too many rows", who);
  hipStream_t st = as_stream(stream);
  FbArgs a{};
  a.logits = static_cast<const uint16_t*>(logits);
  a.rs = row_stride;
  a.out = static_cast<uint16_t*>(grad_logits);
  a.ors = out_row_stride;
  a.M = M;
  a.V = V;
  a.targets = targets;
  a.tbytes = target_bytes;
  a.ignore = ignore_index;
  a.g = grad_loss;
  a.err = error_flag;
  if (want_loss) {
    a.row_loss = static_cast<double*>(workspace);
    a.row_valid = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + (size_t)M * sizeof(double));
  }
  if (M > 0) {
    const int64_t cpr = V / 8;
    const bool vec = V % 8 == 0 && aligned16(logits) && aligned16(grad_logits) &&
                     (M == 1 || (row_stride % 8 == 0 && out_row_stride % 8 == 0)) &&
                     cpr <= (int64_t)kFbThreads * kFbMaxChunks &&
                     M * target_bytes <= 0xffffffffLL;  // the targets' buffer descriptor is 32-bit
    void* args[] = {&a};
    if (vec) {
      int kc = 1;
      while ((int64_t)kc * kFbThreads < cpr) kc *= 2;
      const int64_t cus = cu_count();
      const unsigned blocks = (unsigned)(M < cus ? M : cus);
      launch_dominant_raw(fwd_bwd_vec_kernel(kc), dim3(blocks), dim3(kFbThreads), args, 0, st);
    } else {
      launch_dominant_raw(reinterpret_cast<const void*>(xent_fwd_bwd_scalar), dim3((unsigned)M), dim3(kThreads), args,
                          0, st);
    }
    const int rc = check_launch(who);
    if (rc != KP_OK) return rc;
  }
  if (!want_loss) return KP_OK;
  hipLaunchKernelGGL(xent_fwd_finish, dim3(1), dim3(kFinThreads), 0, st, a.row_loss, a.row_valid, M, (double)scale,
                     loss, total_weight);
  return check_launch(who);
}

}  // extern "C"
