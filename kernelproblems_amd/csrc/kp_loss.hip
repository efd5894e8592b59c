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

// Row-wave epilogue: reduce the lanes' states, then lane 0 writes the row's loss.
__device__ __forceinline__ void finish_row(const FwdArgs& a, int64_t row, float R, float s) {
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
  const int64_t t = target_at(a.targets, a.tbytes, row);
  int valid = t != a.ignore;
  if (valid && (t < 0 || t >= a.V)) {
    valid = 0;
    if (a.err) a.err[0] = 1;
  }
  a.row_loss[row] = valid ? lse - (double)bf_to_f(a.logits[row * a.rs + t]) : 0.0;
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
  const int64_t row = (int64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (row >= a.M) return;
  const int lane = threadIdx.x & (kWave - 1);
  const u32x4* p = reinterpret_cast<const u32x4*>(a.logits + row * a.rs);
  const int64_t cpr = a.V / 8;
  constexpr int64_t kStep = (int64_t)kUnroll * kWave;
  const int64_t full = cpr / kStep * kStep;
  float R = -INFINITY, s = 0.0f;
  for (int64_t c0 = 0; c0 < full; c0 += kStep) fwd_step<false>(p, c0, cpr, lane, R, s);
  if (full < cpr) fwd_step<true>(p, full, cpr, lane, R, s);
  finish_row(a, row, R, s);
}

// Any row stride / alignment / V: lane l reads elements l, l + 64, ...
__global__ __launch_bounds__(kThreads) void xent_fwd_scalar(FwdArgs a) {
  const int64_t row = (int64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (row >= a.M) return;
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
  finish_row(a, row, R, s);
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
  float sum;
  const int64_t t = row_target(a, row, g0 == 0 && lane == 0, sum);
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

}  // extern "C"
