// SwiGLU gate forward and backward for gfx950: the pointwise region between
// the w1/w3 and w2 projections of a Llama feed-forward block.
//
//   forward   out = bf16( bf16(silu(a)) * b )                    (2 reads, 1 write)
//   backward  db  = bf16( g * s )                                 (4 reads, 2 writes)
//             da  = bf16( silu'(a) applied to bf16(g * b) )
//   silu      out = bf16( silu(a) )                               (1 read, 1 write)
//   forward recomputed with the backward (s = bf16(silu(a)) never stored):
//             h = bf16(s * b), db = bf16(g * s), da as above      (3 reads, 3 writes)
//
// with silu(x) = x / (1 + exp(-x)) and silu_backward(t, x) =
// t * sig * (1 + x * (1 - sig)), sig = 1 / (1 + exp(-x)), all in fp32 with the
// bf16 roundings where the eager op sequence materialises a bf16 tensor.
//
// Pure streaming: every element is read and written exactly once, so the
// kernels are HBM-bound one-shot grids.  A block owns 4 x 256 consecutive
// 16-byte chunks (8 bf16 each) of every array; thread t holds chunks
// t + 256 u, so each wave64 load or store moves 1 KiB of consecutive bytes.
// All loads of a chunk group are issued before any math (one wait), loads and
// stores are non-temporal.  Row-strided views run as rows of whole blocks
// (block -> (row, column segment)); contiguous arrays run as one flat row.
// Shapes whose rows, strides or pointers are not 16-byte granular take a
// scalar grid-stride kernel with the same arithmetic.
#include "kp_common.hpp"
#include "kp_internal.hpp"

namespace kp {
namespace {

constexpr int kThreads = 256;
constexpr int kPer = 4;                                    // chunks per thread per array
constexpr int64_t kBlockChunks = (int64_t)kThreads * kPer;  // 16-byte chunks per block per array

// ------------------------------------------------------------------ math
// The eager formulas, evaluated in fp32 the way torch's silu / silu_backward
// kernels do (expf, IEEE division, this operation order).
__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }

// sig = fl(1 / fl(1 + expf(-x))) as eager computes it.  For |x| < 16 the
// IEEE division is replaced by rcp and one Newton step, which gives the same
// fp32 value for every bf16 x in that range (all 33536 of them: compared bit
// for bit on the device by kp_swiglu_math_selftest in tests/test_gpu_swiglu.py):
// ~3 VALU instructions instead of ~10.
__device__ __forceinline__ float sigmoid_f(float x) {
  const float d = 1.0f + expf(-x);
  if (!(__builtin_fabsf(x) < 16.0f)) return 1.0f / d;
  const float r = __builtin_amdgcn_rcpf(d);
  return __builtin_fmaf(__builtin_fmaf(-d, r, 1.0f), r, r);
}

__device__ __forceinline__ float silu_bwd_f(float t, float x) {
  const float sig = sigmoid_f(x);
  return t * sig * (1.0f + x * (1.0f - sig));
}

// bf16(silu(x)) for a bf16 x: bit for bit the bf16 rounding of silu_f(x), at
// well under half of silu_f's VALU cost (~11 instead of ~28 instructions).
// The forward streams 3 arrays at full HBM rate; with silu_f's instruction
// count the chip throttles its clock under sustained load (the kernel drifts
// from 116 to 170 us and back to ~130), with this one it holds 113 us.
//
// Fast path, |x| < 32: e^-x = 2^(x * -hi) * (1 + x * -lo'), hi = log2(e) to 16
// bits (x * hi is exact: 8 + 16 significant bits), lo' = (log2(e) - hi) ln 2
// (first order suffices: |x lo'| < 2^-12); then x * rcp(1 + e^-x).  Over every
// bf16 x with |x| < 32 this lands within 3 fp32 ulps of silu_f(x).
// Rounding test (Ziv): two fp32 values within 3 ulps of each other round to
// different bf16 values only if a bf16 rounding midpoint lies between them,
// so when the fast value is more than kMidUlps (> 3) ulps from every midpoint
// its rounding is silu_f's.  Otherwise -- about 17 in 65536 values -- and for
// |x| >= 32, infinities and NaN, silu_f decides.  The test over all 65536 bf16
// inputs against torch's eager silu is in tests/test_gpu_swiglu.py.
constexpr float kLog2eHi = 1.44268798828125f;   // 0x1.7154p+0: log2(e) rounded to 16 significant bits
constexpr float kLog2eLoLn2 = 4.888495e-06f;    // (log2(e) - kLog2eHi) * ln(2)
constexpr uint32_t kMidUlps = 8;

__device__ __forceinline__ float silu_bf16(float x) {
  const float big = __builtin_amdgcn_exp2f(x * -kLog2eHi);
  const float em = __builtin_fmaf(big, x * -kLog2eLoLn2, big);
  float q = x * __builtin_amdgcn_rcpf(1.0f + em);
  // low 16 bits of q within kMidUlps of 0x8000 <=> within kMidUlps fp32 ulps of a bf16 midpoint
  const uint32_t off = (__float_as_uint(q) + (kMidUlps - 0x8000u)) & 0xffffu;
  if (!(__builtin_fabsf(x) < 32.0f) || off <= 2 * kMidUlps) q = silu_f(x);
  return round_bf(q);
}

enum Op : int { kFwd = 0, kBwd = 1, kSilu = 2, kFwdBwd = 3 };

// Inputs and outputs of each op, in argument order:
//   kFwd (a, b) -> out;  kBwd (g, s, b, a) -> (db, da);  kSilu (a) -> out;
//   kFwdBwd (a, b, g) -> (h, db, da).
constexpr int n_in(int op) { return op == kFwd ? 2 : op == kBwd ? 4 : op == kSilu ? 1 : 3; }
constexpr int n_out(int op) { return op == kFwd ? 1 : op == kBwd ? 2 : op == kSilu ? 1 : 3; }

// One element: x[i] are the inputs as fp32 (bf16 values), y[o] the fp32
// results before their bf16 rounding.
template <int OP>
__device__ __forceinline__ void apply1(const float* x, float* y) {
  if constexpr (OP == kFwd) {
    y[0] = silu_bf16(x[0]) * x[1];
  } else if constexpr (OP == kBwd) {
    y[0] = x[0] * x[1];
    y[1] = silu_bwd_f(round_bf(x[0] * x[2]), x[3]);
  } else if constexpr (OP == kSilu) {
    y[0] = silu_bf16(x[0]);
  } else {
    const float sv = silu_bf16(x[0]);
    y[0] = sv * x[1];
    y[1] = x[2] * sv;
    y[2] = silu_bwd_f(round_bf(x[2] * x[1]), x[0]);
  }
}

template <int OP>
__device__ __forceinline__ void apply8(const u32x4* in, u32x4* out) {
  constexpr int NI = n_in(OP), NO = n_out(OP);
  float x[NI][8], y[NO][8];
#pragma unroll
  for (int i = 0; i < NI; ++i) unpack8(in[i], x[i]);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float xe[NI], ye[NO];
#pragma unroll
    for (int i = 0; i < NI; ++i) xe[i] = x[i][e];
    apply1<OP>(xe, ye);
#pragma unroll
    for (int o = 0; o < NO; ++o) y[o][e] = ye[o];
  }
#pragma unroll
  for (int o = 0; o < NO; ++o) out[o] = pack8(y[o]);
}

// ------------------------------------------------------------------ 16-byte path
// Arrays are [rows, cpr] in 16-byte chunks with per-array row strides (in
// chunks).  Block b covers row b / bpr, chunks [(b % bpr) * kBlockChunks, +kBlockChunks).
struct VecArgs {
  const u32x4* in[4];
  u32x4* out[3];
  int64_t in_rs[4], out_rs[3];  // row strides in chunks
  int64_t cpr;                  // chunks per row
  int bpr;                      // blocks per row
};

template <bool FULL>
__device__ __forceinline__ int64_t chunk_of(const VecArgs& a, int u, int64_t c0, bool& ok) {
  const int64_t c = c0 + threadIdx.x + (int64_t)u * kThreads;
  ok = FULL || c < a.cpr;
  return ok ? c : 0;
}

template <int OP, bool FULL>
__device__ __forceinline__ void tile(const VecArgs& a, int64_t row, int64_t c0) {
  constexpr int NI = n_in(OP), NO = n_out(OP);
  u32x4 v[NI][kPer];
  int64_t c[kPer];
  bool ok[kPer];
#pragma unroll
  for (int u = 0; u < kPer; ++u) c[u] = chunk_of<FULL>(a, u, c0, ok[u]);
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const u32x4* p = a.in[i] + row * a.in_rs[i];
#pragma unroll
    for (int u = 0; u < kPer; ++u) v[i][u] = ld16_stream(p + c[u]);
  }
  // Every load of the tile is in flight before the first use: without this
  // fence the scheduler starts the math of chunk 0 after a few loads.
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    u32x4 in[NI], r[NO];
#pragma unroll
    for (int i = 0; i < NI; ++i) in[i] = v[i][u];
    apply8<OP>(in, r);
    if (ok[u]) {
#pragma unroll
      for (int o = 0; o < NO; ++o) st16_stream(a.out[o] + row * a.out_rs[o] + c[u], r[o]);
    }
  }
}

// Loads of a partial tile are clamped to chunk 0 of the row (always in
// bounds) rather than predicated, so the load batch issues unbranched; only
// the stores are predicated.
template <int OP>
__device__ __forceinline__ void vec_body(const VecArgs& a) {
  const int row = (int)blockIdx.x / a.bpr;
  const int64_t c0 = (int64_t)((int)blockIdx.x - row * a.bpr) * kBlockChunks;
  if (c0 + kBlockChunks <= a.cpr) tile<OP, true>(a, row, c0);
  else tile<OP, false>(a, row, c0);
}

__global__ __launch_bounds__(kThreads) void swiglu_fwd_vec(VecArgs a) { vec_body<kFwd>(a); }
__global__ __launch_bounds__(kThreads) void swiglu_bwd_vec(VecArgs a) { vec_body<kBwd>(a); }
__global__ __launch_bounds__(kThreads) void silu_vec(VecArgs a) { vec_body<kSilu>(a); }
__global__ __launch_bounds__(kThreads) void swiglu_fwd_bwd_vec(VecArgs a) { vec_body<kFwdBwd>(a); }

// ------------------------------------------------------------------ scalar path
struct ScalarArgs {
  const uint16_t* in[4];
  uint16_t* out[3];
  int64_t in_rs[4], out_rs[3];  // row strides in elements
  int64_t M, N;
};

template <int OP>
__device__ __forceinline__ void scalar_body(const ScalarArgs& a) {
  constexpr int NI = n_in(OP), NO = n_out(OP);
  const int64_t total = a.M * a.N;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total; i += (int64_t)gridDim.x * kThreads) {
    const int64_t r = i / a.N, c = i - r * a.N;
    float x[NI], y[NO];
#pragma unroll
    for (int k = 0; k < NI; ++k) x[k] = bf_to_f(a.in[k][r * a.in_rs[k] + c]);
    apply1<OP>(x, y);
#pragma unroll
    for (int k = 0; k < NO; ++k) a.out[k][r * a.out_rs[k] + c] = f_to_bf(y[k]);
  }
}

__global__ __launch_bounds__(kThreads) void swiglu_fwd_scalar(ScalarArgs a) { scalar_body<kFwd>(a); }
__global__ __launch_bounds__(kThreads) void swiglu_bwd_scalar(ScalarArgs a) { scalar_body<kBwd>(a); }
__global__ __launch_bounds__(kThreads) void silu_scalar(ScalarArgs a) { scalar_body<kSilu>(a); }
__global__ __launch_bounds__(kThreads) void swiglu_fwd_bwd_scalar(ScalarArgs a) { scalar_body<kFwdBwd>(a); }

// ------------------------------------------------------------------ host side
// Validates and launches one pointwise op over nin inputs / nout outputs of an
// [M, N] bf16 matrix (unit inner stride, row strides in elements).
const void* vec_kernel(int op) {
  switch (op) {
    case kFwd: return reinterpret_cast<const void*>(swiglu_fwd_vec);
    case kBwd: return reinterpret_cast<const void*>(swiglu_bwd_vec);
    case kSilu: return reinterpret_cast<const void*>(silu_vec);
    default: return reinterpret_cast<const void*>(swiglu_fwd_bwd_vec);
  }
}

const void* scalar_kernel(int op) {
  switch (op) {
    case kFwd: return reinterpret_cast<const void*>(swiglu_fwd_scalar);
    case kBwd: return reinterpret_cast<const void*>(swiglu_bwd_scalar);
    case kSilu: return reinterpret_cast<const void*>(silu_scalar);
    default: return reinterpret_cast<const void*>(swiglu_fwd_bwd_scalar);
  }
}

int launch_pointwise(const char* who, int op, const void* const* in, const int64_t* in_rs, void* const* out,
                     const int64_t* out_rs, int64_t M, int64_t N, hipStream_t stream) {
  const int nin = n_in(op), nout = n_out(op);
  if (M < 0 || N < 0) return fail(KP_EINVAL, "%s: negative shape [%lld, %lld]", who, (long long)M, (long long)N);
  if (M == 0 || N == 0) return KP_OK;
  for (int i = 0; i < nin; ++i) {
    if (in[i] == nullptr) return fail(KP_EINVAL, "%s: input %d is NULL", who, i);
    if (M > 1 && in_rs[i] < N) return fail(KP_EINVAL, "%s: input %d row stride %lld < N=%lld", who, i, (long long)in_rs[i], (long long)N);
  }
  for (int i = 0; i < nout; ++i) {
    if (out[i] == nullptr) return fail(KP_EINVAL, "%s: output %d is NULL", who, i);
    if (M > 1 && out_rs[i] < N)
      return fail(KP_EINVAL, "%s: output %d row stride %lld < N=%lld", who, i, (long long)out_rs[i], (long long)N);
  }
  if (M > (((int64_t)1 << 62) / N)) return fail(KP_EUNSUPPORTED, "%s: [%lld, %lld] too large", who, (long long)M, (long long)N);

  bool vec = (N % 8) == 0;
  bool flat = true;  // every array is one contiguous run of M*N elements
  for (int i = 0; i < nin; ++i) {
    vec = vec && aligned16(in[i]) && (M == 1 || in_rs[i] % 8 == 0);
    flat = flat && (M == 1 || in_rs[i] == N);
  }
  for (int i = 0; i < nout; ++i) {
    vec = vec && aligned16(out[i]) && (M == 1 || out_rs[i] % 8 == 0);
    flat = flat && (M == 1 || out_rs[i] == N);
  }
  if (vec) {
    VecArgs a{};
    int64_t rows = M, cpr = N / 8;
    if (flat) {
      rows = 1;
      cpr = M * N / 8;
    }
    for (int i = 0; i < nin; ++i) {
      a.in[i] = static_cast<const u32x4*>(in[i]);
      a.in_rs[i] = flat ? 0 : in_rs[i] / 8;
    }
    for (int i = 0; i < nout; ++i) {
      a.out[i] = static_cast<u32x4*>(out[i]);
      a.out_rs[i] = flat ? 0 : out_rs[i] / 8;
    }
    a.cpr = cpr;
    const int64_t bpr = ceil_div(cpr, kBlockChunks);
    const int64_t blocks = bpr * rows;
    if (blocks > 0x7fffffffLL) return fail(KP_EUNSUPPORTED, "%s: too many blocks for one launch", who);
    a.bpr = (int)bpr;
    void* args[] = {&a};
    launch_dominant_raw(vec_kernel(op), dim3((unsigned)blocks), dim3(kThreads), args, 0, stream);
    return check_launch(who);
  }
  ScalarArgs a{};
  for (int i = 0; i < nin; ++i) {
    a.in[i] = static_cast<const uint16_t*>(in[i]);
    a.in_rs[i] = in_rs[i];
  }
  for (int i = 0; i < nout; ++i) {
    a.out[i] = static_cast<uint16_t*>(out[i]);
    a.out_rs[i] = out_rs[i];
  }
  a.M = M;
  a.N = N;
  const int64_t want = ceil_div(M * N, kThreads);
  const int64_t cap = (int64_t)cu_count() * 16;
  const unsigned blocks = (unsigned)(want < cap ? want : cap);
  void* args[] = {&a};
  launch_dominant_raw(scalar_kernel(op), dim3(blocks), dim3(kThreads), args, 0, stream);
  return check_launch(who);
}

// Self-test of the arithmetic above over every bf16 input (x = bit pattern
// i): the fast sigmoid against the IEEE quotient it replaces, and the fast
// bf16 silu against the bf16 rounding of silu_f, as fp32 bit patterns.
__global__ __launch_bounds__(kThreads) void swiglu_math_bits(uint32_t* sig_fast, uint32_t* sig_ieee,
                                                             uint32_t* silu_fast, uint32_t* silu_ref) {
  const int i = blockIdx.x * kThreads + threadIdx.x;
  if (i >= 65536) return;
  const float x = bf_to_f((uint16_t)i);
  sig_fast[i] = __float_as_uint(sigmoid_f(x));
  sig_ieee[i] = __float_as_uint(1.0f / (1.0f + expf(-x)));
  silu_fast[i] = __float_as_uint(silu_bf16(x));
  silu_ref[i] = __float_as_uint(round_bf(silu_f(x)));
}

}  // namespace
}  // namespace kp

using namespace kp;

extern "C" {

int kp_swiglu_math_selftest(uint32_t* sig_fast, uint32_t* sig_ieee, uint32_t* silu_fast, uint32_t* silu_ref,
                            void* stream) {
  static const char* who = "kp_swiglu_math_selftest";
  if (!sig_fast || !sig_ieee || !silu_fast || !silu_ref) return fail(KP_EINVAL, "%s: NULL output", who);
  hipLaunchKernelGGL(swiglu_math_bits, dim3(65536 / kThreads), dim3(kThreads), 0, as_stream(stream), sig_fast,
                     sig_ieee, silu_fast, silu_ref);
  return check_launch(who);
}

int kp_swiglu_fwd_bf16(const void* a, int64_t a_rs, const void* b, int64_t b_rs, void* out, int64_t out_rs, int64_t M,
                       int64_t N, void* stream) {
  const void* in[2] = {a, b};
  const int64_t in_rs[2] = {a_rs, b_rs};
  void* outs[1] = {out};
  const int64_t o_rs[1] = {out_rs};
  return launch_pointwise("kp_swiglu_fwd_bf16", kFwd, in, in_rs, outs, o_rs, M, N, as_stream(stream));
}

int kp_swiglu_bwd_bf16(const void* g, int64_t g_rs, const void* s, int64_t s_rs, const void* b, int64_t b_rs,
                       const void* a, int64_t a_rs, void* db, int64_t db_rs, void* da, int64_t da_rs, int64_t M,
                       int64_t N, void* stream) {
  const void* in[4] = {g, s, b, a};
  const int64_t in_rs[4] = {g_rs, s_rs, b_rs, a_rs};
  void* outs[2] = {db, da};
  const int64_t o_rs[2] = {db_rs, da_rs};
  return launch_pointwise("kp_swiglu_bwd_bf16", kBwd, in, in_rs, outs, o_rs, M, N, as_stream(stream));
}

int kp_silu_bf16(const void* a, int64_t a_rs, void* out, int64_t out_rs, int64_t M, int64_t N, void* stream) {
  const void* in[1] = {a};
  const int64_t in_rs[1] = {a_rs};
  void* outs[1] = {out};
  const int64_t o_rs[1] = {out_rs};
  return launch_pointwise("kp_silu_bf16", kSilu, in, in_rs, outs, o_rs, M, N, as_stream(stream));
}

int kp_swiglu_fwd_bwd_bf16(const void* a, int64_t a_rs, const void* b, int64_t b_rs, const void* g, int64_t g_rs,
                           void* h, int64_t h_rs, void* db, int64_t db_rs, void* da, int64_t da_rs, int64_t M,
                           int64_t N, void* stream) {
  const void* in[3] = {a, b, g};
  const int64_t in_rs[3] = {a_rs, b_rs, g_rs};
  void* outs[3] = {h, db, da};
  const int64_t o_rs[3] = {h_rs, db_rs, da_rs};
  return launch_pointwise("kp_swiglu_fwd_bwd_bf16", kFwdBwd, in, in_rs, outs, o_rs, M, N, as_stream(stream));
}

}  // extern "C"
