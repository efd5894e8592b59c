// SwiGLU gate forward and backward for gfx950: the pointwise region between
// the w1/w3 and w2 projections of a Llama feed-forward block.
//
//   forward   out = bf16( bf16(silu(a)) * b )                    (2 reads, 1 write)
//   backward  db  = bf16( g * s )                                 (4 reads, 2 writes)
//             da  = bf16( silu'(a) applied to bf16(g * b) )
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

__device__ __forceinline__ float silu_bwd_f(float t, float x) {
  const float sig = 1.0f / (1.0f + expf(-x));
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

__device__ __forceinline__ u32x4 fwd8(const u32x4& a, const u32x4& b) {
  float af[8], bf[8], o[8];
  unpack8(a, af);
  unpack8(b, bf);
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = silu_bf16(af[i]) * bf[i];
  return pack8(o);
}

__device__ __forceinline__ void bwd8(const u32x4& g, const u32x4& s, const u32x4& b, const u32x4& a, u32x4& db,
                                     u32x4& da) {
  float gf[8], sf[8], bf[8], af[8], o0[8], o1[8];
  unpack8(g, gf);
  unpack8(s, sf);
  unpack8(b, bf);
  unpack8(a, af);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    o0[i] = gf[i] * sf[i];
    o1[i] = silu_bwd_f(round_bf(gf[i] * bf[i]), af[i]);
  }
  db = pack8(o0);
  da = pack8(o1);
}

// ------------------------------------------------------------------ 16-byte path
// Arrays are [rows, cpr] in 16-byte chunks with per-array row strides (in
// chunks).  Block b covers row b / bpr, chunks [(b % bpr) * kBlockChunks, +kBlockChunks).
struct VecArgs {
  const u32x4* in[4];
  u32x4* out[2];
  int64_t in_rs[4], out_rs[2];  // row strides in chunks
  int64_t cpr;                  // chunks per row
  int bpr;                      // blocks per row
};

template <bool FULL>
__device__ __forceinline__ int64_t chunk_of(const VecArgs& a, int u, int64_t c0, bool& ok) {
  const int64_t c = c0 + threadIdx.x + (int64_t)u * kThreads;
  ok = FULL || c < a.cpr;
  return ok ? c : 0;
}

template <bool FULL>
__device__ __forceinline__ void fwd_tile(const VecArgs& a, int64_t row, int64_t c0) {
  const u32x4* pa = a.in[0] + row * a.in_rs[0];
  const u32x4* pb = a.in[1] + row * a.in_rs[1];
  u32x4* po = a.out[0] + row * a.out_rs[0];
  u32x4 va[kPer], vb[kPer];
  int64_t c[kPer];
  bool ok[kPer];
#pragma unroll
  for (int u = 0; u < kPer; ++u) c[u] = chunk_of<FULL>(a, u, c0, ok[u]);
#pragma unroll
  for (int u = 0; u < kPer; ++u) va[u] = ld16_stream(pa + c[u]);
#pragma unroll
  for (int u = 0; u < kPer; ++u) vb[u] = ld16_stream(pb + c[u]);
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const u32x4 r = fwd8(va[u], vb[u]);
    if (ok[u]) st16_stream(po + c[u], r);
  }
}

template <bool FULL>
__device__ __forceinline__ void bwd_tile(const VecArgs& a, int64_t row, int64_t c0) {
  const u32x4* pg = a.in[0] + row * a.in_rs[0];
  const u32x4* ps = a.in[1] + row * a.in_rs[1];
  const u32x4* pb = a.in[2] + row * a.in_rs[2];
  const u32x4* pa = a.in[3] + row * a.in_rs[3];
  u32x4* pdb = a.out[0] + row * a.out_rs[0];
  u32x4* pda = a.out[1] + row * a.out_rs[1];
  u32x4 vg[kPer], vs[kPer], vb[kPer], va[kPer];
  int64_t c[kPer];
  bool ok[kPer];
#pragma unroll
  for (int u = 0; u < kPer; ++u) c[u] = chunk_of<FULL>(a, u, c0, ok[u]);
#pragma unroll
  for (int u = 0; u < kPer; ++u) vg[u] = ld16_stream(pg + c[u]);
#pragma unroll
  for (int u = 0; u < kPer; ++u) vs[u] = ld16_stream(ps + c[u]);
#pragma unroll
  for (int u = 0; u < kPer; ++u) vb[u] = ld16_stream(pb + c[u]);
#pragma unroll
  for (int u = 0; u < kPer; ++u) va[u] = ld16_stream(pa + c[u]);
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    u32x4 db, da;
    bwd8(vg[u], vs[u], vb[u], va[u], db, da);
    if (ok[u]) {
      st16_stream(pdb + c[u], db);
      st16_stream(pda + c[u], da);
    }
  }
}

// Loads of a partial tile are clamped to chunk 0 of the row (always in
// bounds) rather than predicated, so the load batch issues unbranched; only
// the stores are predicated.
__global__ __launch_bounds__(kThreads) void swiglu_fwd_vec(VecArgs a) {
  const int row = (int)blockIdx.x / a.bpr;
  const int64_t c0 = (int64_t)((int)blockIdx.x - row * a.bpr) * kBlockChunks;
  if (c0 + kBlockChunks <= a.cpr) fwd_tile<true>(a, row, c0);
  else fwd_tile<false>(a, row, c0);
}

__global__ __launch_bounds__(kThreads) void swiglu_bwd_vec(VecArgs a) {
  const int row = (int)blockIdx.x / a.bpr;
  const int64_t c0 = (int64_t)((int)blockIdx.x - row * a.bpr) * kBlockChunks;
  if (c0 + kBlockChunks <= a.cpr) bwd_tile<true>(a, row, c0);
  else bwd_tile<false>(a, row, c0);
}

// ------------------------------------------------------------------ scalar path
struct ScalarArgs {
  const uint16_t* in[4];
  uint16_t* out[2];
  int64_t in_rs[4], out_rs[2];  // row strides in elements
  int64_t M, N;
};

__global__ __launch_bounds__(kThreads) void swiglu_fwd_scalar(ScalarArgs a) {
  const int64_t total = a.M * a.N;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total; i += (int64_t)gridDim.x * kThreads) {
    const int64_t r = i / a.N, c = i - r * a.N;
    const float x = bf_to_f(a.in[0][r * a.in_rs[0] + c]);
    const float b = bf_to_f(a.in[1][r * a.in_rs[1] + c]);
    a.out[0][r * a.out_rs[0] + c] = f_to_bf(silu_bf16(x) * b);
  }
}

__global__ __launch_bounds__(kThreads) void swiglu_bwd_scalar(ScalarArgs a) {
  const int64_t total = a.M * a.N;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total; i += (int64_t)gridDim.x * kThreads) {
    const int64_t r = i / a.N, c = i - r * a.N;
    const float g = bf_to_f(a.in[0][r * a.in_rs[0] + c]);
    const float s = bf_to_f(a.in[1][r * a.in_rs[1] + c]);
    const float b = bf_to_f(a.in[2][r * a.in_rs[2] + c]);
    const float x = bf_to_f(a.in[3][r * a.in_rs[3] + c]);
    a.out[0][r * a.out_rs[0] + c] = f_to_bf(g * s);
    a.out[1][r * a.out_rs[1] + c] = f_to_bf(silu_bwd_f(round_bf(g * b), x));
  }
}

// ------------------------------------------------------------------ host side
// Validates and launches one pointwise op over nin inputs / nout outputs of an
// [M, N] bf16 matrix (unit inner stride, row strides in elements).
int launch_pointwise(const char* who, bool backward, const void* const* in, const int64_t* in_rs, int nin,
                     void* const* out, const int64_t* out_rs, int nout, int64_t M, int64_t N, hipStream_t stream) {
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
    launch_dominant_raw(reinterpret_cast<const void*>(backward ? swiglu_bwd_vec : swiglu_fwd_vec),
                        dim3((unsigned)blocks), dim3(kThreads), args, 0, stream);
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
  launch_dominant_raw(reinterpret_cast<const void*>(backward ? swiglu_bwd_scalar : swiglu_fwd_scalar), dim3(blocks),
                      dim3(kThreads), args, 0, stream);
  return check_launch(who);
}

}  // namespace
}  // namespace kp

using namespace kp;

extern "C" {

int kp_swiglu_fwd_bf16(const void* a, int64_t a_rs, const void* b, int64_t b_rs, void* out, int64_t out_rs, int64_t M,
                       int64_t N, void* stream) {
  const void* in[2] = {a, b};
  const int64_t in_rs[2] = {a_rs, b_rs};
  void* outs[1] = {out};
  const int64_t o_rs[1] = {out_rs};
  return launch_pointwise("kp_swiglu_fwd_bf16", false, in, in_rs, 2, outs, o_rs, 1, M, N, as_stream(stream));
}

int kp_swiglu_bwd_bf16(const void* g, int64_t g_rs, const void* s, int64_t s_rs, const void* b, int64_t b_rs,
                       const void* a, int64_t a_rs, void* db, int64_t db_rs, void* da, int64_t da_rs, int64_t M,
                       int64_t N, void* stream) {
  const void* in[4] = {g, s, b, a};
  const int64_t in_rs[4] = {g_rs, s_rs, b_rs, a_rs};
  void* outs[2] = {db, da};
  const int64_t o_rs[2] = {db_rs, da_rs};
  return launch_pointwise("kp_swiglu_bwd_bf16", true, in, in_rs, 4, outs, o_rs, 2, M, N, as_stream(stream));
}

}  // extern "C"
