// Rotary position embedding for gfx950.
//
// One wave64 per (b, s) position handles every head of q and k at that
// position, so the D/2 rotation angles are produced once per position and
// shared by all H_q + H_k heads:
//   - theta mode: lane f computes inv_freq[f] once per kernel (in fp64, rounded
//     to fp32), then per position a = fp32(fp32(p) * inv_freq[f]) and
//     sincosf(a) (full-range OCML reduction, not a fast approximation).  The
//     D/2 (cos, sin) pairs go to a per-wave LDS slot and are read back by the
//     lanes that need them.
//   - table mode: (cos, sin) = freqs_cis[p, i] is read directly (the table row
//     is shared by all heads and stays in L2).
// Work unit = one 16-byte chunk per rotation operand: rotate-half pairs chunk
// [c*8, c*8+8) with [D/2 + c*8, ...); interleaved pairs are the 4 (2i, 2i+1)
// pairs inside one chunk.  Arithmetic is fp32, one RNE rounding to bf16.
#include <math.h>

#include "kp_common.hpp"
#include "kp_internal.hpp"

namespace kp {
namespace {

constexpr int kThreads = 256;
constexpr int kWavesPerBlock = kThreads / 64;
constexpr int kMaxHalf = 256;  // D <= 512

struct RopeTensor {
  const uint16_t* x;
  void* out;  // bf16, or fp32 when out_f32
  int out_f32;
  int64_t H;
  int64_t xs[3];  // b, s, h strides (elements)
  int64_t os[3];
};

struct RopeArgs {
  RopeTensor t[2];
  int nt;
  int64_t B, S, D;
  const void* pos;
  int pb;
  int64_t psb, pss;
  int pairing;
  double theta;
  const float* freqs;  // complex64 table as float pairs
  int64_t frows, frs;  // rows, row stride in complex elements
  int conj;
  int32_t* err;
};

// Output element offset o of tensor T gets 8 (16-byte bf16 / 32-byte fp32) or 1 value.
__device__ __forceinline__ void store8(const RopeTensor& T, int64_t o, const float* v) {
  if (T.out_f32) {
    float* p = static_cast<float*>(T.out) + o;
    *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4*>(p + 4) = f32x4{v[4], v[5], v[6], v[7]};
  } else {
    st16(static_cast<uint16_t*>(T.out) + o, pack8(v));
  }
}
__device__ __forceinline__ void store1(const RopeTensor& T, int64_t o, float v) {
  if (T.out_f32) static_cast<float*>(T.out)[o] = v;
  else static_cast<uint16_t*>(T.out)[o] = f_to_bf(v);
}

__device__ __forceinline__ void rot(float a, float b, float c, float s, float& oa, float& ob) {
  oa = a * c - b * s;
  ob = b * c + a * s;
}

// TABLE is a template parameter so that each instantiation reads its angles
// from exactly one address space (global table or LDS slot); a runtime choice
// lets the compiler merge both into one flat load.
template <bool VEC, bool TABLE>
__global__ __launch_bounds__(kThreads) void rope_kernel(RopeArgs a) {
  __shared__ float cs[kWavesPerBlock][2][kMaxHalf];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t half = a.D / 2;
  constexpr bool table = TABLE;

  // inv_freq[f] for f = lane + 64k (theta mode), kept in registers.
  float inv[kMaxHalf / 64];
#pragma unroll
  for (int k = 0; k < kMaxHalf / 64; ++k) {
    const int f = lane + 64 * k;
    inv[k] = (!table && f < half) ? (float)pow(a.theta, -(double)(2 * f) / (double)a.D) : 0.f;
  }

  const int64_t npos = a.B * a.S;
  const int64_t w0 = (int64_t)blockIdx.x * kWavesPerBlock + wave;
  const int64_t nw = (int64_t)gridDim.x * kWavesPerBlock;
  const float sgn = a.conj ? -1.f : 1.f;
  // The (cos, sin) slot is indexed through the __shared__ array itself (never
  // through a generic pointer) so reads stay ds_read; the workgroup-scope
  // fences around the wave barrier make the other lanes' ds_writes visible.
#define COSV(f) cs[wave][0][f]
#define SINV(f) cs[wave][1][f]

  for (int64_t ps = w0; ps < npos; ps += nw) {
    const int64_t b = ps / a.S, s = ps % a.S;
    int64_t p = s;
    if (a.pos) p = a.pb == 8 ? static_cast<const int64_t*>(a.pos)[b * a.psb + s * a.pss]
                             : (int64_t) static_cast<const int32_t*>(a.pos)[b * a.psb + s * a.pss];
    bool ok = true;
    const float* frow = nullptr;
    if constexpr (TABLE) {
      ok = p >= 0 && p < a.frows;
      if (!ok && lane == 0 && a.err) *a.err = 1;
      frow = a.freqs + 2 * (ok ? p : 0) * a.frs;
    } else {
      const float pf = (float)p;
#pragma unroll
      for (int k = 0; k < kMaxHalf / 64; ++k) {
        const int f = lane + 64 * k;
        if (f < half) {
          float sn, c;
          sincosf(pf * inv[k], &sn, &c);
          COSV(f) = c;
          SINV(f) = sn;
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    }

    for (int ti = 0; ti < a.nt; ++ti) {
      const RopeTensor& T = a.t[ti];
      const uint16_t* xb = T.x + b * T.xs[0] + s * T.xs[1];
      const int64_t ob = b * T.os[0] + s * T.os[1];  // output element offset of this position
      if constexpr (VEC) {
        if (a.pairing == KP_ROPE_HALF) {
          const int64_t nch = half / 8;  // chunks per half
          for (int64_t u = lane; u < T.H * nch; u += 64) {
            const int64_t h = u / nch, c = u % nch;
            const uint16_t* xp = xb + h * T.xs[2] + c * 8;
            const int64_t oo = ob + h * T.os[2] + c * 8;
            float x1[8], x2[8], o1[8], o2[8];
            unpack8(ld16_stream(xp), x1);
            unpack8(ld16_stream(xp + half), x2);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const int64_t f = c * 8 + e;
              float cv, sv;
              if constexpr (TABLE) {
                cv = frow[2 * f];
                sv = frow[2 * f + 1];
              } else {
                cv = COSV(f);
                sv = SINV(f);
              }
              rot(x1[e], x2[e], cv, sgn * sv, o1[e], o2[e]);
              if (!ok) o1[e] = o2[e] = 0.f;
            }
            store8(T, oo, o1);
            store8(T, oo + half, o2);
          }
        } else {
          const int64_t nch = a.D / 8;  // chunks per head, 4 pairs each
          for (int64_t u = lane; u < T.H * nch; u += 64) {
            const int64_t h = u / nch, c = u % nch;
            const uint16_t* xp = xb + h * T.xs[2] + c * 8;
            const int64_t oo = ob + h * T.os[2] + c * 8;
            float xv[8], o[8];
            unpack8(ld16_stream(xp), xv);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int64_t f = c * 4 + q;
              float cv, sv;
              if constexpr (TABLE) {
                cv = frow[2 * f];
                sv = frow[2 * f + 1];
              } else {
                cv = COSV(f);
                sv = SINV(f);
              }
              rot(xv[2 * q], xv[2 * q + 1], cv, sgn * sv, o[2 * q], o[2 * q + 1]);
              if (!ok) o[2 * q] = o[2 * q + 1] = 0.f;
            }
            store8(T, oo, o);
          }
        }
      } else {
        // Scalar path: any alignment / stride, one rotation pair per step.
        for (int64_t u = lane; u < T.H * half; u += 64) {
          const int64_t h = u / half, f = u % half;
          const int64_t ia = a.pairing == KP_ROPE_HALF ? f : 2 * f;
          const int64_t ib = a.pairing == KP_ROPE_HALF ? f + half : 2 * f + 1;
          const uint16_t* xp = xb + h * T.xs[2];
          const int64_t oo = ob + h * T.os[2];
          float cv, sv;
          if constexpr (TABLE) {
            cv = frow[2 * f];
            sv = frow[2 * f + 1];
          } else {
            cv = COSV(f);
            sv = SINV(f);
          }
          float oa, obv;
          rot(bf_to_f(xp[ia]), bf_to_f(xp[ib]), cv, sgn * sv, oa, obv);
          if (!ok) oa = obv = 0.f;
          store1(T, oo + ia, oa);
          store1(T, oo + ib, obv);
        }
      }
    }
    if constexpr (!TABLE) {
      // the next position rewrites this wave's LDS slot
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    }
  }
}

#undef COSV
#undef SINV

bool tensor_vec_ok(const RopeTensor& t, int64_t D, int pairing) {
  if (!aligned16(t.x) || !aligned16(t.out)) return false;
  for (int i = 0; i < 3; ++i)
    if ((t.xs[i] & 7) != 0 || (t.os[i] & 7) != 0) return false;
  return pairing == KP_ROPE_HALF ? (D % 16) == 0 : (D % 8) == 0;
}

}  // namespace
}  // namespace kp

using namespace kp;

extern "C" {

int kp_rope_bf16(const void* x0, void* out0, int64_t H0, const int64_t* x0_strides, const int64_t* out0_strides,
                 const void* x1, void* out1, int64_t H1, const int64_t* x1_strides, const int64_t* out1_strides,
                 int64_t B, int64_t S, int64_t D, const void* positions, int pos_bytes, int64_t pos_stride_b,
                 int64_t pos_stride_s, int pairing, double theta, const float* freqs_cis, int64_t freq_rows,
                 int64_t freq_row_stride, int conj, int out_f32_mask, int32_t* error_flag, void* stream) {
  static const char* who = "kp_rope_bf16";
  if (x0 == nullptr || out0 == nullptr || x0_strides == nullptr || out0_strides == nullptr)
    return fail(KP_EINVAL, "%s: tensor 0 needs x, out and strides", who);
  if (x1 != nullptr && (out1 == nullptr || x1_strides == nullptr || out1_strides == nullptr))
    return fail(KP_EINVAL, "%s: tensor 1 needs out and strides", who);
  if (B < 0 || S < 0 || H0 < 0 || (x1 && H1 < 0)) return fail(KP_EINVAL, "%s: negative size", who);
  if (D <= 0 || (D & 1) || D / 2 > kMaxHalf) return fail(KP_EINVAL, "%s: D must be even and <= %d", who, 2 * kMaxHalf);
  if (pairing != KP_ROPE_HALF && pairing != KP_ROPE_INTERLEAVED) return fail(KP_EINVAL, "%s: bad pairing", who);
  if (positions != nullptr && pos_bytes != 4 && pos_bytes != 8)
    return fail(KP_EINVAL, "%s: pos_bytes must be 4 or 8", who);
  if (freqs_cis == nullptr && !(theta > 0.0)) return fail(KP_EINVAL, "%s: theta must be > 0", who);
  if (freqs_cis != nullptr && (freq_rows <= 0 || freq_row_stride < D / 2))
    return fail(KP_EINVAL, "%s: freqs_cis needs rows > 0 and row stride >= D/2", who);

  RopeArgs a{};
  a.t[0] = RopeTensor{static_cast<const uint16_t*>(x0), out0, out_f32_mask & 1, H0,
                      {x0_strides[0], x0_strides[1], x0_strides[2]},
                      {out0_strides[0], out0_strides[1], out0_strides[2]}};
  a.nt = 1;
  if (x1 != nullptr) {
    a.t[1] = RopeTensor{static_cast<const uint16_t*>(x1), out1, (out_f32_mask >> 1) & 1, H1,
                        {x1_strides[0], x1_strides[1], x1_strides[2]},
                        {out1_strides[0], out1_strides[1], out1_strides[2]}};
    a.nt = 2;
  }
  a.B = B;
  a.S = S;
  a.D = D;
  a.pos = positions;
  a.pb = pos_bytes;
  a.psb = pos_stride_b;
  a.pss = pos_stride_s;
  a.pairing = pairing;
  a.theta = theta;
  a.freqs = freqs_cis;
  a.frows = freq_rows;
  a.frs = freq_row_stride;
  a.conj = conj ? 1 : 0;
  a.err = error_flag;
  const int64_t npos = B * S;
  if (npos == 0) return KP_OK;

  bool vec = tensor_vec_ok(a.t[0], D, pairing) && (a.nt == 1 || tensor_vec_ok(a.t[1], D, pairing));
  const int64_t blocks_needed = ceil_div(npos, kWavesPerBlock);
  const int64_t cap = (int64_t)cu_count() * 16;
  const int grid = (int)(blocks_needed < cap ? blocks_needed : cap);
  hipStream_t s = as_stream(stream);
  const bool tab = freqs_cis != nullptr;
  if (vec && tab) KP_LAUNCH_DOMINANT((rope_kernel<true, true>), dim3(grid), dim3(kThreads), 0, s, a);
  else if (vec) KP_LAUNCH_DOMINANT((rope_kernel<true, false>), dim3(grid), dim3(kThreads), 0, s, a);
  else if (tab) KP_LAUNCH_DOMINANT((rope_kernel<false, true>), dim3(grid), dim3(kThreads), 0, s, a);
  else KP_LAUNCH_DOMINANT((rope_kernel<false, false>), dim3(grid), dim3(kThreads), 0, s, a);
  return check_launch(who);
}

}  // extern "C"
