// Rotary position embedding on complex64 data for gfx950: q and k already
// viewed as complex (fp32 (re, im) pairs) multiplied by a complex64 table row
// per position, complex64 out -- the index -> mul regions of the first
// training-graph captures, where the bf16 -> fp32 -> view_as_complex
// conversion sits outside the fragment.
//
//   out[b, s, h, i] = x[b, s, h, i] * t[p, i]     (or * conj(t[p, i]))
//   (a + bi)(c + di) = (ac - bd) + (ad + bc)i in fp32, torch's complex product,
//   p = positions[b, s] (or s), t = the [rows, P] table.
//
// One wave per (b, s) position.  A 16-byte chunk holds two complex values; a
// head of P = 64 pairs is 32 chunks, so lane l always holds chunk l % 32 of a
// head and loads its two table entries once per position.  Chunks are taken
// kBatch at a time with every load of a batch issued before the arithmetic,
// non-temporal loads and stores.  Views that are not 16-byte granular take
// the 8-byte (one complex value) path with the same arithmetic.
#include "kp_common.hpp"
#include "kp_internal.hpp"

namespace kp {
namespace {

constexpr int kThreads = 256;
constexpr int kWavesPerBlock = kThreads / kWave;
constexpr int kBatch = 8;  // chunks per lane in flight

struct C64Tensor {
  const float* x;  // complex64 as float pairs
  float* out;
  int64_t H;
  int64_t xs[3];  // b, s, h strides in complex elements
  int64_t os[3];
};

struct C64Args {
  C64Tensor t[2];
  int nt;
  int64_t B, S, P;  // P complex pairs per head
  const void* pos;
  int pb;
  int64_t psb, pss;
  const float* freqs;  // [rows, P] complex64 as float pairs
  int64_t frows, frs;  // rows, row stride in complex elements
  float sgn;           // -1 for the conjugate table
  int32_t* err;
};

// (a + bi)(c + di) in fp32 with the contraction spelled out (one rounded
// product, then one fma per component), so the tile and per-position kernels
// give the same bits whatever the compiler would fuse in each.
__device__ __forceinline__ void cmul(float a, float b, float c, float d, float& re, float& im) {
  re = __builtin_fmaf(a, c, -(b * d));
  im = __builtin_fmaf(a, d, b * c);
}

template <bool VEC>
__global__ __launch_bounds__(kThreads) void rope_c64_kernel(C64Args a) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t npos = a.B * a.S;
  const int64_t w0 = (int64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  const int64_t nw = (int64_t)gridDim.x * kWavesPerBlock;
  constexpr int kPer = VEC ? 2 : 1;  // complex values per unit
  const int64_t upr = a.P / kPer;    // units per head
  for (int64_t ps = w0; ps < npos; ps += nw) {
    const int64_t b = ps / a.S, s = ps - b * a.S;
    int64_t p = s;
    if (a.pos) p = a.pb == 8 ? static_cast<const int64_t*>(a.pos)[b * a.psb + s * a.pss]
                             : (int64_t) static_cast<const int32_t*>(a.pos)[b * a.psb + s * a.pss];
    const bool ok = p >= 0 && p < a.frows;
    if (!ok && lane == 0 && a.err) a.err[0] = 1;
    const float* frow = a.freqs + 2 * (ok ? p : 0) * a.frs;
    for (int ti = 0; ti < a.nt; ++ti) {
      const C64Tensor& T = a.t[ti];
      const float* xb = T.x + 2 * (b * T.xs[0] + s * T.xs[1]);
      float* ob = T.out + 2 * (b * T.os[0] + s * T.os[1]);
      const int64_t units = T.H * upr;
      for (int64_t u0 = lane; u0 < units; u0 += (int64_t)kWave * kBatch) {
        if constexpr (VEC) {
          f32x4 v[kBatch], tv[kBatch];
          int64_t h[kBatch], c[kBatch];
#pragma unroll
          for (int k = 0; k < kBatch; ++k) {
            const int64_t u = u0 + (int64_t)k * kWave;
            const int64_t uu = u < units ? u : u0;  // past the end: re-read this lane's first unit
            h[k] = uu / upr;
            c[k] = uu - h[k] * upr;
            v[k] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(xb + 2 * (h[k] * T.xs[2] + 2 * c[k])));
            tv[k] = *reinterpret_cast<const f32x4*>(frow + 4 * c[k]);  // the table row: cached, 16 B per chunk
          }
#pragma unroll
          for (int k = 0; k < kBatch; ++k) {
            if (u0 + (int64_t)k * kWave >= units) break;
            const f32x4 t = tv[k];
            float o[4];
            cmul(v[k][0], v[k][1], t[0], a.sgn * t[1], o[0], o[1]);
            cmul(v[k][2], v[k][3], t[2], a.sgn * t[3], o[2], o[3]);
            const f32x4 r = ok ? f32x4{o[0], o[1], o[2], o[3]} : f32x4{0.f, 0.f, 0.f, 0.f};
            st16f_stream(ob + 2 * (h[k] * T.os[2] + 2 * c[k]), r);
          }
        } else {
#pragma unroll
          for (int k = 0; k < kBatch; ++k) {
            const int64_t u = u0 + (int64_t)k * kWave;
            if (u >= units) break;
            const int64_t hh = u / upr, cc = u - hh * upr;
            const float* xp = xb + 2 * (hh * T.xs[2] + cc);
            float re, im;
            cmul(xp[0], xp[1], frow[2 * cc], a.sgn * frow[2 * cc + 1], re, im);
            if (!ok) re = im = 0.f;
            float* op = ob + 2 * (hh * T.os[2] + cc);
            op[0] = re;
            op[1] = im;
          }
        }
      }
    }
  }
}

// Tile path: every tensor stored [B, S, H, P] contiguously in and out with
// H * P / 2 a multiple of 64 (the v1 captures: P = 64, H = 32 and 8).  A
// block owns 512 consecutive 16-byte chunks of one tensor (thread t: chunks
// t and t + 256, tensor 0's blocks first) -- the streaming probe's layout,
// short-lived blocks instead of one wave walking a position's 10 KiB -- and a
// wave's 64 chunks (a group) always lie in one position, whose id and table
// row are then wave-uniform: wave w takes groups 8 tile + w and 8 tile + w + 4.
// Indices are 32-bit (each tensor below 2^31 chunks, checked on the host);
// the group's position and a chunk's place in its head are multiply-high
// divisions by launch-fixed divisors.  Same arithmetic as rope_c64_kernel,
// hence the same bits.
constexpr int kTileChunks = 2 * kThreads;
constexpr int kTileGroups = kTileChunks / kWave;  // 8

struct C64TileTensor {
  const float* x;
  float* out;
  uint32_t groups;  // B * S * H * P / 128
  Div32 gpp;        // groups per position, H * P / 128
};
struct C64TileArgs {
  C64TileTensor t[2];
  uint32_t nb0;  // blocks of tensor 0
  Div32 S;
  Div32 cph;     // chunks per head, P / 2
  const void* pos;
  int pb;
  int64_t psb, pss;
  const float* freqs;
  int64_t frows, frs;
  float sgn;
  int32_t* err;
};

__global__ __launch_bounds__(kThreads) void rope_c64_tile(C64TileArgs a) {
  const int lane = threadIdx.x & (kWave - 1);
  const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const bool second = blockIdx.x >= a.nb0;
  const C64TileTensor& T = a.t[second ? 1 : 0];
  const uint32_t g0 = (second ? blockIdx.x - a.nb0 : blockIdx.x) * kTileGroups;
  const uint32_t glast = T.groups - 1;
  // groups past the tensor's end (last tile only) re-read the last group and store nothing
  f32x4 v[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const uint32_t g = g0 + wave + 4 * u;
    v[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(T.x) + (size_t)(g < glast ? g : glast) * kWave + lane);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const uint32_t g = g0 + wave + 4 * u, gc = g < glast ? g : glast;
    const uint32_t ps = div32(gc, T.gpp);
    const uint32_t b = div32(ps, a.S), s = ps - b * a.S.d;
    int64_t p = s;
    if (a.pos) {
      const int64_t i = (int64_t)b * a.psb + (int64_t)s * a.pss;
      p = a.pb == 8 ? static_cast<const int64_t*>(a.pos)[i] : (int64_t) static_cast<const int32_t*>(a.pos)[i];
    }
    const bool ok = p >= 0 && p < a.frows;
    if (!ok && lane == 0 && a.err) a.err[0] = 1;
    const uint32_t x = (gc - ps * T.gpp.d) * kWave + lane;  // chunk within its position
    const uint32_t c = x - div32(x, a.cph) * a.cph.d;       // chunk within its head
    const f32x4 t = *reinterpret_cast<const f32x4*>(a.freqs + 2 * (ok ? p : 0) * a.frs + 4 * c);
    float o[4];
    cmul(v[u][0], v[u][1], t[0], a.sgn * t[1], o[0], o[1]);
    cmul(v[u][2], v[u][3], t[2], a.sgn * t[3], o[2], o[3]);
    const f32x4 r = ok ? f32x4{o[0], o[1], o[2], o[3]} : f32x4{0.f, 0.f, 0.f, 0.f};
    if (g <= glast) st16f_stream(reinterpret_cast<f32x4*>(T.out) + (size_t)g * kWave + lane, r);
  }
}

bool tile_view(const C64Tensor& t, int64_t S, int64_t P) {
  const int64_t hp = t.H * P;
  return t.H > 0 && (hp / 2) % kWave == 0 && t.xs[2] == P && t.xs[1] == hp && t.xs[0] == S * hp && t.os[2] == P &&
         t.os[1] == hp && t.os[0] == S * hp;
}

bool aligned_view(const void* p, const int64_t* st, int64_t P) {
  // 16-byte chunks: base aligned, every stride and P a whole number of 2 complex values
  return aligned16(p) && (P % 2 == 0) && st[0] % 2 == 0 && st[1] % 2 == 0 && st[2] % 2 == 0;
}

}  // namespace
}  // namespace kp

using namespace kp;

extern "C" {

int kp_rope_c64(const void* x0, void* out0, int64_t H0, const int64_t* x0_strides, const int64_t* out0_strides,
                const void* x1, void* out1, int64_t H1, const int64_t* x1_strides, const int64_t* out1_strides,
                int64_t B, int64_t S, int64_t P, const void* positions, int pos_bytes, int64_t pos_stride_b,
                int64_t pos_stride_s, const float* freqs_cis, int64_t freq_rows, int64_t freq_row_stride, int conj,
                int32_t* error_flag, void* stream) {
  static const char* who = "kp_rope_c64";
  if (x0 == nullptr || out0 == nullptr || x0_strides == nullptr || out0_strides == nullptr)
    return fail(KP_EINVAL, "%s: tensor 0 needs x, out and strides", who);
  if (x1 != nullptr && (out1 == nullptr || x1_strides == nullptr || out1_strides == nullptr))
    return fail(KP_EINVAL, "%s: tensor 1 needs out and strides", who);
  if (B < 0 || S < 0 || H0 < 0 || (x1 && H1 < 0) || P <= 0) return fail(KP_EINVAL, "%s: bad size", who);
  if (positions != nullptr && pos_bytes != 4 && pos_bytes != 8)
    return fail(KP_EINVAL, "%s: pos_bytes must be 4 or 8", who);
  if (freqs_cis == nullptr || freq_rows <= 0 || freq_row_stride < P)
    return fail(KP_EINVAL, "%s: freqs_cis needs rows > 0 and row stride >= P", who);
  C64Args a{};
  a.t[0] = C64Tensor{static_cast<const float*>(x0), static_cast<float*>(out0), H0,
                     {x0_strides[0], x0_strides[1], x0_strides[2]},
                     {out0_strides[0], out0_strides[1], out0_strides[2]}};
  a.nt = 1;
  if (x1 != nullptr) {
    a.t[1] = C64Tensor{static_cast<const float*>(x1), static_cast<float*>(out1), H1,
                       {x1_strides[0], x1_strides[1], x1_strides[2]},
                       {out1_strides[0], out1_strides[1], out1_strides[2]}};
    a.nt = 2;
  }
  a.B = B;
  a.S = S;
  a.P = P;
  a.pos = positions;
  a.pb = pos_bytes;
  a.psb = pos_stride_b;
  a.pss = pos_stride_s;
  a.freqs = freqs_cis;
  a.frows = freq_rows;
  a.frs = freq_row_stride;
  a.sgn = conj ? -1.0f : 1.0f;
  a.err = error_flag;
  const int64_t npos = B * S;
  if (npos == 0) return KP_OK;
  const int64_t fst[3] = {freq_row_stride, 0, 0};
  bool vec = aligned_view(freqs_cis, fst, P);
  for (int i = 0; i < a.nt; ++i)
    vec = vec && aligned_view(a.t[i].x, a.t[i].xs, P) && aligned_view(a.t[i].out, a.t[i].os, P);
  bool tile = vec;
  for (int i = 0; i < a.nt; ++i) tile = tile && tile_view(a.t[i], S, P);
  if (tile && npos <= INT32_MAX) {
    C64TileArgs ta{};
    bool fits = true;
    for (int i = 0; i < a.nt; ++i) {
      const int64_t gpp = a.t[i].H * P / (2 * kWave);
      fits = fits && gpp <= INT32_MAX / kWave && npos * gpp * kWave <= INT32_MAX;  // 32-bit chunk indices
      if (fits) ta.t[i] = C64TileTensor{a.t[i].x, a.t[i].out, (uint32_t)(npos * gpp), make_div32((uint32_t)gpp)};
    }
    if (fits) {
      ta.nb0 = (uint32_t)ceil_div(ta.t[0].groups, kTileGroups);
      const int64_t nb1 = a.nt > 1 ? ceil_div(ta.t[1].groups, kTileGroups) : 0;
      ta.S = make_div32((uint32_t)S);
      ta.cph = make_div32((uint32_t)(P / 2));
      ta.pos = a.pos;
      ta.pb = a.pb;
      ta.psb = a.psb;
      ta.pss = a.pss;
      ta.freqs = a.freqs;
      ta.frows = a.frows;
      ta.frs = a.frs;
      ta.sgn = a.sgn;
      ta.err = a.err;
      void* targs[] = {&ta};
      launch_dominant_raw(reinterpret_cast<const void*>(rope_c64_tile), dim3((unsigned)(ta.nb0 + nb1)), dim3(kThreads),
                          targs, 0, as_stream(stream));
      return check_launch(who);
    }
  }
  const int64_t blocks_needed = ceil_div(npos, kWavesPerBlock);
  const int64_t cap = (int64_t)cu_count() * 16;
  const unsigned grid = (unsigned)(blocks_needed < cap ? blocks_needed : cap);
  void* args[] = {&a};
  launch_dominant_raw(vec ? reinterpret_cast<const void*>(rope_c64_kernel<true>)
                          : reinterpret_cast<const void*>(rope_c64_kernel<false>),
                      dim3(grid), dim3(kThreads), args, 0, as_stream(stream));
  return check_launch(who);
}

}  // extern "C"
