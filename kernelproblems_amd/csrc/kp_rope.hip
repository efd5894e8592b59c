// Rotary position embedding for gfx950.
//
// One wave64 per (b, s) position handles every head of q and k at that
// position, so the D/2 rotation angles are produced once per position and
// shared by all H_q + H_k heads:
//   - theta mode: inv_freq[f] = fp32(theta^(-2f/D)) (fp64 pow; for D = 128
//     evaluated once per call on the host and passed in the kernel
//     arguments, else by lane f in every wave), then per position
//     a = fp32(fp32(p) * inv_freq[f]) and
//     sincosf(a) (full-range OCML reduction, not a fast approximation).  The
//     D/2 (cos, sin) pairs go to a per-wave LDS slot and are read back by the
//     lanes that need them.
//   - table mode: (cos, sin) = freqs_cis[p, i] is read directly (the table row
//     is shared by all heads and stays in L2).
// Work unit = one 16-byte chunk per rotation operand: rotate-half pairs chunk
// [c*8, c*8+8) with [D/2 + c*8, ...); interleaved pairs are the 4 (2i, 2i+1)
// pairs inside one chunk.  Arithmetic is fp32, one RNE rounding to bf16.
#include <math.h>
#include <stdlib.h>

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
  // theta mode with D = 128: inv_freq[f] = fp32(theta^(-2f/D)), evaluated
  // once per call on the host (have_inv = 1) instead of in every wave (both
  // kernels then read it, so their angles stay identical)
  int have_inv;
  float inv_freq[64];
};

// Output element offset o gets 8 values (16-byte bf16 / 32-byte fp32) or 1 value.
__device__ __forceinline__ void store8p(void* out, int out_f32, int64_t o, const float* v) {
  if (out_f32) {
    st32f(static_cast<float*>(out) + o, v);
  } else {
    st16_stream(static_cast<uint16_t*>(out) + o, pack8(v));
  }
}
__device__ __forceinline__ void store8(const RopeTensor& T, int64_t o, const float* v) { store8p(T.out, T.out_f32, o, v); }
__device__ __forceinline__ void store1(const RopeTensor& T, int64_t o, float v) {
  if (T.out_f32) static_cast<float*>(T.out)[o] = v;
  else static_cast<uint16_t*>(T.out)[o] = f_to_bf(v);
}

// (a, b) rotated by the angle with cosine c and sine s.  The contraction is
// spelled out -- one rounded product, then one fma -- so that every kernel of
// this file (compiled separately, each free to contract a * c - b * s its
// own way) produces the same bits for the same operands.
__device__ __forceinline__ void rot(float a, float b, float c, float s, float& oa, float& ob) {
  oa = __builtin_fmaf(a, c, -(b * s));
  ob = __builtin_fmaf(b, c, a * s);
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
    inv[k] = (!table && f < half)
                 ? (a.have_inv ? a.inv_freq[f & 63] : (float)pow(a.theta, -(double)(2 * f) / (double)a.D))
                 : 0.f;
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

// ------------------------------------------------------------ fast path
// D = 128 with 16-byte aligned rows (every reference fragment and the
// rotate-half configuration): one wave per (b, s) position, and every 16-byte
// chunk of the position's q and k heads is requested before any arithmetic,
// so a wave has up to 16 loads (16 KiB) in flight.  Work unit u of a position
// is (tensor, head, chunk c), q units first; lane l holds units l, l + 64, ...
// Rotate-half: a unit is the chunk pair (c, c + 8) of one head (8 units per
// head, two loads); interleaved: a unit is one chunk of 4 (2i, 2i+1) pairs (16
// units per head, one load).  64 is a multiple of the units per head and q has
// a whole number of heads, so lane l always holds chunk c = l % (units per
// head) and its 8 (or 4) rotation angles serve every unit it holds.  Units
// past the end re-read the last unit (same lines, no predicated loads: see
// the row kernels of kp_rmsnorm.hip) and store nothing.  Arithmetic, rounding
// and angles are those of rope_kernel, so both paths give identical bits.
constexpr int kFastD = 128;
constexpr int kFastMaxLoads = 16;

template <int PAIRING, bool TABLE, int UPL>
__device__ __forceinline__ void rope_fast_body(const RopeArgs& a) {
  constexpr bool kHalf = PAIRING == KP_ROPE_HALF;
  constexpr int HD = kFastD / 2;
  constexpr int CPH = kHalf ? kFastD / 16 : kFastD / 8;  // units per head
  constexpr int FPU = kHalf ? 8 : 4;                     // angles per unit
  __shared__ float cs[kWavesPerBlock][2][HD];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t ps = (int64_t)blockIdx.x * kWavesPerBlock + wave;
  if (ps >= a.B * a.S) return;  // wave-uniform; only wave barriers follow
  const int64_t b = ps / a.S, s = ps - b * a.S;

  const RopeTensor& T0 = a.t[0];
  const RopeTensor& T1 = a.t[a.nt > 1 ? 1 : 0];
  const int U0 = (int)T0.H * CPH;
  const int U = U0 + (a.nt > 1 ? (int)T1.H * CPH : 0);
  const uint16_t* xb0 = T0.x + b * T0.xs[0] + s * T0.xs[1];
  const uint16_t* xb1 = T1.x + b * T1.xs[0] + s * T1.xs[1];

  u32x4 v1[UPL], v2[UPL];
#pragma unroll
  for (int j = 0; j < UPL; ++j) {
    int u = lane + 64 * j;
    u = u < U ? u : U - 1;
    const bool second = u >= U0;
    const int ul = second ? u - U0 : u;
    const int h = ul / CPH, c = ul % CPH;
    const uint16_t* xp = (second ? xb1 + h * T1.xs[2] : xb0 + h * T0.xs[2]) + c * 8;
    v1[j] = ld16_stream(xp);
    if constexpr (kHalf) v2[j] = ld16_stream(xp + HD);
  }
  __builtin_amdgcn_sched_barrier(0);

  int64_t p = s;
  if (a.pos) p = a.pb == 8 ? static_cast<const int64_t*>(a.pos)[b * a.psb + s * a.pss]
                           : (int64_t) static_cast<const int32_t*>(a.pos)[b * a.psb + s * a.pss];
  const int cl = lane % CPH;
  float cv[FPU], sv[FPU];
  bool ok = true;
  if constexpr (TABLE) {
    ok = p >= 0 && p < a.frows;
    if (!ok && lane == 0 && a.err) *a.err = 1;
    const float* frow = a.freqs + 2 * ((ok ? p : 0) * a.frs + cl * FPU);
#pragma unroll
    for (int q = 0; q < FPU / 2; ++q) {
      const f32x4 t = *reinterpret_cast<const f32x4*>(frow + 4 * q);
      cv[2 * q] = t[0];
      sv[2 * q] = t[1];
      cv[2 * q + 1] = t[2];
      sv[2 * q + 1] = t[3];
    }
  } else {
    // lane f < D/2 produces angle f: fp32(fp32(p) * fp32(theta^(-2f/D)))
    const float inv = a.have_inv ? a.inv_freq[lane] : (float)pow(a.theta, -(double)(2 * lane) / (double)kFastD);
    float sn, cn;
    sincosf((float)p * inv, &sn, &cn);
    cs[wave][0][lane] = cn;
    cs[wave][1][lane] = sn;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
#pragma unroll
    for (int e = 0; e < FPU; ++e) {
      cv[e] = cs[wave][0][cl * FPU + e];
      sv[e] = cs[wave][1][cl * FPU + e];
    }
  }
  const float sgn = a.conj ? -1.f : 1.f;
#pragma unroll
  for (int e = 0; e < FPU; ++e) sv[e] = sgn * sv[e];

  // Per-tensor output fields as wave-uniform scalars: selected per lane from
  // kernel-argument memory they become per-unit vector loads, and their waits
  // (vmcnt counts stores too) would serialize the stores.
  const int64_t ob0 = uniform64(b * T0.os[0] + s * T0.os[1]);
  const int64_t ob1 = uniform64(b * T1.os[0] + s * T1.os[1]);
  const int64_t hs0 = uniform64(T0.os[2]), hs1 = uniform64(T1.os[2]);
  // tensor 1's output as a byte offset from tensor 0's (a select of pointers
  // loses the global address space and turns the stores into flat stores)
  char* const out0 = static_cast<char*>(T0.out);
  const int64_t dout = uniform64(static_cast<char*>(T1.out) - out0);
  const int f0 = __builtin_amdgcn_readfirstlane(T0.out_f32), f1 = __builtin_amdgcn_readfirstlane(T1.out_f32);
#pragma unroll
  for (int j = 0; j < UPL; ++j) {
    const int u = lane + 64 * j;
    if (u < U) {
      const bool second = u >= U0;
      const int ul = second ? u - U0 : u;
      const int h = ul / CPH;
      void* out = out0 + (second ? dout : 0);
      const int f32 = second ? f1 : f0;
      const int64_t oo = (second ? ob1 + h * hs1 : ob0 + h * hs0) + cl * 8;
      float x1[8], o1[8];
      unpack8(v1[j], x1);
      if constexpr (kHalf) {
        float x2[8], o2[8];
        unpack8(v2[j], x2);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          rot(x1[e], x2[e], cv[e], sv[e], o1[e], o2[e]);
          if (!ok) o1[e] = o2[e] = 0.f;
        }
        store8p(out, f32, oo, o1);
        store8p(out, f32, oo + HD, o2);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          rot(x1[2 * q], x1[2 * q + 1], cv[q], sv[q], o1[2 * q], o1[2 * q + 1]);
          if (!ok) o1[2 * q] = o1[2 * q + 1] = 0.f;
        }
        store8p(out, f32, oo, o1);
      }
    }
  }
}

template <int PAIRING, bool TABLE, int UPL>
__global__ __launch_bounds__(kThreads) void rope_fast(RopeArgs a) {
  rope_fast_body<PAIRING, TABLE, UPL>(a);
}

// ------------------------------------------------------------ tile path
// D = 128, every tensor stored [B, S, H, 128] contiguously in and out (the
// forward fragments and the rotate-half configuration), H a multiple of 4,
// bf16 or fp32 outputs.  Unlike rope_fast (one wave per position, up to 16 KiB per
// wave), a block owns 512 consecutive 16-byte chunks of one tensor -- thread
// t chunks t and t + 256, tensor 0's blocks first -- the short-lived,
// fine-grained streaming layout that measured fastest on MI355X (c4: 56 us
// against 58.5 us for rope_fast, bit-identical).  A head is 16 chunks, so a
// lane's chunk index c = lane % 16 is fixed; a wave's 64 chunks are a group
// of 4 heads of one position (H % 4 == 0), so a block is 8 groups and wave w
// takes groups 8 tile + w and 8 tile + w + 4.  Every index is 32-bit (the
// host keeps each tensor below 2^31 chunks) and wave-uniform, the group's
// position being a multiply-high division by the groups per position, so
// the per-chunk work is the rotation alone.  Rotate-half pairs chunk c with
// c ^ 8, i.e. lane l with lane l ^ 8 of the same 16-lane DPP row
// (row_ror:8); interleaved pairs are the 4 (2i, 2i+1) pairs inside a chunk.
// Theta mode evaluates the (cos, sin) of the tile's (at most 8) positions
// once per block (threads f, f + 64, ... of position slot i / 64) into LDS
// behind one barrier; rotate-half table mode copies the positions' table
// rows there the same way; interleaved table mode reads the position's row
// (L2-resident) per chunk.  Arithmetic, rounding and angles are those of
// rope_fast, so both give identical bits.
constexpr int kTileChunks = 2 * kThreads;
constexpr int kTileGroups = kTileChunks / 64;  // 8
constexpr int kTileMaxPos = kTileGroups;       // a position is >= 1 group

struct TileTensor {
  const uint16_t* x;
  void* out;        // bf16, or fp32 when out_f32
  uint32_t groups;  // B * S * H / 4
  Div32 gpp;        // groups per position, H / 4
  int out_f32;
  void* out2;       // a second copy of the output (same layout), or NULL
};
struct TileArgs {
  TileTensor t[2];
  uint32_t nb0;  // blocks of tensor 0
  uint32_t npos;  // B * S
  Div32 S;
  const void* pos;
  int pb;
  int64_t psb, pss;
  const float* freqs;
  int64_t frows, frs;
  int conj;
  int32_t* err;
  float inv_freq[64];
};

// Position id of flattened position ps = b S + s (ps < 2^31), in two steps so
// that its load can be issued early and waited for late: tile_pos_words
// loads the id's 32-bit words without a branch on the id type (an int32 id
// loads its one word twice) and without using them; tile_pos_value builds
// the id from them.  Without a position tensor the id is s itself.
struct PosWords {
  uint32_t lo, hi;
};
struct PosArgs {
  const void* pos;
  int pb;
  int64_t psb, pss;
  Div32 S;
};
__device__ __forceinline__ PosWords tile_pos_words(const PosArgs& a, uint32_t ps) {
  if (a.pos == nullptr) return PosWords{0u, 0u};
  const uint32_t b = div32(ps, a.S), s = ps - b * a.S.d;
  const int64_t i = (int64_t)b * a.psb + (int64_t)s * a.pss;
  const bool wide = a.pb == 8;
  const uint32_t* w = static_cast<const uint32_t*>(a.pos) + (wide ? 2 * i : i);
  return PosWords{w[0], w[wide ? 1 : 0]};
}
__device__ __forceinline__ int64_t tile_pos_value(const PosArgs& a, PosWords w, uint32_t ps) {
  if (a.pos == nullptr) return ps - div32(ps, a.S) * a.S.d;
  return a.pb == 8 ? (int64_t)(((uint64_t)w.hi << 32) | w.lo) : (int64_t)(int32_t)w.lo;
}

// The block's scalar arguments in one batch: its tensor (q or k, picked by
// block index) and the position arguments.  The empty asm takes every value
// at once, so they are all loaded at fixed argument offsets together and
// the tensor's fields are then selected; indexing a.t[second] made the
// compiler load each field from a computed address -- with the position
// arguments, a chain of dependent scalar loads ahead of the block's first
// data load.
__device__ __forceinline__ void tile_prologue(const TileArgs& a, bool& second, uint32_t& tile, TileTensor& T,
                                              PosArgs& P) {
  const TileTensor& A = a.t[0];
  const TileTensor& B = a.t[1];
  uint64_t ax = (uint64_t)A.x, bx = (uint64_t)B.x, ao = (uint64_t)A.out, bo = (uint64_t)B.out;
  uint64_t a2 = (uint64_t)A.out2, b2 = (uint64_t)B.out2;
  uint32_t ag = A.groups, bg = B.groups, am = A.gpp.m, bm = B.gpp.m, al = A.gpp.l, bl = B.gpp.l;
  uint32_t ad = A.gpp.d, bd = B.gpp.d, af = (uint32_t)A.out_f32, bf = (uint32_t)B.out_f32;
  uint32_t nb0 = a.nb0, pb = (uint32_t)a.pb, Sm = a.S.m, Sl = a.S.l, Sd = a.S.d;
  uint64_t pos = (uint64_t)a.pos, psb = (uint64_t)a.psb, pss = (uint64_t)a.pss;
  asm volatile("" : "+s"(ax), "+s"(bx), "+s"(ao), "+s"(bo), "+s"(a2), "+s"(b2), "+s"(ag), "+s"(bg), "+s"(am),
               "+s"(bm), "+s"(al), "+s"(bl), "+s"(ad), "+s"(bd), "+s"(af), "+s"(bf), "+s"(nb0), "+s"(pb), "+s"(Sm),
               "+s"(Sl), "+s"(Sd), "+s"(pos), "+s"(psb), "+s"(pss));
  second = blockIdx.x >= nb0;
  tile = second ? blockIdx.x - nb0 : blockIdx.x;  // the block's tile within its tensor
  T = TileTensor{reinterpret_cast<const uint16_t*>(second ? bx : ax), reinterpret_cast<void*>(second ? bo : ao),
                 second ? bg : ag, Div32{second ? bm : am, second ? bl : al, second ? bd : ad},
                 (int)(second ? bf : af), reinterpret_cast<void*>(second ? b2 : a2)};
  P = PosArgs{reinterpret_cast<const void*>(pos), (int)pb, (int64_t)psb, (int64_t)pss, Div32{Sm, Sl, Sd}};
}

template <int PAIRING, bool TABLE>
__global__ __launch_bounds__(kThreads) void rope_tile(TileArgs a) {
  constexpr bool kHalf = PAIRING == KP_ROPE_HALF;
  constexpr int FPU = kHalf ? 8 : 4;  // angles per chunk
  // kStage: the block's angles go through LDS -- per position slot cos,
  // s' = sc sin and -s' (sc = -1 for conj), so that no lane multiplies its
  // sines by a sign -- evaluated in theta mode, copied from the table row in
  // rotate-half table mode (with the slot's validity).  Interleaved table
  // mode reads its 4 angles per chunk straight from the row (2 x 16 bytes,
  // an L2 hit; staging them measured 0.8% slower there, while it takes
  // rotate-half's 8 angles per chunk -- 4 x 16 bytes -- from 62 to 55 us at c4).
  constexpr bool kStage = !TABLE || kHalf;
  __shared__ float cs[kStage ? kTileMaxPos : 1][3][64];
  __shared__ int slot_ok[TABLE && kStage ? kTileMaxPos : 1];
  const int lane = threadIdx.x & 63;
  const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  bool second;
  uint32_t tile;
  TileTensor T;
  PosArgs pa;
  tile_prologue(a, second, tile, T, pa);
  const uint32_t g0 = tile * kTileGroups;
  const uint32_t glast = T.groups - 1;
  // Everything the angles depend on -- the position ids of this thread's
  // angle items (vector loads) and the inverse frequency -- is requested
  // before the data: vector loads complete in issue order, so waiting for
  // these is not waiting for the data, and the angle work and the barrier
  // overlap the data's latency instead of following it (c4: ids requested
  // after the data cost ~2.5 us per call).  Item i (threads t and t + 256)
  // is frequency i % 64 of position slot i / 64; a slot past the block's
  // last reads the last one's id and leaves it unused.
  const uint32_t ps0 = div32(g0, T.gpp);
  const uint32_t gl = g0 + kTileGroups - 1 < glast ? g0 + kTileGroups - 1 : glast;
  const int npos = (int)(div32(gl, T.gpp) - ps0) + 1;  // <= kTileMaxPos
  float inv = 0.f;
  if constexpr (!TABLE) inv = a.inv_freq[lane];
  uint32_t pps[2];
  PosWords pw[2];
  if constexpr (kStage) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int slot = ((int)threadIdx.x + k * kThreads) >> 6;  // npos * 64 <= 2 * kThreads
      pps[k] = ps0 + (uint32_t)(slot < npos ? slot : npos - 1);
      pw[k] = tile_pos_words(pa, pps[k]);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // Groups past the tensor's end (last tile only) re-read the last group and store nothing.
  u32x4 v[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const uint32_t g = g0 + wave + 4 * u;
    v[u] = ld16_stream(T.x + ((size_t)(g < glast ? g : glast) * 64 + lane) * 8);
  }
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (!kStage) {
    // interleaved table mode: a group's id is wave-uniform, a scalar load
    // whose wait (lgkmcnt) is independent of the data's (vmcnt)
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const uint32_t g = g0 + wave + 4 * u;
      pps[u] = div32(g < glast ? g : glast, T.gpp);
      pw[u] = tile_pos_words(pa, pps[u]);
    }
  }
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int i = (int)threadIdx.x + k * kThreads;
    if (kStage && i < npos * 64) {
      const int slot = i >> 6;
      const int64_t p = tile_pos_value(pa, pw[k], pps[k]);
      float sn, cn;
      if constexpr (TABLE) {
        // the row's complex entry `lane` (an out-of-range id reads row 0: its outputs are zeroed)
        const bool ok = p >= 0 && p < a.frows;
        const f32x2 t = *reinterpret_cast<const f32x2*>(a.freqs + 2 * ((ok ? p : 0) * a.frs + lane));
        cn = t[0];
        sn = t[1];
        if (lane == 0) {
          slot_ok[slot] = ok ? 1 : 0;
          if (!ok && a.err) *a.err = 1;
        }
      } else {
        sincosf((float)p * inv, &sn, &cn);
      }
      const float sp = a.conj ? -sn : sn;
      cs[slot][0][lane] = cn;
      cs[slot][1][lane] = sp;
      cs[slot][2][lane] = -sp;
    }
  }
  if constexpr (kStage) __syncthreads();
  const int c = lane & 15;
  const int f0 = (kHalf ? (c & 7) : c) * FPU;
  const bool lo = c < 8;
  // Rotate-half, lane holding x1 (lo): x1 c - x2 s; holding x2: x2 c + x1 s --
  // both fma(own, c, partner * s') with s' = -s or s (the table row picked
  // by the lane), the same roundings as rot()'s two outputs (the negation is
  // exact).  conj flips s' again.
  const int srow = (kHalf && lo) ? 2 : 1;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const uint32_t g = g0 + wave + 4 * u;
    const uint32_t ps = div32(g < glast ? g : glast, T.gpp);
    const int slot = (int)(ps - ps0);
    bool ok = true;
    float cv[FPU], sv[FPU];
    if constexpr (kStage) {
      if constexpr (TABLE) ok = slot_ok[slot] != 0;
#pragma unroll
      for (int e = 0; e < FPU; e += 4) {
        const f32x4 cq = *reinterpret_cast<const f32x4*>(&cs[slot][0][f0 + e]);
        const f32x4 sq = *reinterpret_cast<const f32x4*>(&cs[slot][srow][f0 + e]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          cv[e + j] = cq[j];
          sv[e + j] = sq[j];
        }
      }
    } else {
      const int64_t p = tile_pos_value(pa, pw[u], pps[u]);
      ok = p >= 0 && p < a.frows;
      if (!ok && lane == 0 && a.err) *a.err = 1;
      const float* frow = a.freqs + 2 * ((ok ? p : 0) * a.frs + f0);
      const float sc = a.conj ? -1.f : 1.f;  // interleaved: the conjugate's sign alone
#pragma unroll
      for (int q = 0; q < FPU / 2; ++q) {
        const f32x4 t = *reinterpret_cast<const f32x4*>(frow + 4 * q);
        cv[2 * q] = t[0];
        sv[2 * q] = sc * t[1];
        cv[2 * q + 1] = t[2];
        sv[2 * q + 1] = sc * t[3];
      }
    }
    float own[8], o[8];
    unpack8(v[u], own);
    if constexpr (kHalf) {
      u32x4 pv;
#pragma unroll
      for (int i = 0; i < 4; ++i) pv[i] = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v[u][i], 0x128, 0xF, 0xF, false);
      float par[8];
      unpack8(pv, par);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        o[e] = __builtin_fmaf(own[e], cv[e], par[e] * sv[e]);
        if (!ok) o[e] = 0.f;
      }
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        rot(own[2 * q], own[2 * q + 1], cv[q], sv[q], o[2 * q], o[2 * q + 1]);
        if (!ok) o[2 * q] = o[2 * q + 1] = 0.f;
      }
    }
    if (g <= glast) {
      const size_t e0 = ((size_t)g * 64 + lane) * 8;  // first element of this chunk
      if (T.out_f32) {  // block-uniform: the fp32 rotation result, 32 bytes per chunk
        st32f(static_cast<float*>(T.out) + e0, o);
        if (T.out2) st32f(static_cast<float*>(T.out2) + e0, o);
      } else {
        const u32x4 pk = pack8(o);
        st16_stream(static_cast<uint16_t*>(T.out) + e0, pk);
        if (T.out2) st16_stream(static_cast<uint16_t*>(T.out2) + e0, pk);
      }
    }
  }
}

// The tile path applies: D = 128, every tensor contiguous [B, S, H, 128] in
// and out with H % 4 == 0, bf16 out, 16-byte aligned (and an aligned table
// with an even row stride in table mode).
bool tile_ok(const RopeArgs& a, bool table) {
  static const bool enabled = [] {  // KP_ROPE_TILE=0 (tuning knob): one wave per position instead
    const char* e = getenv("KP_ROPE_TILE");
    return e == nullptr || atoi(e) != 0;
  }();
  if (!enabled || a.D != kFastD || (!table && !a.have_inv)) return false;
  if (table && (!aligned16(a.freqs) || (a.frs & 1) != 0)) return false;
  const int64_t npos = a.B * a.S;
  if (npos <= 0 || npos > INT32_MAX) return false;
  for (int i = 0; i < a.nt; ++i) {
    const RopeTensor& t = a.t[i];
    const int64_t hd = t.H * kFastD;
    if (t.H <= 0 || (t.H & 3) != 0 || !aligned16(t.x) || !aligned16(t.out)) return false;
    if (t.H > INT32_MAX / 16 || npos * t.H * 16 > INT32_MAX) return false;  // 32-bit chunk indices
    if (t.xs[2] != kFastD || t.xs[1] != hd || t.xs[0] != a.S * hd) return false;
    if (t.os[2] != kFastD || t.os[1] != hd || t.os[0] != a.S * hd) return false;
  }
  return true;
}

typedef void (*RopeKernel)(RopeArgs);

template <int PAIRING, bool TABLE>
RopeKernel fast_for_upl(int upl) {
  switch (upl) {
    case 1: return rope_fast<PAIRING, TABLE, 1>;
    case 2: return rope_fast<PAIRING, TABLE, 2>;
    case 3: return rope_fast<PAIRING, TABLE, 3>;
    case 4: return rope_fast<PAIRING, TABLE, 4>;
    case 5: return rope_fast<PAIRING, TABLE, 5>;
    case 6: return rope_fast<PAIRING, TABLE, 6>;
    case 8: return rope_fast<PAIRING, TABLE, 8>;
  }
  if constexpr (PAIRING == KP_ROPE_INTERLEAVED) {
    switch (upl) {
      case 10: return rope_fast<PAIRING, TABLE, 10>;
      case 12: return rope_fast<PAIRING, TABLE, 12>;
      case 16: return rope_fast<PAIRING, TABLE, 16>;
    }
  }
  return nullptr;
}

// The fast kernel for this call, or nullptr (then rope_kernel runs).
RopeKernel pick_fast(const RopeArgs& a, int pairing, bool table) {
  if (a.D != kFastD) return nullptr;
  if (table && (!aligned16(a.freqs) || (a.frs & 1) != 0)) return nullptr;
  const bool half = pairing == KP_ROPE_HALF;
  const int64_t cph = half ? kFastD / 16 : kFastD / 8;
  const int64_t units = (a.t[0].H + (a.nt > 1 ? a.t[1].H : 0)) * cph;
  if (units <= 0) return nullptr;
  int64_t upl = ceil_div(units, 64);
  if (upl * (half ? 2 : 1) > kFastMaxLoads) return nullptr;
  static const int kUpl[] = {1, 2, 3, 4, 5, 6, 8, 10, 12, 16};
  for (int c : kUpl)
    if (c >= upl) {
      upl = c;
      break;
    }
  if (half) return table ? fast_for_upl<KP_ROPE_HALF, true>((int)upl) : fast_for_upl<KP_ROPE_HALF, false>((int)upl);
  return table ? fast_for_upl<KP_ROPE_INTERLEAVED, true>((int)upl) : fast_for_upl<KP_ROPE_INTERLEAVED, false>((int)upl);
}

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

// Both entry points: out0_copy / out1_copy (kp_rope_bf16_twice) receive the
// same values as out0 / out1, laid out with the same strides.
static int rope_impl(const char* who, const void* x0, void* out0, int64_t H0, const int64_t* x0_strides,
                     const int64_t* out0_strides, const void* x1, void* out1, int64_t H1,
                     const int64_t* x1_strides, const int64_t* out1_strides, int64_t B, int64_t S, int64_t D,
                     const void* positions, int pos_bytes, int64_t pos_stride_b, int64_t pos_stride_s, int pairing,
                     double theta, const float* freqs_cis, int64_t freq_rows, int64_t freq_row_stride, int conj,
                     int out_f32_mask, void* out0_copy, void* out1_copy, int32_t* error_flag, void* stream) {
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
  if (freqs_cis == nullptr && D == kFastD) {  // the fast kernel's angles: one evaluation per call
    a.have_inv = 1;
    for (int f = 0; f < kFastD / 2; ++f) a.inv_freq[f] = (float)pow(theta, -(double)(2 * f) / (double)kFastD);
  }
  const int64_t npos = B * S;
  if (npos == 0) return KP_OK;

  bool vec = tensor_vec_ok(a.t[0], D, pairing) && (a.nt == 1 || tensor_vec_ok(a.t[1], D, pairing));
  const int64_t blocks_needed = ceil_div(npos, kWavesPerBlock);
  const bool copies_aligned = (out0_copy == nullptr || aligned16(out0_copy)) && (out1_copy == nullptr || aligned16(out1_copy));
  if (vec && copies_aligned && tile_ok(a, freqs_cis != nullptr)) {
    TileArgs ta{};
    for (int i = 0; i < a.nt; ++i)
      ta.t[i] = TileTensor{a.t[i].x, a.t[i].out, (uint32_t)(npos * (a.t[i].H / 4)),
                           make_div32((uint32_t)(a.t[i].H / 4)), a.t[i].out_f32, i == 0 ? out0_copy : out1_copy};
    ta.nb0 = (uint32_t)ceil_div(ta.t[0].groups, kTileGroups);
    const int64_t nb1 = a.nt > 1 ? ceil_div(ta.t[1].groups, kTileGroups) : 0;
    ta.npos = (uint32_t)npos;
    ta.S = make_div32((uint32_t)S);
    ta.pos = a.pos;
    ta.pb = a.pb;
    ta.psb = a.psb;
    ta.pss = a.pss;
    ta.freqs = a.freqs;
    ta.frows = a.frows;
    ta.frs = a.frs;
    ta.conj = a.conj;
    ta.err = a.err;
    for (int f = 0; f < 64; ++f) ta.inv_freq[f] = a.inv_freq[f];
    const bool tab = freqs_cis != nullptr, half = pairing == KP_ROPE_HALF;
    const void* fk = half ? (tab ? reinterpret_cast<const void*>(rope_tile<KP_ROPE_HALF, true>)
                                 : reinterpret_cast<const void*>(rope_tile<KP_ROPE_HALF, false>))
                          : (tab ? reinterpret_cast<const void*>(rope_tile<KP_ROPE_INTERLEAVED, true>)
                                 : reinterpret_cast<const void*>(rope_tile<KP_ROPE_INTERLEAVED, false>));
    void* args[] = {&ta};
    launch_dominant_raw(fk, dim3((unsigned)(ta.nb0 + nb1)), dim3(kThreads), args, 0, as_stream(stream));
    return check_launch(who);
  }
  // Other layouts: one launch per copy (the copies' rows are written by a
  // second pass over the inputs).
  const bool copies = out0_copy != nullptr;
  if (copies) vec = vec && copies_aligned;
  for (int rep = 0; rep < (copies ? 2 : 1); ++rep) {
    if (rep == 1) {
      a.t[0].out = out0_copy;
      if (a.nt > 1) a.t[1].out = out1_copy;
    }
    const RopeKernel fk = vec ? pick_fast(a, pairing, freqs_cis != nullptr) : nullptr;
    if (fk != nullptr && blocks_needed <= INT32_MAX) {
      void* args[] = {&a};
      launch_dominant_raw(reinterpret_cast<const void*>(fk), dim3((unsigned)blocks_needed), dim3(kThreads), args, 0,
                          as_stream(stream));
    } else {
      const int64_t cap = (int64_t)cu_count() * 16;
      const int grid = (int)(blocks_needed < cap ? blocks_needed : cap);
      hipStream_t s = as_stream(stream);
      const bool tab = freqs_cis != nullptr;
      if (vec && tab) KP_LAUNCH_DOMINANT((rope_kernel<true, true>), dim3(grid), dim3(kThreads), 0, s, a);
      else if (vec) KP_LAUNCH_DOMINANT((rope_kernel<true, false>), dim3(grid), dim3(kThreads), 0, s, a);
      else if (tab) KP_LAUNCH_DOMINANT((rope_kernel<false, true>), dim3(grid), dim3(kThreads), 0, s, a);
      else KP_LAUNCH_DOMINANT((rope_kernel<false, false>), dim3(grid), dim3(kThreads), 0, s, a);
    }
    const int st = check_launch(who);
    if (st != KP_OK) return st;
  }
  return KP_OK;
}

int kp_rope_bf16(const void* x0, void* out0, int64_t H0, const int64_t* x0_strides, const int64_t* out0_strides,
                 const void* x1, void* out1, int64_t H1, const int64_t* x1_strides, const int64_t* out1_strides,
                 int64_t B, int64_t S, int64_t D, const void* positions, int pos_bytes, int64_t pos_stride_b,
                 int64_t pos_stride_s, int pairing, double theta, const float* freqs_cis, int64_t freq_rows,
                 int64_t freq_row_stride, int conj, int out_f32_mask, int32_t* error_flag, void* stream) {
  return rope_impl("kp_rope_bf16", x0, out0, H0, x0_strides, out0_strides, x1, out1, H1, x1_strides, out1_strides, B,
                   S, D, positions, pos_bytes, pos_stride_b, pos_stride_s, pairing, theta, freqs_cis, freq_rows,
                   freq_row_stride, conj, out_f32_mask, nullptr, nullptr, error_flag, stream);
}

int kp_rope_bf16_twice(const void* x0, void* out0, int64_t H0, const int64_t* x0_strides,
                       const int64_t* out0_strides, const void* x1, void* out1, int64_t H1,
                       const int64_t* x1_strides, const int64_t* out1_strides, int64_t B, int64_t S, int64_t D,
                       const void* positions, int pos_bytes, int64_t pos_stride_b, int64_t pos_stride_s,
                       int pairing, double theta, const float* freqs_cis, int64_t freq_rows,
                       int64_t freq_row_stride, int conj, int out_f32_mask, void* out0_copy, void* out1_copy,
                       int32_t* error_flag, void* stream) {
  static const char* who = "kp_rope_bf16_twice";
  if (out0_copy == nullptr || (x1 != nullptr && out1_copy == nullptr))
    return fail(KP_EINVAL, "%s: every rotated tensor needs its copy", who);
  if (out0_copy == out0 || (x1 != nullptr && out1_copy == out1))
    return fail(KP_EINVAL, "%s: a copy must not be its own output", who);
  return rope_impl(who, x0, out0, H0, x0_strides, out0_strides, x1, out1, H1, x1_strides, out1_strides, B, S, D,
                   positions, pos_bytes, pos_stride_b, pos_stride_s, pairing, theta, freqs_cis, freq_rows,
                   freq_row_stride, conj, out_f32_mask, out0_copy, x1 != nullptr ? out1_copy : nullptr, error_flag,
                   stream);
}

}  // extern "C"
