// Shared device helpers for the gfx950 (CDNA4, wave64) fragment kernels.
//
// Everything here is written for one target: gfx950.  bf16 values travel as raw
// uint16 bit patterns packed two to a dword; 16-byte vectors (8 bf16) are the
// unit of every global load/store on the fast paths so that each wave64 memory
// instruction moves 1 KiB.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/kp.h"
#include "kp_div32.hpp"

namespace kp {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// ---------------------------------------------------------------- bf16 <-> f32
__device__ __forceinline__ float bf_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf_hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }
__device__ __forceinline__ float bf_to_f(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

// Two floats -> packed bf16x2, round-to-nearest-even (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  f32x2 v = {lo, hi};
  bf16x2 r = __builtin_convertvector(v, bf16x2);
  return __builtin_bit_cast(uint32_t, r);
}
__device__ __forceinline__ uint16_t f_to_bf(float f) { return (uint16_t)(pack_bf2(f, 0.f) & 0xffffu); }
// fp32 value rounded to the nearest bf16 and widened back to fp32.
__device__ __forceinline__ float round_bf(float f) { return bf_lo(pack_bf2(f, 0.f)); }

// 8 bf16 (one 16-byte vector) -> 8 floats.
__device__ __forceinline__ void unpack8(const u32x4& v, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf_lo(v[i]);
    f[2 * i + 1] = bf_hi(v[i]);
  }
}
__device__ __forceinline__ u32x4 pack8(const float* f) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = pack_bf2(f[2 * i], f[2 * i + 1]);
  return r;
}
// Elementwise bf16 + bf16 -> bf16 the way an eager bf16 add does it: both
// operands widened to fp32, one fp32 add, one RNE rounding.
__device__ __forceinline__ u32x4 add_bf8(const u32x4& a, const u32x4& b) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    r[i] = pack_bf2(bf_lo(a[i]) + bf_lo(b[i]), bf_hi(a[i]) + bf_hi(b[i]));
  return r;
}

// ------------------------------------------------------------ global memory
__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
// Streaming load: data used exactly once (nt hint keeps it from displacing reused lines).
__device__ __forceinline__ u32x4 ld16_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ void st16(void* p, const u32x4& v) { *reinterpret_cast<u32x4*>(p) = v; }
// Streaming store (nt): output written once and not re-read by this kernel.
// Measured on MI355X: streaming stores raise large copy-like kernels by ~5%
// over default write-back stores and shorten the end-of-kernel drain.
__device__ __forceinline__ void st16_stream(void* p, const u32x4& v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}
__device__ __forceinline__ void st16f_stream(void* p, const f32x4& v) {
  __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(p));
}
// A lane's 32 contiguous fp32 bytes as two 16-byte default (write-back)
// stores.  When each lane of a wave writes 32 bytes, one store instruction
// covers every other 16 bytes, so a line is only whole once both have
// landed: write-back stores let L2 merge the halves, whereas streaming
// stores of half lines cost the fp32 RoPE output ~11% (measured on MI355X:
// v7/0f38bc55457c 46.1 -> 41.2 us per call).
__device__ __forceinline__ void st32f(float* p, const float* v) {
  *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
  *reinterpret_cast<f32x4*>(p + 4) = f32x4{v[4], v[5], v[6], v[7]};
}

// ------------------------------------------------------------ wave64 reductions
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
// A wave-uniform 64-bit value moved into scalar registers (readfirstlane of
// both halves), so that later per-lane selects between such values stay selects.
__device__ __forceinline__ int64_t uniform64(int64_t v) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)((uint64_t)v >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ float readlane_f(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Sum of one float over the 64 lanes of a wave.  Within each 16-lane DPP row
// the tree is quad xor-1, quad xor-2, half-row mirror, row mirror (every lane
// of a row ends with the identical row sum); the four row sums are then read
// as scalars and combined as (r0 + r1) + (r2 + r3).  The result is bitwise the
// same in every lane and the order is fixed, so the reduction is deterministic.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f<0x141>(v);  // row_half_mirror
  v += dpp_f<0x140>(v);  // row_mirror
  float r0 = readlane_f(v, 0), r1 = readlane_f(v, 16), r2 = readlane_f(v, 32), r3 = readlane_f(v, 48);
  return (r0 + r1) + (r2 + r3);
}


__host__ __device__ __forceinline__ int64_t ceil_div_dev(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace kp
