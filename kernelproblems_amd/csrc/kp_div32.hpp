// Division of a 32-bit n < 2^31 by a divisor d (1 <= d < 2^31) that is fixed
// for a launch, without a divide sequence: with l = ceil(log2 d) and
// m = floor(2^32 (2^l - d) / d) + 1 (< 2^32), n / d = (mulhi(n, m) + n) >> l
// (Granlund & Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994, section 4; the multiplier's 2^32 term is the
// "+ n", which cannot overflow since mulhi(n, m) < n < 2^31).  The host
// computes (m, l) once; in a kernel a wave-uniform n takes two scalar ops.
//
// Both functions are constexpr, which hipcc compiles for host and device
// alike, so the kernels and the host-side unit test (g++, no HIP headers)
// run this one definition.
#pragma once

#include <stdint.h>

namespace kp {

struct Div32 {
  uint32_t m, l, d;
};

constexpr Div32 make_div32(uint32_t d) {
  uint32_t l = 0;
  while ((1ull << l) < d) ++l;
  return Div32{(uint32_t)(((1ull << 32) * ((1ull << l) - d)) / d + 1), l, d};
}

// mulhi as the high word of the 64-bit product (v_mul_hi_u32 / s_mul_hi_u32
// on the device).
constexpr uint32_t div32(uint32_t n, const Div32& q) {
  return (uint32_t)((((uint64_t)n * q.m) >> 32) + n) >> q.l;
}

}  // namespace kp
