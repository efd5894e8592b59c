// Host check of kp::make_div32 / kp::div32 (kernelproblems_amd/csrc/kp_div32.hpp,
// the same constexpr definitions the kernels compile) against the quotient n / d.
// Divisors: 1..4096, every 2^k and 2^k +- 1 / +- 2, the largest values below
// 2^31, and random ones; numerators: 0, 1, around every multiple k d (k small
// and k near (2^31 - 1) / d), around 2^31 - 1, and random ones.  Prints the
// number of pairs checked and of mismatches (exit status 1 on any mismatch).
#include <cstdint>
#include <cstdio>
#include <vector>

#include "kp_div32.hpp"

static uint64_t g_state = 0x9E3779B97F4A7C15ull;
static uint32_t rnd31() {  // splitmix64, top 31 bits
  uint64_t z = (g_state += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  z ^= z >> 31;
  return (uint32_t)(z >> 33);
}

static uint64_t g_checked = 0, g_bad = 0;
static void check(uint32_t n, uint32_t d, const kp::Div32& q) {
  const uint32_t want = n / d, got = kp::div32(n, q);
  ++g_checked;
  if (got != want) {
    if (g_bad < 10) std::printf("mismatch n=%u d=%u got=%u want=%u\n", n, d, got, want);
    ++g_bad;
  }
}

int main() {
  const uint32_t kMaxN = 0x7fffffffu;
  std::vector<uint32_t> divisors;
  for (uint32_t d = 1; d <= 4096; ++d) divisors.push_back(d);
  for (int k = 1; k <= 31; ++k) {
    const int64_t p = (int64_t)1 << k;
    for (int64_t e = -2; e <= 2; ++e)
      if (p + e >= 1 && p + e <= kMaxN) divisors.push_back((uint32_t)(p + e));
  }
  for (uint32_t e = 0; e < 64; ++e) divisors.push_back(kMaxN - e);
  for (int i = 0; i < 2000; ++i) divisors.push_back(1 + rnd31() % kMaxN);
  for (int i = 0; i < 2000; ++i) divisors.push_back(1 + rnd31() % 65536);

  for (uint32_t d : divisors) {
    const kp::Div32 q = kp::make_div32(d);
    if (q.d != d) {
      std::printf("make_div32(%u) stored d=%u\n", d, q.d);
      ++g_bad;
    }
    const uint32_t kmax = kMaxN / d;
    for (uint32_t k = 0; k <= 8 && k <= kmax; ++k)
      for (int64_t e = -1; e <= 1; ++e) {
        const int64_t n = (int64_t)k * d + e;
        if (n >= 0 && n <= kMaxN) check((uint32_t)n, d, q);
      }
    for (uint32_t k = kmax > 8 ? kmax - 8 : 0; k <= kmax; ++k)
      for (int64_t e = -1; e <= 1; ++e) {
        const int64_t n = (int64_t)k * d + e;
        if (n >= 0 && n <= kMaxN) check((uint32_t)n, d, q);
      }
    for (uint32_t e = 0; e < 16; ++e) check(kMaxN - e, d, q);
    for (int i = 0; i < 256; ++i) check(rnd31(), d, q);
  }
  std::printf("checked %llu pairs, %llu mismatches\n", (unsigned long long)g_checked, (unsigned long long)g_bad);
  return g_bad == 0 ? 0 : 1;
}
