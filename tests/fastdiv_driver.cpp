// Checks ec::fast_div (megatron-lm_amd/csrc/fastdiv.h) against the hardware
// divide: every divisor up to 4096 and around every power of two, each with
// numerators at the ends of the range, around multiples of the divisor and
// drawn at random.  Built with g++ (the HIP qualifiers defined away).
#include <cstdio>
#include <cstdint>
#include <random>
#include <vector>

#include "fastdiv.h"

static int check(uint32_t d, uint32_t n) {
  const uint32_t got = ec::fast_div(n, ec::make_fastdiv(d));
  if (got != n / d) {
    std::printf("fast_div(%u, %u) = %u, want %u\n", n, d, got, n / d);
    return 1;
  }
  return 0;
}

int main() {
  std::vector<uint32_t> divisors;
  for (uint32_t d = 1; d <= 4096; ++d) divisors.push_back(d);
  for (int b = 12; b < 31; ++b)
    for (int64_t e = -3; e <= 3; ++e) divisors.push_back((uint32_t)((1ll << b) + e));
  divisors.push_back(0x7fffffffu);
  divisors.push_back(0x7ffffffeu);
  std::mt19937_64 rng(12345);
  const uint32_t top = 0x7fffffffu;
  int bad = 0;
  for (uint32_t d : divisors) {
    for (uint32_t n : {0u, 1u, 2u, d - 1, d, d + 1, top, top - 1, top - d + 1, top - d})
      if (n <= top) bad += check(d, n);
    const uint32_t q_top = top / d;
    for (int i = 0; i < 64; ++i) {
      const uint64_t q = rng() % (uint64_t)(q_top + 1);
      for (int64_t r : {(int64_t)-1, (int64_t)0, (int64_t)1, (int64_t)d - 1}) {
        const int64_t n = (int64_t)q * d + r;
        if (n >= 0 && n <= top) bad += check(d, (uint32_t)n);
      }
      bad += check(d, (uint32_t)(rng() & top));
    }
    if (bad) return 1;
  }
  std::printf("fastdiv driver ok: %zu divisors\n", divisors.size());
  return 0;
}
