// fastdiv.h — division by a divisor fixed at launch, as a multiply and a
// shift (Granlund and Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994, round-up method).
//
// For 1 <= d < 2^31 let p = ceil(log2 d) and m = ceil(2^(31+p) / d), which
// fits 32 bits.  Then for every 0 <= n < 2^31
//     floor(n * m / 2^(31+p)) = floor(n / d):
// m = (2^(31+p) + e) / d with 0 <= e < d <= 2^p, so n * m / 2^(31+p) =
// n / d + n * e / (d * 2^(31+p)), and n * e < 2^(31+p) keeps the added term
// below 1/d, too little to carry n / d past the next integer.
//
// The kernels divide workgroup indices (< 2^31) by per-launch counts; the
// hardware has no integer divide, and the compiler's sequence for a run-time
// divisor costs a float reciprocal and a few dozen instructions per
// workgroup.
#pragma once

#include <stdint.h>

namespace ec {

struct FastDiv {
  uint32_t mul;
  uint32_t shift;  // 31 + p
};

// Host side: the multiplier and shift for a divisor 1 <= d < 2^31.
inline FastDiv make_fastdiv(uint32_t d) {
  uint32_t p = 0;
  while ((1ull << p) < d) ++p;
  const uint64_t num = 1ull << (31 + p);
  return FastDiv{(uint32_t)((num + d - 1) / d), 31 + p};
}

// n / d for 0 <= n < 2^31.
__host__ __device__ __forceinline__ uint32_t fast_div(uint32_t n, FastDiv f) {
  return (uint32_t)(((uint64_t)n * f.mul) >> f.shift);
}

}  // namespace ec
