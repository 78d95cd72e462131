// Division by an invariant divisor as a multiply-high and two shifts
// (Granlund and Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994, figure 4.1), exact for every 32-bit unsigned
// dividend n and divisor d >= 1: with l = ceil(log2 d),
//   m = floor(2^32 (2^l - d) / d) + 1   (fits in 32 bits, since 2^(l-1) < d),
//   t = mulhi(m, n),
//   n / d = (t + ((n - t) >> min(l, 1))) >> max(l - 1, 0).
// Plain C++: the host builds the constants, the kernels apply them (fast_div
// in common.h), and fast_div_host lets a CPU test check the same arithmetic.
#pragma once

#include <stdint.h>

namespace ako {

struct FastDiv {
  uint32_t m;
  uint32_t s1, s2;
};

// d must be at least 1.
inline FastDiv make_fastdiv(uint32_t d) {
  uint32_t l = 0;
  while ((uint64_t(1) << l) < d) ++l;
  const uint64_t m = (uint64_t(1) << 32) * ((uint64_t(1) << l) - d) / d + 1;
  return FastDiv{static_cast<uint32_t>(m), l < 1 ? l : 1u, l > 1 ? l - 1 : 0u};
}

inline uint32_t fast_div_host(uint32_t n, const FastDiv& f) {
  const uint32_t t = static_cast<uint32_t>((uint64_t(f.m) * n) >> 32);
  return (t + ((n - t) >> f.s1)) >> f.s2;
}

}  // namespace ako
