// Division of 32-bit unsigned integers by a divisor fixed at launch time, without the
// integer-divide sequence in the kernels' inner loops.
//
// Method: Granlund & Montgomery, "Division by invariant integers using multiplication"
// (PLDI 1994), round-up variant.  For a divisor d >= 1 let s = ceil(log2 d) and
// m = floor(2^32 * (2^s - d) / d) + 1 (m < 2^32).  Then for every n < 2^32
//   n / d == (mulhi32(n, m) + n) >> s
// with the sum formed in 64 bits.  d = 1 and powers of two give m = 1, mulhi = 0, a shift.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define BARQ_HD __host__ __device__
#else
#define BARQ_HD
#endif

struct FastDiv {
  uint32_t d;
  uint32_t m;
  uint32_t s;

  static FastDiv make(uint32_t divisor) {
    FastDiv f;
    f.d = divisor ? divisor : 1u;
    uint32_t s = 0;
    while ((1ull << s) < f.d) ++s;
    f.s = s;
    f.m = (uint32_t)((((1ull << s) - f.d) << 32) / f.d + 1ull);
    return f;
  }

  BARQ_HD uint32_t div(uint32_t n) const {
#if defined(__HIP_DEVICE_COMPILE__)
    const uint32_t hi = __umulhi(n, m);
#else
    const uint32_t hi = (uint32_t)(((uint64_t)n * m) >> 32);
#endif
    return (uint32_t)(((uint64_t)hi + n) >> s);
  }
};
