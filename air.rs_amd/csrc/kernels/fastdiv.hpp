// Division of 32-bit unsigned integers by a divisor fixed for a launch: one
// high multiply, a subtract, an add and two shifts instead of the
// multi-instruction integer division a runtime divisor otherwise costs per
// use.  The method is Granlund and Montgomery, "Division by invariant
// integers using multiplication" (PLDI 1994, figure 4.1) with N = 32:
//   l = ceil(log2 d),  m = floor(2^32 (2^l - d) / d) + 1  (m < 2^32),
//   t = floor(m n / 2^32),  q = (t + ((n - t) >> min(l, 1))) >> max(l - 1, 0),
// and q = floor(n / d) for every 0 <= n < 2^32 and 1 <= d < 2^32.  Plain C++
// on the host (tests/fastdiv_check.cpp checks these lines against the
// division operator), the same lines in device code.
#pragma once

#include <stdint.h>

#ifdef __HIPCC__
#define AIRKV_HD __host__ __device__
#else
#define AIRKV_HD
#endif

namespace airkv {

struct FastDiv {
    uint32_t m, d, s1, s2;
};

inline FastDiv make_fast_div(uint32_t d) {   // d >= 1
    uint32_t l = 0;
    while (l < 32 && (1ull << l) < d) ++l;
    const uint64_t m = ((1ull << 32) * ((1ull << l) - d)) / d + 1;
    return FastDiv{(uint32_t)m, d, l < 1 ? l : 1u, l > 1 ? l - 1 : 0u};
}

AIRKV_HD inline uint32_t fast_div(uint32_t n, const FastDiv &f) {
    const uint32_t t = (uint32_t)(((uint64_t)f.m * n) >> 32);
    return (t + ((n - t) >> f.s1)) >> f.s2;
}

}  // namespace airkv
