// The kernels' invariant-divisor division (air.rs_amd/csrc/kernels/
// fastdiv.hpp, included as it is compiled into the device code) against the
// division operator: every divisor 1 .. 300 (head_dim / 8, kv heads, any
// other launch constant the kernels divide by), each with every n below
// 2^21, the 2^20 values below 2^32, every multiple k d (k < 4096) and its
// predecessor, and 2^20 xorshift values; then 1000 random divisors up to
// 2^32 - 1 on the edges and random values.  Prints "<checked> checked,
// <bad> differ".
#include <cstdio>
#include <cstdint>

#include "kernels/fastdiv.hpp"

int main() {
    using airkv::fast_div;
    using airkv::make_fast_div;
    uint64_t checked = 0, bad = 0;
    auto check = [&](uint32_t n, const airkv::FastDiv &f) {
        ++checked;
        if (fast_div(n, f) != n / f.d && bad++ < 5) std::printf("d=%u n=%u: %u\n", f.d, n, fast_div(n, f));
    };
    uint64_t x = 88172645463325252ull;
    auto next = [&]() {
        x ^= x << 13;
        x ^= x >> 7;
        x ^= x << 17;
        return (uint32_t)x;
    };
    for (uint32_t d = 1; d <= 300; ++d) {
        const airkv::FastDiv f = make_fast_div(d);
        for (uint32_t n = 0; n < (1u << 21); ++n) check(n, f);
        for (uint64_t n = 0xFFFFFFFFull - (1u << 20); n <= 0xFFFFFFFFull; ++n) check((uint32_t)n, f);
        for (uint64_t k = 1; k < 4096 && k * d <= 0xFFFFFFFFull; ++k) {
            check((uint32_t)(k * d), f);
            check((uint32_t)(k * d - 1), f);
        }
        for (int i = 0; i < (1 << 20); ++i) check(next(), f);
    }
    for (int j = 0; j < 1000; ++j) {
        const uint32_t d = next() | 1u;
        const airkv::FastDiv f = make_fast_div(d);
        for (uint32_t e = 0; e < 64; ++e) {
            check(d - 1 + e, f);
            check(0xFFFFFFFFu - e, f);
            check(2 * (uint64_t)d - 1 + e <= 0xFFFFFFFFull ? 2 * d - 1 + e : e, f);
        }
        for (int i = 0; i < 4096; ++i) check(next(), f);
    }
    std::printf("%llu checked, %llu differ\n", (unsigned long long)checked, (unsigned long long)bad);
    return bad != 0;
}
