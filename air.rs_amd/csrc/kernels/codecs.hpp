// Device-side scalar codecs, bit-exact with the reference's CPU arithmetic.
//
// The library is compiled without fast-math: f32 division is correctly
// rounded and f32 denormals are kept, which the quantizers below rely on.
// Floating-point contraction is switched off inside every codec so each f32
// operation rounds exactly once, as Rust's does.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace airkv {

// f32 -> bf16 bits, round to nearest even; NaN keeps its high half with the
// quiet bit set (half 2.7.1 bf16::from_f32, the conversion candle and the
// reference use, src/pd_disagg.rs:66-69).
__device__ __forceinline__ uint16_t bf16_rne(float x) {
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x0040u);
    uint32_t lsb = (u >> 16) & 1u;
    return (uint16_t)((u + 0x7FFFu + lsb) >> 16);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// F8E4M3::from_f32 (src/fp8.rs:54-91): -0.0 -> 0x00 (sign is x < 0), |x| >= 448
// and exponent field 15 saturate to 0x7E, the mantissa rounds half-up and is
// capped at 7 (no carry), subnormal results flush to signed zero, NaN -> 0x7F.
// Written as selects, no branches: |x| >= 448 (infinity included) has an
// exponent field of at least 15 and saturates with it, and zero has field
// -120 and flushes with the subnormals; the sign joins every non-zero,
// non-NaN value.
__device__ __forceinline__ uint8_t fp8_encode(float x) {
    const uint32_t bits = __float_as_uint(x), a = bits & 0x7FFFFFFFu;
    const int exp8 = (int)(a >> 23) - 120;
    uint32_t mant3 = ((a & 0x007FFFFFu) + (1u << 19)) >> 20;
    mant3 = mant3 > 7u ? 7u : mant3;
    uint32_t v = ((uint32_t)exp8 << 3) | mant3;
    v = exp8 >= 15 ? 0x7Eu : v;
    v = exp8 <= 0 ? 0u : v;
    v |= a != 0u ? (bits >> 24) & 0x80u : 0u;
    return (uint8_t)(a > 0x7F800000u ? 0x7Fu : v);
}

// F8E4M3::to_f32 (src/fp8.rs:94-112): 0x7F is NaN, exponent field 0 decodes to
// +0.0 whatever the sign, 0xFF decodes to -480.  Every value is an exact f32.
__device__ __forceinline__ float fp8_decode(uint32_t b) {
    b &= 0xFFu;
    uint32_t e = (b >> 3) & 0xFu;
    uint32_t bits = ((b & 0x80u) << 24) | (((b & 0x7Fu) << 20) + (120u << 23));
    float v = __uint_as_float(bits);
    v = e == 0u ? 0.0f : v;
    return b == 0x7Fu ? __uint_as_float(0x7FC00000u) : v;
}

// One step of the absmax fold `m.max(v.abs())` (src/kv_cache.rs:60,
// src/fp8.rs:228-232): Rust's f32::max returns the other operand when one is
// NaN, signalling or quiet.  v_max_f32 in IEEE mode turns a signalling NaN
// into a quiet NaN result instead, so the fold is a compare-select, which
// ignores every NaN and never produces one from a non-NaN accumulator.
__device__ __forceinline__ float absmax_step(float m, float x) {
    const float a = fabsf(x);
    return a > m ? a : m;
}

// Rust `f32::round` then saturating `as i8` after a clamp to +-127
// (src/kv_cache.rs:69): NaN -> 0.
// Computed on the magnitude as pd_code below does, capped at 127 (checked
// against the reference rule the same way).
__device__ __forceinline__ int8_t q8_code(float x, float inv) {
#pragma clang fp contract(off)
    const float y = x * inv;
    const float a = __builtin_fabsf(y);
    float r = !(a >= 0.5f) ? 0.0f : __builtin_floorf(a + 0.5f);
    r = __builtin_fminf(r, 127.0f);
    return (int8_t)(int)__builtin_copysignf(r, y);
}

// KvBlock::int8_quantize's code (src/pd_disagg.rs:78-80): Rust `f32::round`
// then a saturating `as i8` with no clamp before it, so an infinite product
// (1 / scale overflows when the block's absmax is subnormal) gives -128 or
// 127, and NaN gives 0.
// Computed on the magnitude: round half away from zero is 0 below 0.5 and
// floor(|y| + 0.5) from there (equal to exact rounding for every float up to
// 300; larger ones saturate anyway), a NaN fails the comparison and gives 0,
// and the magnitude is capped at 128 before the sign goes back on (checked
// against the reference rule for every float of magnitude below 300, the
// special values and 2^24 random bit patterns).
__device__ __forceinline__ int8_t pd_code(float x, float inv) {
#pragma clang fp contract(off)
    const float y = x * inv;
    const float a = __builtin_fabsf(y);
    float r = !(a >= 0.5f) ? 0.0f : __builtin_floorf(a + 0.5f);
    r = __builtin_fminf(r, 128.0f);
    const int c = (int)__builtin_copysignf(r, y);
    return (int8_t)(c > 127 ? 127 : c);
}

// Q8_0 scale from the group's absmax (src/kv_cache.rs:60-62).
__device__ __forceinline__ float q8_scale(float max_abs) {
#pragma clang fp contract(off)
    return max_abs == 0.0f ? 1.0f : max_abs / 127.0f;
}

// FP8 group scale (Fp8Layer rule, src/fp8.rs:230-234).
__device__ __forceinline__ float fp8_scale(float max_abs) {
#pragma clang fp contract(off)
    return max_abs < 1e-8f ? 1.0f : max_abs / 448.0f;
}

// The code of x / scale, with y = RN(1 / scale) and `mark` = scale and y both
// normal (a group's values, computed once).  The quotient is then
// q0 = RN(x * y) corrected once, q = RN(q0 + fma(-q0, scale, x) * y)
// (Markstein): RN(x / scale) whenever the remainder is exact, which holds for
// every |q| >= 2^-6 -- the only quotients whose code depends on more than
// their sign (here |x| >= 2^-6 * scale >= 2^-42, far from the subnormals).
// Below that the code is the sign alone, and a quotient that comes out
// subnormal or zero is divided exactly, so a tiny negative one is not turned
// into a zero.  The codes equal the division's on random and boundary cases
// (tests/fp8_quotient_check.c; 4e8 cases run once, none differing).
__device__ __forceinline__ uint8_t fp8_code(float x, float scale, float y, bool mark) {
#pragma clang fp contract(off)
    if (mark) {
        float q = x * y;
        q = __builtin_fmaf(__builtin_fmaf(-q, scale, x), y, q);
        if (__builtin_fabsf(q) >= 0x1p-126f) return fp8_encode(q);
    }
    return fp8_encode(x / scale);
}

// fp8_encode of a value known to be neither zero nor NaN (|x| >= 2^-126 or
// infinite): the sign always joins, and NaN cannot occur.
__device__ __forceinline__ uint32_t fp8_encode_nonzero(float x) {
    const uint32_t bits = __float_as_uint(x), a = bits & 0x7FFFFFFFu;
    const int exp8 = (int)(a >> 23) - 120;
    uint32_t mant3 = ((a & 0x007FFFFFu) + (1u << 19)) >> 20;
    mant3 = mant3 > 7u ? 7u : mant3;
    uint32_t v = ((uint32_t)exp8 << 3) | mant3;
    v = exp8 >= 15 ? 0x7Eu : v;
    v = exp8 <= 0 ? 0u : v;
    return v | ((bits >> 24) & 0x80u);
}

// fp8_code of N elements sharing a scale: the corrected products for all
// N, and one branch (rarely taken) that divides those whose quotient needs
// the exact division, then the codes, four per word (element 4i + j in byte
// j of w[i]).
template <int N>
__device__ __forceinline__ void fp8_codes(const float (&x)[N], float scale, float y, bool mark,
                                          uint32_t (&w)[N / 4]) {
#pragma clang fp contract(off)
    float q[N];
    bool slow = !mark;
#pragma unroll
    for (int j = 0; j < N; ++j) {
        const float p = x[j] * y;
        q[j] = __builtin_fmaf(__builtin_fmaf(-p, scale, x[j]), y, p);
        slow |= !(__builtin_fabsf(q[j]) >= 0x1p-126f);
    }
#pragma unroll
    for (int i = 0; i < N / 4; ++i) w[i] = 0;
    if (__builtin_expect(slow, 0)) {
#pragma unroll
        for (int j = 0; j < N; ++j)
            if (!mark || !(__builtin_fabsf(q[j]) >= 0x1p-126f)) q[j] = x[j] / scale;
#pragma unroll
        for (int j = 0; j < N; ++j) w[j / 4] |= (uint32_t)fp8_encode(q[j]) << (8 * (j % 4));
    } else {                    // every quotient at least 2^-126 in magnitude (or infinite)
#pragma unroll
        for (int j = 0; j < N; ++j) w[j / 4] |= fp8_encode_nonzero(q[j]) << (8 * (j % 4));
    }
}

}  // namespace airkv
