/* Test infrastructure: the fp8 append codes of x / scale (F8E4M3::from_f32 of
 * the quotient, src/fp8.rs:54-91, scale = absmax / 448 as src/fp8.rs:228-240)
 * computed by division and by the Markstein-corrected reciprocal product the
 * GPU append uses (air.rs_amd/csrc/kernels/codecs.hpp fp8_code), compared on
 * random and boundary cases.  Exit status 0 when no code differs.
 * usage: fp8_quotient_check [cases] */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static uint32_t fbits(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static float ffrom(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

/* the reference encoder's rules: -0 -> 0x00, >= 448 and exponent field 15
 * -> 0x7E, mantissa half-up capped at 7, subnormal results flush to the sign */
static uint8_t encode(float x) {
    if (x != x) return 0x7F;
    uint32_t sign = x < 0.0f ? 0x80u : 0u, bits = fbits(x) & 0x7FFFFFFFu;
    float a = ffrom(bits);
    if (a == 0.0f) return (uint8_t)sign;
    if (a >= 448.0f) return (uint8_t)(sign | 0x7Eu);
    int e = (int)(bits >> 23) - 120;
    if (e <= 0) return (uint8_t)sign;
    if (e >= 15) return (uint8_t)(sign | 0x7Eu);
    uint32_t m = ((bits & 0x007FFFFFu) + (1u << 19)) >> 20;
    return (uint8_t)(sign | ((uint32_t)e << 3) | (m > 7u ? 7u : m));
}

static float scale_of(float m) { volatile float s = m < 1e-8f ? 1.0f : m / 448.0f; return s; }

static uint8_t code_product(float x, float s) {
    volatile float y = 1.0f / s;
    if (isnormal(s) && isnormal(y)) {
        volatile float q = x * y;
        volatile float r = fmaf(-q, s, x);
        volatile float q1 = fmaf(r, y, q);
        if (fabsf(q1) >= 0x1p-126f) return encode(q1);
    }
    volatile float qd = x / s;
    return encode(qd);
}

static uint64_t state = 0x9E3779B97F4A7C15ull;
static uint64_t next(void) { state ^= state << 13; state ^= state >> 7; state ^= state << 17; return state; }

int main(int argc, char **argv) {
    long n = argc > 1 ? atol(argv[1]) : 20000000L, tested = 0, bad = 0;
    /* quotients exactly at the rounding boundary of zero: |x| / scale = 2^-150
     * (ties to the even zero) and one step either side of it */
    for (int k = 1; k <= 64; ++k) {
        for (int sgn = 0; sgn < 2; ++sgn) {
            for (int d = -1; d <= 1; ++d) {
                float x = ffrom((uint32_t)k);                          /* k * 2^-149 */
                float m = ldexpf(448.0f * (float)k, 1);                /* scale = 2k: x / scale = 2^-150 */
                m = ffrom(fbits(m) + (uint32_t)d);
                if (sgn) x = -x;
                float s = scale_of(m);
                volatile float qd = x / s;
                uint8_t want = encode(qd), got = code_product(x, s);
                ++tested;
                if (want != got) {
                    if (bad < 8) printf("tie x=%a absmax=%a: division %02x, product %02x\n", x, m, want, got);
                    ++bad;
                }
            }
        }
    }
    for (long i = 0; i < n; ++i) {
        uint64_t r = next(), r2 = next();
        float x, m;
        switch (i % 6) {
        case 5: { /* a group holding an infinity or a NaN (scale not normal) */
            const uint32_t kind = (uint32_t)(r2 % 4);
            m = kind == 0 ? NAN : INFINITY;
            x = kind == 1 ? INFINITY : ffrom((uint32_t)(r & 0x7F7FFFFFu));
            if (kind == 3) x = ffrom((uint32_t)(r & 0x007FFFFFu));
            break;
        }
        case 0:   /* x a random fraction of a random absmax */
            m = ffrom((uint32_t)(r & 0x7F7FFFFFu));
            x = m * (float)((double)(r2 >> 11) / 9007199254740992.0);
            break;
        case 1:   /* x subnormal, absmax anywhere above it */
            x = ffrom((uint32_t)(r & 0x007FFFFFu) | 1u);
            m = ffrom((uint32_t)(r2 & 0x7F7FFFFFu));
            break;
        case 2: { /* quotients around the smallest subnormal, 2^-150 .. 2^-139 */
            x = ffrom((uint32_t)(r & 0x00FFFFFFu) | 1u);
            double t = ldexp(1.0 + (double)(r2 & 0xFFFFF) / 1048576.0, -150 + (int)((r2 >> 20) % 12));
            m = (float)((double)fabsf(x) / t * 448.0);
            break;
        }
        case 3: { /* quotients at the encoder's half-up mantissa boundaries */
            const double q = ldexp(1.0 + (double)(2 * (int)(r2 % 8) + 1) / 16.0, (int)((r2 >> 3) % 14) - 6);
            m = ffrom((uint32_t)((r % 200u + 20u) << 23) | (uint32_t)((r >> 8) & 0x7FFFFFu));
            float s0 = scale_of(m);
            x = (float)(q * (double)s0);
            x = ffrom(fbits(x) + (uint32_t)((int)((r2 >> 7) % 5) - 2));   /* a few ulps either side */
            if (fabsf(x) > m) m = fabsf(x);
            break;
        }
        default:  /* normal x, absmax >= |x|: every code of [2^-6, 448] */
            x = ffrom(((uint32_t)(r % 253u + 1u) << 23) | (uint32_t)(r2 & 0x7FFFFFu));
            m = fabsf(x) / (float)((double)(((r2 >> 23) & 0xFFFFFF) | 1) / 16777216.0);
            break;
        }
        if (i % 6 != 5 && (!(m == m) || isinf(m) || m < fabsf(x))) m = fabsf(x);
        if (r & (1ull << 63)) x = -x;
        /* a NaN absmax is skipped by the fold (Rust's f32::max); an infinite
         * one gives scale = inf */
        float s = m != m ? 1.0f : scale_of(m);
        volatile float qd = x / s;
        uint8_t want = encode(qd), got = code_product(x, s);
        ++tested;
        if (want != got) {
            if (bad < 8) printf("x=%a absmax=%a: division %02x, product %02x\n", x, m, want, got);
            ++bad;
        }
    }
    printf("fp8 quotient codes: %ld cases, %ld differ\n", tested, bad);
    return bad != 0;
}
