// Warm-tier KV codecs of src/kv_compress.rs on the GPU, bit-exact with the
// reference's scalar arithmetic:
//   CompressedKey::compress (:79-109)   sign(k_i >= mean) bits, |k|, mean
//   CompressedValue::compress (:187-218) affine u8 codes, (max-min)/255, min
//   QjlKey::compress (:930-951)         sign(R k) bits, |k|
//   the matching decompressions (:112-127, :221-226) and approx_cos_sim /
//   approx_dot (:959-975).
//
// The reference folds each vector left to right (Iterator::sum, f32::min /
// max folds, a dot product per projected row), and the fold order fixes the
// rounding of the mean, the norm and every projection.  So one lane owns one
// row and runs the folds in that order (the value codec's min / max folds,
// whose result does not depend on how the row is split, take four lanes per
// row).  It loads its whole row itself (any
// pool dtype, dequantized by the shared page loader) with back-to-back
// 16-byte pieces, so every cache line is fetched once, and keeps it in
// registers.  Products and sums round separately (no contraction), as
// Rust's do.
//
// Rows come either from a dense [n_rows][dim] array or from pool blocks: row
// r of a block list is row r % (n_kv_heads * block_size) of the K or V slab
// of block ids[r / (n_kv_heads * block_size)], i.e. [block][head][token].
#include <hip/hip_runtime.h>

#include <cmath>

#include "../pool.hpp"
#include "codecs.hpp"
#include "compress_common.hpp"
#include "page_io.hpp"

namespace airkv {
namespace {

constexpr int kThreads = 256;
constexpr int kProjRows = 32;       // projection rows staged in LDS at a time

// One step of the NaN-ignoring folds `value.iter().fold(INF, f32::min)` and
// `fold(-INF, f32::max)` as the oracle states them (a < b ? a : b, the
// other operand on NaN).  The accumulator starts at +-inf and only ever
// takes non-NaN values, so each step is one unordered compare and a select:
// keep the accumulator when it wins strictly or x is NaN, else take x (on a
// tie, x, as `a < b ? a : b` returns b).
__device__ __forceinline__ float fold_min(float acc, float x) { return !(acc >= x) ? acc : x; }
__device__ __forceinline__ float fold_max(float acc, float x) { return !(acc <= x) ? acc : x; }

// Element offset of row r and whether its block is inside the pool.
__device__ __forceinline__ bool row_elem(const RowSource &s, int64_t r, int dim, int64_t &elem) {
    if (!s.ids) {
        elem = r * dim;
        return true;
    }
    const int64_t bi = r / s.rows_per_block;
    const int32_t blk = s.ids[bi];
    const bool ok = blk >= 0 && blk < s.num_blocks;
    elem = ((int64_t)(ok ? blk : 0) * s.rows_per_block + r % s.rows_per_block) * dim;
    return ok;
}

// Row r (or its N elements from `first`) into registers: N / 8 pieces of 8
// elements, read back to back by the same lane.  Plain (cacheable) loads: the lanes of a
// wave read 64 different rows, so each 128-byte line is needed by several
// consecutive loads of one lane and must stay in cache between them (a
// streaming load would fetch it again).  INT8 / FP8 rows are dequantized as
// q * scale with one rounding (src/kv_cache.rs:88, src/fp8.rs:263-264).
// Rows of out-of-pool blocks read as zeros (block 0's bytes when ZERO_DEAD is
// false: for callers that overwrite every output of such a row) and `live`
// is false for them.
template <int DT, int D, int N = D, bool ZERO_DEAD = true>
__device__ __forceinline__ void load_row(const RowSource &s, int64_t r, float (&x)[N], bool &live,
                                         int first = 0) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    static_assert(N % 8 == 0, "whole 8-element pieces");
    int64_t e;
    live = row_elem(s, r, D, e);
    e += first;
#pragma unroll
    for (int c = 0; c < N / 8; ++c) {
        const int64_t el = e + 8 * c;
        float v[8];
        if constexpr (DT == AIR_KV_F32) {
            const f32x4 *p = reinterpret_cast<const f32x4 *>((const float *)s.base + el);
            const f32x4 a = p[0], b = p[1];
#pragma unroll
            for (int j = 0; j < 4; ++j) { v[j] = a[j]; v[4 + j] = b[j]; }
        } else if constexpr (DT == AIR_KV_BF16) {
            const u32x4 w = *reinterpret_cast<const u32x4 *>((const uint16_t *)s.base + el);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v[2 * j] = __uint_as_float(w[j] << 16);
                v[2 * j + 1] = __uint_as_float(w[j] & 0xFFFF0000u);
            }
        } else {
            const u32x2 w = *reinterpret_cast<const u32x2 *>((const uint8_t *)s.base + el);
            const float sc = s.scales[el / s.scale_group];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t byte = (w[j >> 2] >> (8 * (j & 3))) & 0xFFu;
                const float val = DT == AIR_KV_INT8 ? (float)(int32_t)(int8_t)byte : fp8_decode(byte);
                {
#pragma clang fp contract(off)
                    v[j] = val * sc;
                }
            }
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) x[8 * c + j] = (!ZERO_DEAD || live) ? v[j] : 0.0f;
    }
}

// |k| = sqrt of the left fold of squares from -0.0 (src/kv_compress.rs:90, :938).
template <int D>
__device__ __forceinline__ float l2_norm(const float (&x)[D]) {
#pragma clang fp contract(off)
    float ss = -0.0f;
#pragma unroll
    for (int j = 0; j < D; ++j) {
        const float p = x[j] * x[j];
        ss += p;
    }
    return sqrtf(ss);
}

template <int DT, int D>
__global__ __launch_bounds__(kThreads) void key_compress_kernel(CompressArgs a) {
    constexpr int W = (D + 63) / 64;
    for (int64_t r = (int64_t)blockIdx.x * kThreads + threadIdx.x; r < a.n_rows;
         r += (int64_t)gridDim.x * kThreads) {
        float x[D];
        bool live;
        load_row<DT, D>(a.src, r, x, live);
        if (!live && a.errors && (r % a.src.rows_per_block) == 0) atomicAdd(a.errors, 1ull);
        float mean, mag;
        uint64_t bits[W];
        {
#pragma clang fp contract(off)
            float s = -0.0f;
#pragma unroll
            for (int j = 0; j < D; ++j) s += x[j];
            mean = s / (float)D;                       // (:83-87)
#pragma unroll
            for (int w = 0; w < W; ++w) {
                uint64_t word = 0;
#pragma unroll
                for (int j = 0; j < 64 && 64 * w + j < D; ++j)
                    word |= (uint64_t)(x[64 * w + j] >= mean) << j;   // (:95-100)
                bits[w] = word;
            }
            mag = l2_norm<D>(x);
        }
        if (!live) { mean = 0.0f; mag = 0.0f; for (int w = 0; w < W; ++w) bits[w] = 0; }
#pragma unroll
        for (int w = 0; w < W; ++w) a.bits[r * W + w] = bits[w];
        a.f0[r] = mag;
        a.f1[r] = mean;
    }
}

// The same codec for sources whose rows come in contiguous runs of 64 (dense
// rows, or pool blocks of n_kv_heads * block_size rows, a multiple of 64): a
// wave takes 64 consecutive rows, lane l owning row l.  Loading row by row
// sends each load instruction to 64 cache lines; here the wave reads its
// rows' bytes as consecutive 16-byte pieces (each instruction covers whole
// lines), 128 bytes of every row at a time, parks them in its own LDS slice
// (row pitch 144 bytes: the 16 rows that one read phase serves start on 16
// distinct 4-bank groups) and reads its own row back.  The folds then run in
// the reference's order on the row kept in registers in its stored form
// (f32, bf16 pairs or 1-byte codes, converted on each pass exactly as the
// per-row loader converts them).  All passes' loads are issued before the
// first staging (one memory round trip per 64 rows, not one per pass) and are
// non-temporal: each byte is read once, and these loads measured 4-5% faster
// than cached ones.
constexpr int kStagePiece = 128;                     // row bytes staged per pass
constexpr int kStagePitch = kStagePiece + 16;

template <int DT>
constexpr int elem_bytes() {
    return DT == AIR_KV_F32 ? 4 : (DT == AIR_KV_BF16 ? 2 : 1);
}

template <int DT, int D>
__global__ __launch_bounds__(kThreads) void key_compress_staged_kernel(CompressArgs a) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    constexpr int EB = elem_bytes<DT>();
    constexpr int RB = D * EB;                           // row bytes
    constexpr int PB = RB < kStagePiece ? RB : kStagePiece;
    constexpr int CPR = PB / 16;                         // 16-byte chunks per row and pass
    constexpr int W = (D + 63) / 64;
    static_assert(RB % PB == 0 && PB % 16 == 0, "whole 16-byte chunks");
    __shared__ __align__(16) uint8_t smem[kThreads / 64][64 * kStagePitch];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    uint8_t *lds = smem[wave];
    const int64_t groups = (a.n_rows + 63) / 64;
    for (int64_t g = (int64_t)blockIdx.x * (kThreads / 64) + wave; g < groups;
         g += (int64_t)gridDim.x * (kThreads / 64)) {
        const int64_t r0 = 64 * g, r = r0 + lane;
        int64_t e0;
        const bool live = row_elem(a.src, r0, D, e0);    // the 64 rows share one block
        const uint8_t *gbase = (const uint8_t *)a.src.base + e0 * EB;
        uint32_t raw[RB / 4];
        u32x4 call[RB / PB][CPR];                        // chunk k = 64 i + lane: row k / CPR
#pragma unroll
        for (int p = 0; p < RB / PB; ++p)
#pragma unroll
            for (int i = 0; i < CPR; ++i) {
                const int k = 64 * i + lane, row = k / CPR, ch = k % CPR;
                const u32x4 *src = reinterpret_cast<const u32x4 *>(gbase + (int64_t)row * RB + p * PB + 16 * ch);
                call[p][i] = live && r0 + row < a.n_rows ? __builtin_nontemporal_load(src) : u32x4{0u, 0u, 0u, 0u};
            }
#pragma unroll
        for (int p = 0; p < RB / PB; ++p) {
            const u32x4 (&c)[CPR] = call[p];
#pragma unroll
            for (int i = 0; i < CPR; ++i) {
                const int k = 64 * i + lane, row = k / CPR, ch = k % CPR;
                *reinterpret_cast<u32x4 *>(lds + row * kStagePitch + 16 * ch) = c[i];
            }
#pragma unroll
            for (int ch = 0; ch < CPR; ++ch) {
                const u32x4 v = *reinterpret_cast<const u32x4 *>(lds + lane * kStagePitch + 16 * ch);
#pragma unroll
                for (int j = 0; j < 4; ++j) raw[(p * PB + 16 * ch) / 4 + j] = v[j];
            }
            __builtin_amdgcn_sched_barrier(0);           // one pass's LDS writes and reads at a time
        }
        if (r >= a.n_rows) continue;
        if (!live && a.errors && (r % a.src.rows_per_block) == 0) atomicAdd(a.errors, 1ull);
        float sc[(EB == 1) ? D / 8 : 1];                 // scale of each 8 elements (1-byte rows;
        if constexpr (EB == 1) {                         // scale groups are multiples of 8)
            const int64_t el = e0 + (int64_t)lane * D;
#pragma unroll
            for (int j = 0; j < D / 8; ++j) sc[j] = live ? a.src.scales[(el + 8 * j) / a.src.scale_group] : 0.0f;
        }
        auto xv = [&](int j) -> float {
            if constexpr (DT == AIR_KV_F32) {
                return __uint_as_float(raw[j]);
            } else if constexpr (DT == AIR_KV_BF16) {
                return (j & 1) ? __uint_as_float(raw[j >> 1] & 0xFFFF0000u) : __uint_as_float(raw[j >> 1] << 16);
            } else {
#pragma clang fp contract(off)
                const uint32_t byte = (raw[j >> 2] >> (8 * (j & 3))) & 0xFFu;
                const float val = DT == AIR_KV_INT8 ? (float)(int32_t)(int8_t)byte : fp8_decode(byte);
                return val * sc[j >> 3];
            }
        };
        float mean, mag;
        uint64_t bits[W];
        {
#pragma clang fp contract(off)
            float s = -0.0f, ss = -0.0f;               // both folds left to right, (:83-87), (:90)
#pragma unroll
            for (int j = 0; j < D; ++j) {
                const float x = xv(j);
                const float q = x * x;
                s += x;
                ss += q;
                // the folds are sequential: hoisting the products far ahead
                // only holds them in registers (and halves the waves per SIMD)
                if (j % 8 == 7) __builtin_amdgcn_sched_barrier(0);
            }
            mean = s / (float)D;
            mag = sqrtf(ss);
            // convert again for the sign pass rather than keep D floats live
#pragma unroll
            for (int i = 0; i < RB / 4; ++i) asm volatile("" : "+v"(raw[i]));
#pragma unroll
            for (int w = 0; w < W; ++w) {
                uint64_t word = 0;
                // bit j = (x_j >= mean) (:95-100), each 32-bit half built from
                // its top bit down: shift-or, no per-bit mask constants
#pragma unroll
                for (int h = 1; h >= 0; --h) {
                    uint32_t half = 0;
#pragma unroll
                    for (int j = 31; j >= 0; --j) {
                        const int e = 64 * w + 32 * h + j;
                        if (e < D) half = (half << 1) | (uint32_t)(xv(e) >= mean);
                        if (j % 8 == 0) __builtin_amdgcn_sched_barrier(0);
                    }
                    word = (word << 32) | half;
                }
                bits[w] = word;
            }
        }
        if (!live) { mean = 0.0f; mag = 0.0f; for (int w = 0; w < W; ++w) bits[w] = 0; }
#pragma unroll
        for (int w = 0; w < W; ++w) a.bits[r * W + w] = bits[w];
        a.f0[r] = mag;
        a.f1[r] = mean;
    }
}

// Four lanes per row, each folding a quarter: min / max need no fixed order
// across quarters.  The fold keeps the accumulator unless x <= it (x < it for
// max's mirror), so fold(L ++ R) from +inf equals fold_min(fold(L),
// fold(R)) for consecutive parts L, R -- the right part's own fold wins
// exactly when it reaches the left result, ties included -- and combining
// the quarters left to right reproduces the reference's left fold bit for
// bit (signed zeros and NaN skipping included).  A wave then reads 16 whole
// rows and writes 16 contiguous code rows.
// Row r's codes, scale and min from its quarter `part` (elements part * D / 4
// .. + D / 4) in x, held by the lane; the row's four lanes are one quad of
// the wave and call this together.  A row of an out-of-pool block (live
// false) gets zero codes, scale and min whatever x holds.
template <int D>
__device__ __forceinline__ void value_encode_row(const CompressArgs &a, int64_t r, int part,
                                                 const float (&x)[D / 4], bool live) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    constexpr int N = D / 4;
    {
        // (:198-199).  The folds' value is the row's NaN-ignoring min / max,
        // which the hardware min / max give in one instruction per element
        // once signalling NaNs are quieted (given one, they return a NaN
        // rather than the other operand); they may differ from the folds only
        // in the sign of a zero result, so rows whose min or max is zero run
        // the folds themselves.
        float lo = INFINITY, hi = -INFINITY;
#pragma unroll
        for (int j = 0; j < N; ++j) {
            const float c = __builtin_canonicalizef(x[j]);
            lo = __builtin_fminf(lo, c);
            hi = __builtin_fmaxf(hi, c);
        }
        lo = __builtin_fminf(lo, __shfl_xor(lo, 1));
        hi = __builtin_fmaxf(hi, __shfl_xor(hi, 1));
        lo = __builtin_fminf(lo, __shfl_xor(lo, 2));
        hi = __builtin_fmaxf(hi, __shfl_xor(hi, 2));
        if (lo == 0.0f || hi == 0.0f) {
            lo = INFINITY;
            hi = -INFINITY;
#pragma unroll
            for (int j = 0; j < N; ++j) {
                lo = fold_min(lo, x[j]);
                hi = fold_max(hi, x[j]);
            }
        }
        // quarters 0+1 and 2+3, then the halves: the lower part is the left
        // operand (on rows that took the hardware min / max every quarter
        // holds the same value and this changes nothing)
        float o = __shfl_xor(lo, 1);
        lo = (part & 1) ? fold_min(o, lo) : fold_min(lo, o);
        o = __shfl_xor(hi, 1);
        hi = (part & 1) ? fold_max(o, hi) : fold_max(hi, o);
        o = __shfl_xor(lo, 2);
        lo = (part & 2) ? fold_min(o, lo) : fold_min(lo, o);
        o = __shfl_xor(hi, 2);
        hi = (part & 2) ? fold_max(o, hi) : fold_max(hi, o);
        float scale;
        uint32_t q[N / 4];
        {
#pragma clang fp contract(off)
            const float range = hi - lo;
            scale = range > 0.0f ? range / 255.0f : 1.0f;   // (:201-202)
            // round((v - min) / scale) (:204-209).  The quotient is the
            // correctly rounded IEEE one either way: with y = RN(1 / scale)
            // and q0 = RN(d * y) within an ulp, one correction q0 + (d - q0 *
            // scale) * y, the remainder exact by fma, is RN(d / scale)
            // (Markstein).  That needs scale and 1 / scale normal and no
            // overflow (quotients here are at most ~255; ones that underflow
            // round to code 0 either way); other rows (a subnormal or
            // infinite scale, i.e. tiny or non-finite data) divide exactly.
            const float y = 1.0f / scale;
            if (__builtin_isnormal(scale) && __builtin_isnormal(y)) {
                // d = v - min >= 0 (or NaN) here.  max(., 0) sends NaN to 0
                // (`as u8`) and min(., 255) clamps; on [0, 255] round half away
                // from zero is the truncation of quo + (0.5 - 2^-25): the sum
                // reaches the next integer exactly when quo reaches the half
                // (ties land on it, anything below stays an ulp short), and
                // below 0.5 it stays under 1 (0.5 itself would round 0.5 - 2^-25
                // up to 1).
#pragma unroll
                for (int j4 = 0; j4 < N / 4; ++j4) {
                    uint32_t w = 0;
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const float d = x[4 * j4 + k] - lo;
                        const float q0 = d * y;
                        const float rem = __builtin_fmaf(-q0, scale, d);
                        const float quo = __builtin_fmaf(rem, y, q0);
                        const float cq = __builtin_fminf(__builtin_fmaxf(quo, 0.0f), 255.0f);
                        w |= (uint32_t)(cq + 0.49999997f) << (8 * k);
                    }
                    q[j4] = w;
                }
            } else {
#pragma unroll
                for (int j4 = 0; j4 < N / 4; ++j4) {
                    uint32_t w = 0;
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        float tq = roundf((x[4 * j4 + k] - lo) / scale);
                        tq = tq < 0.0f ? 0.0f : tq;
                        tq = tq > 255.0f ? 255.0f : tq;
                        const uint32_t c = (tq != tq) ? 0u : (uint32_t)tq;   // `as u8`: NaN -> 0
                        w |= c << (8 * k);
                    }
                    q[j4] = w;
                }
            }
        }
        if (!live) { scale = 0.0f; lo = 0.0f; for (int j = 0; j < N / 4; ++j) q[j] = 0; }
        uint8_t *dst = a.codes + r * D + part * N;
        if constexpr (N >= 16) {
#pragma unroll
            for (int j = 0; j < N / 16; ++j)
                reinterpret_cast<u32x4 *>(dst)[j] = u32x4{q[4 * j], q[4 * j + 1], q[4 * j + 2], q[4 * j + 3]};
        } else {
            *reinterpret_cast<u32x2 *>(dst) = u32x2{q[0], q[1]};
        }
        if (part == 0) {
            a.f0[r] = scale;
            a.f1[r] = lo;
        }
    }
}

// The value codec with staged loads: a wave takes 16 consecutive rows (one
// pool block's, or dense rows: contiguous either way), reads their bytes as
// consecutive 16-byte pieces (each load instruction covers whole lines;
// non-temporal, each byte is read once), parks them in its own LDS slice
// and gives lane 4 i + p quarter p of row i, converted as load_row converts
// it.  Per-row loads made each instruction touch 32 lines and use a quarter
// of each.
template <int DT, int D>
__global__ __launch_bounds__(kThreads) void value_compress_staged_kernel(CompressArgs a) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    constexpr int EB = elem_bytes<DT>();
    constexpr int RB = D * EB, QB = RB / 4;           // row and quarter-row bytes
    constexpr int PITCH = RB + 16;
    constexpr int CPL = RB / 64;                      // 16-byte pieces per lane for 16 rows
    constexpr int N = D / 4;
    if constexpr (QB % 16 != 0) {
        // quarter rows under 16 bytes (1-byte rows of 32): the per-row loader
        const int part = threadIdx.x & 3;
        for (int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x; t / 4 < a.n_rows;
             t += (int64_t)gridDim.x * kThreads) {
            const int64_t r = t / 4;
            float x[N];
            bool live;
            load_row<DT, D, N, false>(a.src, r, x, live, part * N);
            if (!live && a.errors && part == 0 && (r % a.src.rows_per_block) == 0) atomicAdd(a.errors, 1ull);
            value_encode_row<D>(a, r, part, x, live);
        }
        return;
    } else {
    __shared__ __align__(16) uint8_t smem[kThreads / 64][16 * PITCH];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    uint8_t *lds = smem[wave];
    const int row = lane >> 2, part = lane & 3;
    const int64_t groups = (a.n_rows + 15) / 16;
    for (int64_t g = (int64_t)blockIdx.x * (kThreads / 64) + wave; g < groups;
         g += (int64_t)gridDim.x * (kThreads / 64)) {
        const int64_t r0 = 16 * g, r = r0 + row;
        int64_t e0;
        const bool live = row_elem(a.src, r0, D, e0);    // the 16 rows share one block
        const uint8_t *gbase = (const uint8_t *)a.src.base + e0 * EB;
        u32x4 c[CPL];
#pragma unroll
        for (int i = 0; i < CPL; ++i) {                   // piece k = 64 i + lane: row 16 k / RB
            const int k = 64 * i + lane, kr = (16 * k) / RB, kb = (16 * k) % RB;
            const u32x4 *src = reinterpret_cast<const u32x4 *>(gbase + (int64_t)kr * RB + kb);
            c[i] = live && r0 + kr < a.n_rows ? __builtin_nontemporal_load(src) : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int k = 64 * i + lane, kr = (16 * k) / RB, kb = (16 * k) % RB;
            *reinterpret_cast<u32x4 *>(lds + kr * PITCH + kb) = c[i];
        }
        float x[N];
#pragma unroll
        for (int i = 0; i < QB / 16; ++i) {
            const u32x4 w = *reinterpret_cast<const u32x4 *>(lds + row * PITCH + part * QB + 16 * i);
            if constexpr (DT == AIR_KV_F32) {
#pragma unroll
                for (int j = 0; j < 4; ++j) x[4 * i + j] = __uint_as_float(w[j]);
            } else if constexpr (DT == AIR_KV_BF16) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    x[8 * i + 2 * j] = __uint_as_float(w[j] << 16);
                    x[8 * i + 2 * j + 1] = __uint_as_float(w[j] & 0xFFFF0000u);
                }
            } else {
                // 16 codes: elements part * N + 16 i .. + 16 of the row, their
                // group scales as load_row reads them (groups of >= 8)
                const int64_t el = e0 + (int64_t)row * D + part * N + 16 * i;
                const float s0 = live ? a.src.scales[el / a.src.scale_group] : 0.0f;
                const float s1 = live ? a.src.scales[(el + 8) / a.src.scale_group] : 0.0f;
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const uint32_t byte = (w[j >> 2] >> (8 * (j & 3))) & 0xFFu;
                    const float val = DT == AIR_KV_INT8 ? (float)(int32_t)(int8_t)byte : fp8_decode(byte);
                    {
#pragma clang fp contract(off)
                        x[16 * i + j] = val * (j < 8 ? s0 : s1);
                    }
                }
            }
        }
        if (r >= a.n_rows) continue;          // a quad's lanes share r: whole quads leave
        if (!live && a.errors && part == 0 && (r % a.src.rows_per_block) == 0) atomicAdd(a.errors, 1ull);
        value_encode_row<D>(a, r, part, x, live);
    }
    }
}

template <int DT, int D>
__global__ __launch_bounds__(kThreads) void qjl_compress_kernel(CompressArgs a) {
    __shared__ __align__(16) float proj[kProjRows * D];
    const int m = a.proj_dim, W = (m + 63) / 64;
    // every thread runs the same number of iterations (the projection rows
    // are staged with barriers); rows past n_rows compute on zeros and store
    // nothing
    for (int64_t base = (int64_t)blockIdx.x * kThreads; base < a.n_rows; base += (int64_t)gridDim.x * kThreads) {
        const int64_t r = base + threadIdx.x;
        const bool own = r < a.n_rows;
        float x[D];
        bool live = false;
        if (own) load_row<DT, D>(a.src, r, x, live);
        else
#pragma unroll
            for (int j = 0; j < D; ++j) x[j] = 0.0f;
        if (own && !live && a.errors && (r % a.src.rows_per_block) == 0) atomicAdd(a.errors, 1ull);
        uint64_t word = 0;
        for (int i0 = 0; i0 < m; i0 += kProjRows) {
            // rows i0 .. i0 + 31 of R (zeros past m)
            __syncthreads();
            for (int e = threadIdx.x; e < kProjRows * D; e += kThreads) {
                const int i = i0 + e / D;
                proj[e] = i < m ? a.proj[(int64_t)i * D + e % D] : 0.0f;
            }
            __syncthreads();
            for (int ii = 0; ii < kProjRows && i0 + ii < m; ++ii) {
                float dot = -0.0f;
                {
#pragma clang fp contract(off)
#pragma unroll
                    for (int j = 0; j < D; ++j) {        // (:941-943)
                        const float p = proj[ii * D + j] * x[j];
                        dot += p;
                    }
                }
                const int i = i0 + ii;
                word |= (uint64_t)(dot > 0.0f) << (i & 63);   // (:945-947)
                if ((i & 63) == 63 || i == m - 1) {
                    if (own) a.bits[r * W + (i >> 6)] = live ? word : 0ull;
                    word = 0;
                }
            }
        }
        if (own) a.f0[r] = live ? l2_norm<D>(x) : 0.0f;
    }
}

// CompressedKey::decompress (:112-127): sign * (|k| / sqrt(dim)) + mean, one
// thread per element.
__global__ __launch_bounds__(kThreads) void key_decompress_kernel(DecompressArgs a) {
    const int64_t n = a.n_rows * a.dim;
    const int W = (a.dim + 63) / 64;
    for (int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x; idx < n;
         idx += (int64_t)gridDim.x * kThreads) {
#pragma clang fp contract(off)
        const int64_t r = idx / a.dim;
        const int j = (int)(idx % a.dim);
        const float scale = a.f0[r] / sqrtf((float)a.dim);
        const float sign = ((a.bits[r * W + (j >> 6)] >> (j & 63)) & 1ull) ? 1.0f : -1.0f;
        const float p = sign * scale;
        a.out[idx] = p + a.f1[r];
    }
}

// CompressedValue::decompress (:221-226): q * scale + min.
__global__ __launch_bounds__(kThreads) void value_decompress_kernel(DecompressArgs a) {
    const int64_t n = a.n_rows * a.dim;
    for (int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x; idx < n;
         idx += (int64_t)gridDim.x * kThreads) {
#pragma clang fp contract(off)
        const int64_t r = idx / a.dim;
        const float p = (float)a.codes[idx] * a.f0[r];
        a.out[idx] = p + a.f1[r];
    }
}

// approx_cos_sim / approx_dot (:959-975) of one query against n keys: the
// Hamming distance indexes the host-computed table cos(pi * h / m).
__global__ __launch_bounds__(kThreads) void qjl_scores_kernel(QjlScoreArgs a) {
    const int W = (a.proj_dim + 63) / 64;
    for (int64_t k = (int64_t)blockIdx.x * kThreads + threadIdx.x; k < a.n_keys;
         k += (int64_t)gridDim.x * kThreads) {
#pragma clang fp contract(off)
        int ham = 0;
        for (int w = 0; w < W; ++w) ham += __popcll(a.key_bits[k * W + w] ^ a.query_bits[w]);
        const float c = a.cos_table[ham];
        if (a.cos_out) a.cos_out[k] = c;
        if (a.dot_out) {
            const float t = c * a.key_magnitude[k];
            a.dot_out[k] = t * a.query_magnitude;
        }
    }
}

int grid_for(int64_t work, int per_block, int cus) {
    const int64_t b = (work + per_block - 1) / per_block;
    const int64_t cap = (int64_t)cus * 16;
    return (int)(b < 1 ? 1 : (b > cap ? cap : b));
}

#define AIRKV_LAUNCH_DT(KERNEL, D, a, s, grid)                                                     \
    switch ((a).src_dtype) {                                                                       \
    case AIR_KV_F32: hipLaunchKernelGGL((KERNEL<AIR_KV_F32, D>), grid, dim3(kThreads), 0, s, a); break; \
    case AIR_KV_BF16: hipLaunchKernelGGL((KERNEL<AIR_KV_BF16, D>), grid, dim3(kThreads), 0, s, a); break; \
    case AIR_KV_INT8: hipLaunchKernelGGL((KERNEL<AIR_KV_INT8, D>), grid, dim3(kThreads), 0, s, a); break; \
    default: hipLaunchKernelGGL((KERNEL<AIR_KV_FP8, D>), grid, dim3(kThreads), 0, s, a); break;   \
    }

#define AIRKV_LAUNCH_D(KERNEL, a, s, grid)                       \
    switch ((a).dim) {                                           \
    case 32: AIRKV_LAUNCH_DT(KERNEL, 32, a, s, grid) break;      \
    case 64: AIRKV_LAUNCH_DT(KERNEL, 64, a, s, grid) break;      \
    default: AIRKV_LAUNCH_DT(KERNEL, 128, a, s, grid) break;     \
    }

}  // namespace

bool compress_dim_supported(int dim) { return dim == 32 || dim == 64 || dim == 128; }

hipError_t launch_compress(CompressKind kind, const CompressArgs &a, int cus, hipStream_t s) {
    if (a.n_rows == 0) return hipSuccess;
    const dim3 grid((unsigned)grid_for(a.n_rows, kThreads, cus));
    // rows in contiguous runs of 64: the staged key codec, one wave per 64 rows
    const bool runs64 = !a.src.ids || a.src.rows_per_block % 64 == 0;
    if (kind == CompressKind::Key && runs64) {
        const dim3 g((unsigned)grid_for((a.n_rows + 63) / 64 * 64, kThreads, cus));
        AIRKV_LAUNCH_D(key_compress_staged_kernel, a, s, g)
        return hipGetLastError();
    }
    if (kind == CompressKind::Value) {
        // one wave per 16 rows (a pool block holds n_kv_heads * block_size
        // rows, a multiple of 16, so they share one block)
        const dim3 g((unsigned)grid_for((a.n_rows + 15) / 16 * 64, kThreads, cus));
        AIRKV_LAUNCH_D(value_compress_staged_kernel, a, s, g)
        return hipGetLastError();
    }
    switch (kind) {
    case CompressKind::Key: AIRKV_LAUNCH_D(key_compress_kernel, a, s, grid) break;
    default: AIRKV_LAUNCH_D(qjl_compress_kernel, a, s, grid) break;
    }
    return hipGetLastError();
}

hipError_t launch_decompress(bool key, const DecompressArgs &a, int cus, hipStream_t s) {
    const int64_t n = a.n_rows * a.dim;
    if (n == 0) return hipSuccess;
    const dim3 grid((unsigned)grid_for(n, kThreads, cus));
    if (key) hipLaunchKernelGGL(key_decompress_kernel, grid, dim3(kThreads), 0, s, a);
    else hipLaunchKernelGGL(value_decompress_kernel, grid, dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_qjl_scores(const QjlScoreArgs &a, int cus, hipStream_t s) {
    if (a.n_keys == 0) return hipSuccess;
    const dim3 grid((unsigned)grid_for(a.n_keys, kThreads, cus));
    hipLaunchKernelGGL(qjl_scores_kernel, grid, dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

}  // namespace airkv
