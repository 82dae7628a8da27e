// Paged decode attention on the matrix cores (bf16 pages, head_dim 128).
//
// Work distribution.  The cached tokens of the batch are cut into 16-token
// tiles, numbered sequence after sequence (tile t of the batch belongs to the
// sequence b with prefix[b] <= t < prefix[b + 1], prefix[b] = tiles of the
// sequences before b).  For each kv head these tiles are split into `slices`
// equal contiguous ranges of `chunk` tiles, one per wave, so every wave
// streams the same number of K/V bytes whatever the length mix of the batch
// (a grid of per-sequence partitions leaves the GPU waiting on the longest
// sequences).  A slice may end inside a sequence and continue into the next:
// at every sequence boundary the wave emits the (max, sum, O) of the piece it
// holds.  The pieces of sequence b come from slices w0(b) = prefix[b] / chunk
// .. w1(b) = (prefix[b + 1] - 1) / chunk and are stored at slots b + w, which
// never collide across sequences because w0(b + 1) >= w1(b).  The chunk is
// widened when needed so that no sequence has more than max_splits pieces
// (configs[3]'s bound: split-K over up to 64 partitions).  A sequence that
// lies in one slice is normalised and written by that wave; the others are
// combined by decode_merge_kernel by log-sum-exp (src/flash_decode.rs:114-142).
//
// Per 16-token tile, on the matrix cores:
//   S  = K . Q^T   v_mfma_f32_16x16x32_bf16, M = 16 tokens, N = 16 heads (G
//                  used), K = head_dim in steps of 32.  K is loaded straight
//                  from its page in the A-operand layout (row = lane % 16,
//                  16 contiguous bytes per lane); Q^T stays in registers.
//   P  = exp2(S * scale * log2 e - m)     online softmax per head; the max is
//                  shared by the four lanes holding a head's 16 tokens.
//   O^T += V^T . P^T   v_mfma_f32_16x16x16bf16_1k, M = 16 head_dim columns,
//                  N = 16 heads, K = 16 tokens.  P^T is already in the B-operand
//                  layout where the QK product left it (lane = head + 16 * token
//                  group), so it never moves; it is split into hi + lo bf16
//                  halves (two MFMAs) so the probabilities keep ~16 mantissa
//                  bits.  V needs head_dim-major operands, so each wave stages
//                  its V tile in LDS (row pitch 264 B: the four token groups
//                  land on different banks) and reads it back transposed.
//
// Each wave resolves the sequence, block id and valid token count of 64 of its
// tiles at once (lane k: tile k), then takes them with readlane, so tile
// addresses live in scalar registers and no load waits on another.  By
// default a wave loads a tile and then computes it, with nothing else in
// flight: the other waves of its SIMD overlap its loads, and for these
// scattered page reads that measured faster than keeping one or two more
// tiles in flight per wave (a ring of register sets, a build-time knob).
#include <hip/hip_runtime.h>

#include <cmath>

#include "../host/status.hpp"
#include "../pool.hpp"
#include "codecs.hpp"
#include "decode_common.hpp"
#include "page_io.hpp"

namespace airkv {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxBatch = 4096;            // sequences per launch (the host splits larger batches)
constexpr int kMinChunk = 4;               // tiles per slice at least

// Build-time tuning knobs (defaults are the shipped configuration).
#ifndef AIRKV_DECODE_WAVES_PER_EU
#define AIRKV_DECODE_WAVES_PER_EU 2        // register budget: waves per SIMD, bf16 pages
#endif
#ifndef AIRKV_DECODE_QWAVES_PER_EU
#define AIRKV_DECODE_QWAVES_PER_EU 3       // the same for int8 pages (fewer raw registers per tile)
#endif
#ifndef AIRKV_DECODE_FP8_WAVES_PER_EU
#define AIRKV_DECODE_FP8_WAVES_PER_EU 3    // fp8 pages
#endif
#ifndef AIRKV_DECODE_RING
#define AIRKV_DECODE_RING 1               // tile register sets per wave, bf16 pages (ring - 1 in flight)
#endif
#ifndef AIRKV_DECODE_QRING
#define AIRKV_DECODE_QRING 1              // the same for 1-byte pages
#endif
#ifndef AIRKV_DECODE_NT_LOADS
#define AIRKV_DECODE_NT_LOADS 1            // non-temporal K/V loads, bf16 pages
#endif
#ifndef AIRKV_DECODE_K16
#define AIRKV_DECODE_K16 1                 // 1-byte pages: K as 16-byte loads re-paired across lanes (else 8-byte loads)
#endif
#ifndef AIRKV_DECODE_QNT_LOADS
#define AIRKV_DECODE_QNT_LOADS 1           // 1-byte pages: every K/V/scale load nt (else the per-stream policy below)
#endif

// Buffer descriptor word 3 for raw (untyped) buffer access on gfx9-class
// GPUs, and the cache-policy bits of the K/V loads: 2 = nt, streaming.  K/V
// bytes are read exactly once, and on MI355X random 4 KB page reads run at
// ~6.85 TB/s with nt against ~6.05 TB/s without (measured); the bf16 decode
// keeps that ratio (c2 105 against 118 us).
constexpr int kBufferWord3 = 0x00020000;
constexpr int kLoadAux = AIRKV_DECODE_NT_LOADS ? 2 : 0;

// 1-byte pages: every code and scale load is nt now that each load
// instruction reads whole rows.  With instructions that read half of every
// row, the policy had to be chosen per stream (nt scale loads 124.0 -> 120.6
// us at c3, 371.2 -> 360.7 us at c4; nt fp8 K loads gave c4 367.7 us, nt V
// loads 125.0 and 413 us), and a probe reading scattered 2 KB pages that way
// ran at 5.1-5.3 TB/s with nt against 6.0 without.
template <int DT> constexpr int k_code_aux() { return (AIRKV_DECODE_QNT_LOADS || DT == AIR_KV_INT8) ? 2 : 0; }
constexpr int kVCodeAux = AIRKV_DECODE_QNT_LOADS ? 2 : 0;
constexpr int kScaleAux = 2;

__device__ __forceinline__ f32x4 mfma_qk(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma_pv(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a),
                                                     __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
}

// bf16 bits (round to nearest even) of a finite f32.
__device__ __forceinline__ uint32_t bf16_bits(float x) {
    const uint32_t u = __float_as_uint(x);
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// x = hi + lo with both halves bf16: hi carries 8 significant bits, lo the next 8.
__device__ __forceinline__ void split_bf16(float x, uint32_t &hi, uint32_t &lo) {
    hi = bf16_bits(x);
    lo = bf16_bits(x - __uint_as_float(hi << 16));
}

// The same for a pair of finite values, packed (element 0 in the low half),
// with the hardware round-to-nearest-even conversions.
__device__ __forceinline__ void split_pair(float x, float y, uint32_t &hi, uint32_t &lo) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    const f32x2 v = {x, y};
    const bf16x2 h = __builtin_convertvector(v, bf16x2);
    const f32x2 r = v - __builtin_convertvector(h, f32x2);
    hi = __builtin_bit_cast(uint32_t, h);
    lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(r, bf16x2));
}

__device__ __forceinline__ uint32_t bf16_pair(float x, float y) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{x, y}), bf16x2));
}

// Reductions across the lanes 16 and 32 apart with the gfx950 lane-swap
// instructions instead of LDS permutes.  permlane16_swap(v, v) returns
// {v[l & ~16], v[l | 16]} in lane l, permlane32_swap(v, v) returns
// {v[l & ~32], v[l | 32]}: the two halves of each pair, in the same order
// in both lanes, so both lanes compute the same bits.
__device__ __forceinline__ float max_x16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_x32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_x16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_x32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Register-pair transposes: afterwards x_b in lane l holds what x_c held in
// lane l', where c is lane l's bit 3 (bit 5) and l' is l with that bit set
// to b.  Bit 3: DPP row_ror:8 (lane l ^ 8 within each row of 16), written
// only to the lanes whose bit 3 differs from the register index (bank masks
// 0xC: lanes 8..15 of each row, 0x3: lanes 0..7).  Bit 5: the lane swap
// across the wave's halves.
__device__ __forceinline__ void swap_lane_bit3(u32x4 &x0, u32x4 &x1) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int a = (int)x0[j], b = (int)x1[j];
        x0[j] = (uint32_t)__builtin_amdgcn_update_dpp(a, b, 0x128, 0xF, 0xC, false);
        x1[j] = (uint32_t)__builtin_amdgcn_update_dpp(b, a, 0x128, 0xF, 0x3, false);
    }
}
__device__ __forceinline__ void swap_lane_bit5(u32x4 &x0, u32x4 &x1) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const auto r = __builtin_amdgcn_permlane32_swap(x0[j], x1[j], false, false);
        x0[j] = r[0];
        x1[j] = r[1];
    }
}

__device__ __forceinline__ void store_out(const DecodeArgs &a, int64_t idx, float v) {
    if (a.out_dtype == AIR_KV_F32) ((float *)a.out)[idx] = v;
    else ((uint16_t *)a.out)[idx] = bf16_rne(v);
}

// Four consecutive outputs (idx a multiple of 4).
__device__ __forceinline__ void store_out4(const DecodeArgs &a, int64_t idx, f32x4 v) {
    if (a.out_dtype == AIR_KV_F32) {
        *reinterpret_cast<f32x4 *>((float *)a.out + idx) = v;
    } else {
        const u32x2 w = {(uint32_t)bf16_rne(v[0]) | ((uint32_t)bf16_rne(v[1]) << 16),
                         (uint32_t)bf16_rne(v[2]) | ((uint32_t)bf16_rne(v[3]) << 16)};
        *reinterpret_cast<u32x2 *>((uint16_t *)a.out + idx) = w;
    }
}

__device__ __forceinline__ int64_t clamp_len(int64_t len, int64_t max_len) {
    return len < 0 ? 0 : (len > max_len ? max_len : len);
}

// Tiles per slice: an equal share of `total`, at least kMinChunk, and large
// enough that no sequence is cut into more than max_splits pieces.  A
// sequence of T tiles starting anywhere meets at most ceil((T - 1) / chunk) +
// 1 slices, so chunk >= ceil((T - 1) / (max_splits - 1)) for the longest
// sequence (tmax tiles) bounds every one; max_splits 1 leaves one slice per
// kv head.
__device__ __forceinline__ int slice_chunk(int total, int slices, int tmax, int max_splits) {
    int c = (total + slices - 1) / slices;
    c = c < kMinChunk ? kMinChunk : c;
    if (max_splits <= 1) return c > total ? c : total;
    const int cs = (tmax - 1 + max_splits - 2) / (max_splits - 1);
    return c > cs ? c : cs;
}

// pre[b] = tiles (ceil(len / 16), len clamped to [0, max_blocks * BS]) of the
// sequences before b, for b = 0..batch, in LDS, and pre[B + 1] = the most
// tiles of one sequence.  All threads take part.
template <int BS>
// long_seq (optional, B bits, zero on entry): bit b set when sequence b is
// longer than its table.
__device__ void tile_prefix(const DecodeArgs &a, int32_t *pre, int32_t *wsum, uint32_t *long_seq = nullptr) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int B = a.batch;
    const int64_t max_len = (int64_t)a.max_blocks * BS;
    int tmax = 0;
    for (int b = tid; b < B; b += kThreads) {
        const int32_t len = a.lens[b];
        const int32_t t = (int32_t)((clamp_len(len, max_len) + 15) / 16);
        pre[b + 1] = t;
        tmax = t > tmax ? t : tmax;
        if (long_seq && len > max_len) atomicOr(&long_seq[b >> 5], 1u << (b & 31));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const int y = __shfl_xor(tmax, o);
        tmax = y > tmax ? y : tmax;
    }
    if (lane == 0) wsum[wave] = tmax;
    if (tid == 0) pre[0] = 0;
    __syncthreads();
    if (tid == 0) {
        int m = wsum[0];
        for (int w = 1; w < kWaves; ++w) m = wsum[w] > m ? wsum[w] : m;
        pre[B + 1] = m;
    }
    __syncthreads();
    // each thread scans a run of `per` entries; runs are chained by a
    // wave-level then a workgroup-level exclusive scan of the run sums
    const int per = (B + kThreads - 1) / kThreads;
    const int lo = 1 + tid * per;
    const int hi = lo + per < B + 1 ? lo + per : B + 1;
    int sum = 0;
    for (int i = lo; i < hi; ++i) sum += pre[i];
    int incl = sum;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(incl, o);
        if (lane >= o) incl += y;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    int run = incl - sum;
    for (int w = 0; w < wave; ++w) run += wsum[w];
    for (int i = lo; i < hi; ++i) {
        run += pre[i];
        pre[i] = run;
    }
    __syncthreads();
}

// The sequence holding tile t (0 <= t < pre[B]): the b with pre[b] <= t < pre[b + 1].
// The loop count depends on B only, so the lanes of a wave stay converged.
__device__ __forceinline__ int seq_of_tile(const int32_t *pre, int B, int t) {
    int lo = 0, hi = B;
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (pre[mid] <= t) lo = mid;
        else hi = mid;
    }
    return lo;
}

// Raw registers of one 16-token tile as loaded, before any conversion.
// bf16 pages: K in the MFMA A-operand layout (lane: row r16, head_dim 8*g4 +
// 32*ks .. +8 for step ks) and four 16-byte V chunks.  1-byte pages (int8
// Q8_0 codes, fp8): K in the same layout (8 codes per step: k-step ks is
// head_dim 32*ks .. +32, one scale group), the lane's own K row scale (row
// r16, head_dim 32*g4), and 32 contiguous codes -- one scale group -- of one
// V row with its scale.  (1-byte k16 and v hold the whole-row load order
// until compute_tile transposes them into this layout.)
template <int DT> struct Tile {
    u32x2 k[4];          // 8-byte K loads: step ks
    u32x4 k16[2];        // 16-byte K loads: head_dim 64*m + 16*g4 .. +16
    u32x4 v[2];
    uint32_t ks, vs;
    // fused-append kernels, a sequence's last tile: the new token's codes
    // (lanes 0..15: K head_dim 8*lane .. +8, lanes 16..31: V head_dim
    // 8*(lane - 16) .. +8) and the scale of the lane's group
    uint32_t qlo, qhi;
    float qs;
};
template <> struct Tile<AIR_KV_BF16> {
    u32x4 k[4], v[4];
    // fused-append kernels, a sequence's last tile: the new token's f32 K
    // (this lane's head_dim 32*ks + 8*g4 .. +8 as kn[2ks], kn[2ks + 1]) and
    // V (head_dim vcol .. +8) rows
    f32x4 kn[8], vn[2];
};

// Four 1-byte codes of one word times `s`, as two bf16 pairs.  The f32 value
// is the reference's dequantized cache element, q as f32 * scale
// (src/kv_cache.rs:78-92) or to_f32(code) * scale (src/fp8.rs:263-264),
// computed with one rounding; it is then rounded to bf16 for the matrix
// cores.  int8: the code is biased to an unsigned byte (x ^ 0x80 = q + 128)
// so one byte-to-float conversion applies, and fma(q + 128, s, -128 s) is
// code * s with a single rounding.  fp8: the hardware converts the OCP E4M3
// encoding, which agrees with the reference decoder on every code its
// encoder emits (zero exponent fields only as +-0, 0xFF never; 0x7F is NaN
// in both).
template <int DT>
__device__ __forceinline__ u32x2 dequant4(uint32_t w, float s) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    f32x2 lo, hi;
    if constexpr (DT == AIR_KV_INT8) {
        const uint32_t u = w ^ 0x80808080u;
        const float off = -128.0f * s;
        lo = f32x2{__builtin_fmaf((float)(u & 0xFFu), s, off), __builtin_fmaf((float)((u >> 8) & 0xFFu), s, off)};
        hi = f32x2{__builtin_fmaf((float)((u >> 16) & 0xFFu), s, off), __builtin_fmaf((float)(u >> 24), s, off)};
    } else {
        lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false) * s;
        hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true) * s;
    }
    return u32x2{__builtin_bit_cast(uint32_t, __builtin_convertvector(lo, bf16x2)),
                 __builtin_bit_cast(uint32_t, __builtin_convertvector(hi, bf16x2))};
}

// Eight 1-byte K codes as four bf16 pairs, exactly (element 0 in the low
// half of word 0).  int8: the code biased to an unsigned byte, q + 128 (x ^
// 0x80), whose value 1..255 bf16 holds exactly; the bias is taken out of the
// product by starting the accumulator at -128 * (sum of the query's elements
// over the step).  fp8: the hardware's OCP E4M3 -> bf16 conversion at unit
// scale, exact for every code the reference encoder emits (every E4M3 value
// is a bf16 value; zero exponent fields only as +-0, 0xFF never).
template <int DT>
__device__ __forceinline__ u32x4 codes_bf16(u32x2 w) {
    if constexpr (DT == AIR_KV_INT8) {
        const uint32_t u0 = w[0] ^ 0x80808080u, u1 = w[1] ^ 0x80808080u;
        return u32x4{bf16_pair((float)(u0 & 0xFFu), (float)((u0 >> 8) & 0xFFu)),
                     bf16_pair((float)((u0 >> 16) & 0xFFu), (float)(u0 >> 24)),
                     bf16_pair((float)(u1 & 0xFFu), (float)((u1 >> 8) & 0xFFu)),
                     bf16_pair((float)((u1 >> 16) & 0xFFu), (float)(u1 >> 24))};
    } else {
        return u32x4{__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w[0], 1.0f, false)),
                     __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w[0], 1.0f, true)),
                     __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w[1], 1.0f, false)),
                     __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w[1], 1.0f, true))};
    }
}

// Waves per SIMD the slice kernel is built for (its register budget) and
// launched with (slices per kv head).
constexpr int waves_per_simd(int dt) {
    return dt == AIR_KV_BF16  ? AIRKV_DECODE_WAVES_PER_EU
           : dt == AIR_KV_FP8 ? AIRKV_DECODE_FP8_WAVES_PER_EU
                              : AIRKV_DECODE_QWAVES_PER_EU;
}

// The register budget of a build: every query dtype of a page dtype has the
// same one (f32 queries on 1-byte pages are rounded to bf16 once, below, so
// they carry no lo halves); the fused append on fp8 pages, whose new rows are
// quantized inside the tile loop, is built for 3 waves per SIMD (at 4 its
// encoder's temporaries spilled to scratch inside the loop).
constexpr int kernel_waves_per_simd(int dt, bool append) {
    return (append && dt == AIR_KV_FP8) ? 3 : waves_per_simd(dt);
}

// The build's waves per SIMD are its minimum and its maximum: with the
// maximum the register allocator plans for that occupancy, not a higher one
// the launch never uses (c4 fp8 355 against 362-364 us, same box, two runs
// each; c2 104.1-104.4 against 104.7-105.0; c3 and c5 unchanged).
// APPEND (bf16 pages): the launch also writes each sequence's new token,
// a.k_new / a.v_new, as described at the fused append below.
template <int D, int BS, bool QF32, int DT, bool APPEND>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(kernel_waves_per_simd(DT, APPEND), kernel_waves_per_simd(DT, APPEND))))
void decode_mfma_kernel(DecodeArgs a) {
    static_assert(D == 128, "lane mappings assume head_dim 128");
    constexpr bool QUANT = DT != AIR_KV_BF16;
    static_assert(!(APPEND && QUANT && !AIRKV_DECODE_K16), "the fused 1-byte append fills 16-byte K loads");
    constexpr int EB = QUANT ? 1 : 2;         // bytes per cache element
    constexpr int KSTEPS = D / 32;            // QK k-steps
    constexpr int DTILES = D / 16;            // PV output tiles along head_dim
    // V tile layout in LDS: row pitch 320 bytes, and the 8-byte column chunks
    // of row r stored at chunk ^ (r & 7).  With it the transposing reads and
    // both store patterns (1-byte and bf16 pages) touch every bank once per
    // cycle (a 288-byte pitch without the swizzle left the 1-byte stores
    // 4-way conflicted).
    constexpr int PITCH = D + 32;
    constexpr int VTILE = 16 * PITCH;         // bf16 elements per wave's V tile
    static_assert(BS % 16 == 0, "a 16-token tile must not straddle pages");
    __shared__ int32_t s_pre[kMaxBatch + 2];
    __shared__ int32_t s_wsum[kWaves];
    __shared__ __align__(16) uint16_t s_v[kWaves * VTILE];
    // 1-byte pages: the tile's K scales [k-step][token] per wave (lane (r16,
    // g4) holds row r16's scale of step g4; the S rows it needs are 4*g4..+3)
    __shared__ __align__(16) float s_ksc[kWaves][QUANT ? 64 : 4];

    // fused append: sequences longer than their table (they append nothing)
    __shared__ uint32_t s_long[APPEND ? kMaxBatch / 32 : 1];
    if constexpr (APPEND) {
        for (int i = threadIdx.x; i < (a.batch + 31) / 32; i += kThreads) s_long[i] = 0;
        __syncthreads();
        tile_prefix<BS>(a, s_pre, s_wsum, s_long);
    } else {
        tile_prefix<BS>(a, s_pre, s_wsum);
    }
    const int B = a.batch;
    const int total = s_pre[B];
    const int chunk = slice_chunk(total, a.slices, s_pre[B + 1], a.max_splits);
    if (blockIdx.x == 0) {                     // for the merge kernel: prefix, then the chunk
        for (int i = threadIdx.x; i <= B; i += kThreads) a.prefix[i] = s_pre[i];
        if (threadIdx.x == 0) a.prefix[B + 1] = chunk;
    }

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: scalar loop control
    const int g4 = lane >> 4, r16 = lane & 15;
    const int G = a.group;
    // Consecutive waves take consecutive kv heads of one slice: their pages
    // are neighbours within the same blocks.
    const int gw = blockIdx.x * kWaves + wave;
    const int kh = gw % a.n_kv_heads, w = gw / a.n_kv_heads;
    if (w >= a.slices || (int64_t)w * chunk >= total) return;
    const int lo = w * chunk;
    const int hi = total - lo < chunk ? total : lo + chunk;
    const int64_t max_len = (int64_t)a.max_blocks * BS;

    // Per 64-tile window starting at tile c0, lane k describes tile c0 + k:
    // its sequence, tile index within the sequence, block id and valid tokens.
    int32_t tbl = 0, seq_l = 0, j_l = 0, nv_l = 0;
    uint64_t first_m = 0, last_m = 0;      // tile starts / ends a piece
    uint64_t seqend_m = 0;                 // tile holds its sequence's last token
    auto load_window = [&](int c0) {
        const int t = c0 + lane < hi ? c0 + lane : hi - 1;
        const int bq = seq_of_tile(s_pre, B, t);
        const int j = t - s_pre[bq];
        const int64_t len = clamp_len(a.lens[bq], max_len);
        tbl = a.tables[(int64_t)bq * a.max_blocks + (16 * j) / BS];
        seq_l = bq;
        j_l = j;
        const int64_t rest = len - 16 * (int64_t)j;
        nv_l = rest < 16 ? (int)rest : 16;
        const bool valid = c0 + lane < hi;
        first_m = __ballot(valid && (t == lo || j == 0));
        last_m = __ballot(valid && (t + 1 == hi || t + 1 == s_pre[bq + 1]));
        if constexpr (APPEND)
            seqend_m = __ballot(valid && t + 1 == s_pre[bq + 1] && !((s_long[bq >> 5] >> (bq & 31)) & 1));
    };

    // ---- Q^T in the B-operand layout.  The QK contraction runs over head_dim
    // as d = 32*ks + 8*g4 + j: lane (r16, g4) holds 8 consecutive elements
    // of K row r16 per step (16 bytes of bf16 pages, 8 codes of 1-byte
    // pages), and step ks is head_dim 32*ks .. +32, one scale group of
    // 1-byte pages.
    // The loads go through a buffer descriptor that spans exactly the group's
    // G query rows: lanes of heads >= G fall outside it and read zeros, so
    // there is no branch (a branch around a load inside the tile loop costs
    // the compiler ~50 extra registers).
    u32x4 qhi[KSTEPS], qlo[KSTEPS];
    float qbias[KSTEPS];                     // int8 pages: -128 * sum of q over step ks (head r16)
    auto load_q = [&](int bq) {
        constexpr int QB = QF32 ? 4 : 2;
        const char *qg = (const char *)a.q + ((int64_t)bq * a.n_q_heads + kh * G) * D * QB;
        const __amdgpu_buffer_rsrc_t rq =
            __builtin_amdgcn_make_buffer_rsrc((void *)qg, (short)0, G * D * QB, kBufferWord3);
        constexpr int step = 32 * QB;
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
            // the step's element order (see the K operands): 1-byte pages
            // with 16-byte K loads hold, in slot g4, head_dim 32*ks +
            // 16*(g4 & 1) + 8*(g4 >> 1) .. +8
            const int qoff = (QUANT && AIRKV_DECODE_K16) ? (r16 * D + 16 * (g4 & 1) + 8 * (g4 >> 1)) * QB
                                                         : (r16 * D + 8 * g4) * QB;
            if constexpr (QF32 && QUANT) {
                // 1-byte pages: the query rounded to bf16 once.  Its error
                // (2^-9 relative per element) is an order below the codes' own
                // quantization and the 2e-2 tolerance of these pools; the hi
                // + lo products of bf16 pages would cost a second product per
                // k-step and a third of the waves.
                const u32x4 x0 = __builtin_amdgcn_raw_buffer_load_b128(rq, qoff + step * ks, 0, 0);
                const u32x4 x1 = __builtin_amdgcn_raw_buffer_load_b128(rq, qoff + step * ks + 16, 0, 0);
                qhi[ks] = u32x4{bf16_bits(__uint_as_float(x0[0])) | (bf16_bits(__uint_as_float(x0[1])) << 16),
                                bf16_bits(__uint_as_float(x0[2])) | (bf16_bits(__uint_as_float(x0[3])) << 16),
                                bf16_bits(__uint_as_float(x1[0])) | (bf16_bits(__uint_as_float(x1[1])) << 16),
                                bf16_bits(__uint_as_float(x1[2])) | (bf16_bits(__uint_as_float(x1[3])) << 16)};
                qlo[ks] = u32x4{0, 0, 0, 0};
            } else if constexpr (QF32) {
                const u32x4 x0 = __builtin_amdgcn_raw_buffer_load_b128(rq, qoff + step * ks, 0, 0);
                const u32x4 x1 = __builtin_amdgcn_raw_buffer_load_b128(rq, qoff + step * ks + 16, 0, 0);
                const uint32_t x[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
                uint32_t hh[8], ll[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) split_bf16(__uint_as_float(x[j]), hh[j], ll[j]);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    qhi[ks][j] = hh[2 * j] | (hh[2 * j + 1] << 16);
                    qlo[ks][j] = ll[2 * j] | (ll[2 * j + 1] << 16);
                }
            } else {
                qhi[ks] = __builtin_amdgcn_raw_buffer_load_b128(rq, qoff + step * ks, 0, 0);
                qlo[ks] = u32x4{0, 0, 0, 0};
            }
        }
        if constexpr (DT == AIR_KV_INT8) {
#pragma unroll
            for (int ks = 0; ks < KSTEPS; ++ks) {
                float sum = 0.0f;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    sum += __uint_as_float(qhi[ks][j] << 16) + __uint_as_float(qhi[ks][j] & 0xFFFF0000u);

                }
                sum += __shfl_xor(sum, 16);
                sum += __shfl_xor(sum, 32);
                qbias[ks] = -128.0f * sum;
            }
        }
        // Q is loaded on a branch (a new sequence), so at the QK products the
        // compiler waits for it as if it were in flight, and vector loads
        // retire in order: every tile waits there for most of the next
        // tile's page loads.  Consuming Q here instead (an empty asm use)
        // removes that wait and measured slower on every page dtype: fewer
        // loads in flight is faster for these scattered page reads.
    };

    f32x4 acc[DTILES];
    float m_run = -INFINITY, l_run = 0.0f;

    const char *kp = (const char *)a.k_pages;
    const char *vp = (const char *)a.v_pages;
    uint16_t *sv = s_v + wave * VTILE;
    // Lane offsets inside a tile (loop invariant).  bf16: K as the A operand,
    // V as 16-byte chunks of rows lane / 16 + 4 * v.  1-byte: compute_tile
    // works on K row r16 and V row lane / 4, 32 codes from column 32 * g4
    // (K) or 32 * (lane % 4) (V), but each 16-byte load instruction reads
    // eight whole 128-byte rows: K load m gives lane l row 8m + (l & 7),
    // 16-byte chunk 4 bit3(l) + 2 bit5(l) + bit4(l); V load i row
    // 8i + ((l >> 2) & 7), chunk 4 bit1(l) + 2 bit0(l) + bit5(l).  One
    // transpose of lane bit 3 (K) or 5 (V) with the load index turns that
    // into the layout above.  (Loads reading half of every row they touch
    // ran scattered 2 KB pages at 5.1-5.3 TB/s with the non-temporal bit,
    // against 6.7-6.9 for whole rows.)
    const int vrow = QUANT ? lane >> 2 : lane >> 4;
    const int vcol = QUANT ? 32 * (lane & 3) : 8 * (lane & 15);
    const int k_boff = (QUANT && AIRKV_DECODE_K16)
                           ? (lane & 7) * D + 16 * (4 * ((lane >> 3) & 1) + 2 * ((lane >> 5) & 1) + ((lane >> 4) & 1))
                           : (r16 * D + 8 * g4) * EB;
    const int v_boff = QUANT ? ((lane >> 2) & 7) * D + 16 * (4 * ((lane >> 1) & 1) + 2 * (lane & 1) + ((lane >> 5) & 1))
                             : (vrow * D + vcol) * EB;
    const int n_sc = QUANT ? D / a.scale_group : 0;              // scales per row
    const int k_soff = QUANT ? (r16 * n_sc + (32 * g4) / a.scale_group) * 4 : 0;
    const int v_soff = QUANT ? (vrow * n_sc + vcol / a.scale_group) * 4 : 0;

    // Tiles are loaded unconditionally (an id outside the pool reads block 0)
    // and skipped at compute time, so no branch ever merges freshly loaded
    // registers.
    auto load_tile = [&](int idx, Tile<DT> &t) -> bool {
        int32_t blk = __builtin_amdgcn_readlane(tbl, idx);
        const int j = __builtin_amdgcn_readlane(j_l, idx);
        const bool ok = blk >= 0 && blk < a.num_blocks;
        blk = ok ? blk : 0;
        const int64_t row0 = ((int64_t)blk * a.n_kv_heads + kh) * BS + (16 * j) % BS;
        // Buffer loads: the tile's base lives in a scalar resource descriptor
        // and each lane's offset is a loop-invariant register, so no vector
        // address register is rewritten while earlier loads are in flight.
        // The descriptor also bounds the access to the 16-row tile.
        const __amdgpu_buffer_rsrc_t rk =
            __builtin_amdgcn_make_buffer_rsrc((void *)(kp + row0 * D * EB), (short)0, 16 * D * EB, kBufferWord3);
        const __amdgpu_buffer_rsrc_t rv =
            __builtin_amdgcn_make_buffer_rsrc((void *)(vp + row0 * D * EB), (short)0, 16 * D * EB, kBufferWord3);
        if constexpr (QUANT) {
            if constexpr (APPEND) {
                // Fused append, 1-byte pages, a sequence's last tile: before
                // the tile's loads are issued (few registers are live here),
                // the new token's K and V rows load, are quantized as
                // air_kv_append quantizes them (quantize_chunk: 16 lanes per
                // row, 8 elements each, scale_group / 8 lanes per group) and
                // are written to page row nv - 1 with their group scales.
                // The tile loads below may read that row before or after the
                // write: compute_tile replaces it in registers either way.
                if (ok && ((seqend_m >> idx) & 1)) {
                    const int bq = __builtin_amdgcn_readlane(seq_l, idx);
                    const int rn = __builtin_amdgcn_readlane(nv_l, idx) - 1;
                    const int64_t prow = row0 + rn;
                    const int64_t src = ((int64_t)bq * a.n_kv_heads + kh) * D;
                    // lanes 0..15 read K, 16..31 V, 8 floats each; the other
                    // lanes fall outside both descriptors and read zeros
                    const __amdgpu_buffer_rsrc_t rkn = __builtin_amdgcn_make_buffer_rsrc(
                        (void *)(a.k_new + src), (short)0, D * 4, kBufferWord3);
                    const __amdgpu_buffer_rsrc_t rvn = __builtin_amdgcn_make_buffer_rsrc(
                        (void *)(a.v_new + src), (short)0, D * 4, kBufferWord3);
                    const int koff = lane < 16 ? 32 * lane : D * 4;
                    const int voff = (lane >= 16 && lane < 32) ? 32 * (lane - 16) : D * 4;
                    float x[8];
#pragma unroll
                    for (int i = 0; i < 2; ++i) {
                        const f32x4 kx = __builtin_bit_cast(
                            f32x4, __builtin_amdgcn_raw_buffer_load_b128(rkn, koff + 16 * i, 0, 0));
                        const f32x4 vx = __builtin_bit_cast(
                            f32x4, __builtin_amdgcn_raw_buffer_load_b128(rvn, voff + 16 * i, 0, 0));
#pragma unroll
                        for (int j = 0; j < 4; ++j) x[4 * i + j] = lane < 16 ? kx[j] : vx[j];
                    }
                    const int lpg = a.scale_group >> 3;
                    quantize_chunk<DT>(x, lpg, t.qlo, t.qhi, t.qs);
                    const int c = lane & 15;                         // chunk: head_dim 8c .. +8
                    if (lane < 32) {
                        uint8_t *pg = (uint8_t *)(lane < 16 ? a.k_pages : a.v_pages);
                        *reinterpret_cast<u32x2 *>(pg + prow * D + 8 * c) = u32x2{t.qlo, t.qhi};
                        if (c % lpg == 0)
                            const_cast<float *>(lane < 16 ? a.k_scales : a.v_scales)[prow * n_sc + c / lpg] = t.qs;
                    }
                }
            }
            if constexpr (AIRKV_DECODE_K16) {
#pragma unroll
                for (int m = 0; m < 2; ++m)
                    t.k16[m] = __builtin_amdgcn_raw_buffer_load_b128(rk, k_boff + 8 * D * m, 0, k_code_aux<DT>());
            } else {
#pragma unroll
                for (int ks = 0; ks < KSTEPS; ++ks)
                    t.k[ks] = __builtin_amdgcn_raw_buffer_load_b64(rk, k_boff + 32 * ks, 0, k_code_aux<DT>());
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
                t.v[i] = __builtin_amdgcn_raw_buffer_load_b128(rv, v_boff + 8 * D * i, 0, kVCodeAux);
            const int64_t srow = row0 * n_sc;
            const __amdgpu_buffer_rsrc_t rks = __builtin_amdgcn_make_buffer_rsrc(
                (void *)(a.k_scales + srow), (short)0, 16 * n_sc * 4, kBufferWord3);
            const __amdgpu_buffer_rsrc_t rvs = __builtin_amdgcn_make_buffer_rsrc(
                (void *)(a.v_scales + srow), (short)0, 16 * n_sc * 4, kBufferWord3);
            t.ks = __builtin_amdgcn_raw_buffer_load_b32(rks, k_soff, 0, kScaleAux);
            t.vs = __builtin_amdgcn_raw_buffer_load_b32(rvs, v_soff, 0, kScaleAux);
        } else {
#pragma unroll
            for (int ks = 0; ks < KSTEPS; ++ks)
                t.k[ks] = __builtin_amdgcn_raw_buffer_load_b128(rk, k_boff + 64 * ks, 0, kLoadAux);
#pragma unroll
            for (int v = 0; v < 4; ++v)
                t.v[v] = __builtin_amdgcn_raw_buffer_load_b128(rv, v_boff + v * 4 * D * 2, 0, kLoadAux);
            if constexpr (APPEND) {
                // a sequence's last tile: its new K / V rows load with the
                // tile, so their latency hides behind the page loads
                if (ok && ((seqend_m >> idx) & 1)) {
                    const int bq = __builtin_amdgcn_readlane(seq_l, idx);
                    const int64_t src = ((int64_t)bq * a.n_kv_heads + kh) * D;
                    const __amdgpu_buffer_rsrc_t rkn = __builtin_amdgcn_make_buffer_rsrc(
                        (void *)(a.k_new + src), (short)0, D * 4, kBufferWord3);
                    const __amdgpu_buffer_rsrc_t rvn = __builtin_amdgcn_make_buffer_rsrc(
                        (void *)(a.v_new + src), (short)0, D * 4, kBufferWord3);
#pragma unroll
                    for (int i = 0; i < 8; ++i)
                        t.kn[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                                rkn, (32 * (i >> 1) + 8 * g4 + 4 * (i & 1)) * 4, 0, 0));
#pragma unroll
                    for (int i = 0; i < 2; ++i)
                        t.vn[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                                rvn, (vcol + 4 * i) * 4, 0, 0));
                }
            }
        }
        return ok;
    };

    // The piece of sequence bq held by this wave ends: write it out.
    auto emit = [&](int bq) {
        const float l = sum_x32(sum_x16(l_run));
        const int w0 = s_pre[bq] / chunk, w1 = (s_pre[bq + 1] - 1) / chunk;
        if (r16 < G) {
            if (w0 == w1) {                  // the whole sequence: final output
                const float inv = 1.0f / l;
                const int64_t orow = ((int64_t)bq * a.n_q_heads + kh * G + r16) * D + 4 * g4;
#pragma unroll
                for (int n = 0; n < DTILES; ++n) store_out4(a, orow + 16 * n, acc[n] * inv);
            } else {
                const int64_t row = ((int64_t)kh * a.slots + bq + w) * G + r16;
                float *po = a.part_o + row * D + 4 * g4;
#pragma unroll
                for (int n = 0; n < DTILES; ++n) *reinterpret_cast<f32x4 *>(po + 16 * n) = acc[n];
                if (g4 == 0) {
                    a.part_ml[row * 2] = m_run;
                    a.part_ml[row * 2 + 1] = l;
                }
            }
        }
    };

    auto compute_tile = [&](int k, int idx, Tile<DT> &t, bool ok) {
        const int bq = __builtin_amdgcn_readlane(seq_l, idx);
        if ((first_m >> idx) & 1) {          // a new sequence starts in this slice
            if (k != lo) load_q(bq);
            m_run = -INFINITY;
            l_run = 0.0f;
#pragma unroll
            for (int n = 0; n < DTILES; ++n) acc[n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
        // A table entry outside the pool is counted and its tile masked out;
        // the tile still runs every instruction, so the loaded registers are
        // consumed on all paths and the loads in flight never need draining.
        if (!ok && lane == 0) atomicAdd(a.errors, 1ull);
        const int nv = ok ? __builtin_amdgcn_readlane(nv_l, idx) : 0;   // valid tokens
        if constexpr (QUANT) {
            // the whole-row load order into the Tile layout (V here only for
            // the fused append, which replaces a row first; else at its use)
            if constexpr (AIRKV_DECODE_K16) swap_lane_bit3(t.k16[0], t.k16[1]);
            if constexpr (APPEND) swap_lane_bit5(t.v[0], t.v[1]);
        }
        if constexpr (APPEND && QUANT) {
            // Fused append, 1-byte pages: the new token's codes and scales,
            // quantized and written to the page by load_tile, move by lane
            // permutes into the tile registers of row nv - 1, in place of
            // whatever the tile loads read there.
            if (ok && ((seqend_m >> idx) & 1)) {
                const int rn = nv - 1;
                const int lpg = a.scale_group >> 3;                  // lanes per scale group
                const uint32_t lo = t.qlo, hi = t.qhi;
                const float qs = t.qs;
                // K row rn: lane (rn, g4) holds head_dim 64m + 16 g4 .. +16 in
                // k16[m], chunks 8m + 2 g4 and the next; its scale is group
                // 32 g4 / scale_group's
                const bool krow = r16 == rn;
#pragma unroll
                for (int m = 0; m < 2; ++m) {
                    const int sl = 8 * m + 2 * g4;
                    const u32x4 w = {(uint32_t)__shfl((int)lo, sl), (uint32_t)__shfl((int)hi, sl),
                                     (uint32_t)__shfl((int)lo, sl + 1), (uint32_t)__shfl((int)hi, sl + 1)};
                    t.k16[m] = krow ? w : t.k16[m];
                }
                const float kq = __shfl(qs, (32 * g4) / a.scale_group * lpg);
                t.ks = krow ? __float_as_uint(kq) : t.ks;
                // V row rn: lanes with vrow = rn hold head_dim vcol .. +32,
                // chunks 16 + vcol / 8 .. +4
                const bool vhit = vrow == rn;
                const int sv0 = 16 + vcol / 8;
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const int sl = sv0 + 2 * i;
                    const u32x4 w = {(uint32_t)__shfl((int)lo, sl), (uint32_t)__shfl((int)hi, sl),
                                     (uint32_t)__shfl((int)lo, sl + 1), (uint32_t)__shfl((int)hi, sl + 1)};
                    t.v[i] = vhit ? w : t.v[i];
                }
                const float vq = __shfl(qs, 16 + vcol / a.scale_group * lpg);
                t.vs = vhit ? __float_as_uint(vq) : t.vs;
            }
        }
        if constexpr (APPEND && !QUANT) {
            // Fused append: the decode step's new token is row nv - 1 of its
            // sequence's last tile, which this wave alone reads (a sequence
            // longer than its table has no such tile: it appends nothing).
            // Its K / V rows, loaded with the tile and rounded to bf16 as
            // air_kv_append rounds them, replace that row in the tile's
            // registers and are written to the page.
            if (ok && ((seqend_m >> idx) & 1)) {
                const int rn = nv - 1;
                const int32_t blk = __builtin_amdgcn_readlane(tbl, idx);
                const int jt = __builtin_amdgcn_readlane(j_l, idx);
                const int64_t prow = ((int64_t)blk * a.n_kv_heads + kh) * BS + (16 * jt) % BS + rn;
                auto pack8 = [](f32x4 x0, f32x4 x1) {
                    return u32x4{(uint32_t)bf16_rne(x0[0]) | ((uint32_t)bf16_rne(x0[1]) << 16),
                                 (uint32_t)bf16_rne(x0[2]) | ((uint32_t)bf16_rne(x0[3]) << 16),
                                 (uint32_t)bf16_rne(x1[0]) | ((uint32_t)bf16_rne(x1[1]) << 16),
                                 (uint32_t)bf16_rne(x1[2]) | ((uint32_t)bf16_rne(x1[3]) << 16)};
                };
                const bool krow = r16 == rn;     // K row rn: lanes (rn, g4), head_dim 32 ks + 8 g4 .. +8
#pragma unroll
                for (int ks = 0; ks < KSTEPS; ++ks) {
                    const u32x4 w = pack8(t.kn[2 * ks], t.kn[2 * ks + 1]);
                    t.k[ks] = krow ? w : t.k[ks];
                    if (krow) *reinterpret_cast<u32x4 *>((uint16_t *)a.k_pages + prow * D + 32 * ks + 8 * g4) = w;
                }
                // V row rn: lanes with vrow = rn % 4, register set rn / 4
                // (a select per set: a store to t.v[rn / 4] would index the
                // tile dynamically, in private memory)
                const bool vhit = vrow == (rn & 3);
                const u32x4 w = pack8(t.vn[0], t.vn[1]);
#pragma unroll
                for (int v = 0; v < 4; ++v) t.v[v] = (vhit && v == (rn >> 2)) ? w : t.v[v];
                if (vhit) *reinterpret_cast<u32x4 *>((uint16_t *)a.v_pages + prow * D + vcol) = w;
            }
        }
        // lane holds S[token 4*g4 + i][head r16]
        float sc[4];
        if constexpr (QUANT) {
            // 1-byte pages: the codes themselves are the A operands (exact in
            // bf16) and each k-step is one scale group, so the products are
            // exact and the group scales apply to the step sums afterwards:
            // S[t] = sum_ks scale[t][ks] * (codes[t] . q over step ks)
            s_ksc[wave][g4 * 16 + r16] = __uint_as_float(t.ks);
            // The step's 8 codes of row r16 for slot g4.  16-byte loads give
            // lane (r16, g4) head_dim 64*m + 16*g4 .. +16 (codes w0..w3), so
            // group 2m sits in lanes g4 < 2 and group 2m + 1 in lanes g4 >= 2,
            // 16 codes each.  One lane swap of (w0, w2) -- and of (w1, w3) --
            // across the two halves of the wave gives step 2m the lower
            // lanes' own w0, w1 and, in the upper lanes, the lower partner's
            // w2, w3, and gives step 2m + 1 the upper partner's w0, w1 in the
            // lower lanes and the upper lanes' own w2, w3: in both steps slot
            // g4 holds head_dim 16*(g4 & 1) + 8*(g4 >> 1) .. +8 of the group.
            u32x2 kc[KSTEPS];
            if constexpr (AIRKV_DECODE_K16) {
#pragma unroll
                for (int m = 0; m < 2; ++m) {
                    const u32x4 w = t.k16[m];
                    const auto s0 = __builtin_amdgcn_permlane32_swap(w[0], w[2], false, false);
                    const auto s1 = __builtin_amdgcn_permlane32_swap(w[1], w[3], false, false);
                    kc[2 * m] = u32x2{s0[0], s1[0]};
                    kc[2 * m + 1] = u32x2{s0[1], s1[1]};
                }
            } else {
#pragma unroll
                for (int ks = 0; ks < KSTEPS; ++ks) kc[ks] = t.k[ks];
            }
            f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ks = 0; ks < KSTEPS; ++ks) {
                const float b0 = DT == AIR_KV_INT8 ? qbias[ks] : 0.0f;
                f32x4 p = mfma_qk(codes_bf16<DT>(kc[ks]), qhi[ks], f32x4{b0, b0, b0, b0});

                // the step's scales of this lane's tokens 4*g4 .. +3
                const f32x4 ksc = *reinterpret_cast<const f32x4 *>(&s_ksc[wave][ks * 16 + 4 * g4]);
#pragma unroll
                for (int i = 0; i < 4; ++i) s[i] = __builtin_fmaf(ksc[i], p[i], s[i]);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) sc[i] = s[i] * a.scale_log2;
        } else {
            f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ks = 0; ks < KSTEPS; ++ks) {
                s = mfma_qk(t.k[ks], qhi[ks], s);
                if constexpr (QF32) s = mfma_qk(t.k[ks], qlo[ks], s);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) sc[i] = s[i] * a.scale_log2;
        }
        // only a sequence's last tile (or a tile of an out-of-pool block) is
        // partial: the masks run on those tiles alone (nv is uniform)
        const bool full = nv == 16;
        if (!full) {
#pragma unroll
            for (int i = 0; i < 4; ++i) sc[i] = 4 * g4 + i < nv ? sc[i] : -INFINITY;
        }
        float mt = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
        mt = max_x32(max_x16(mt));
        // The running max is raised only when some head's tile max exceeds it
        // by more than 2^8 (and on the first tile): probabilities then stay
        // below 256, exact in the hi + lo split, and most tiles skip the
        // rescale of the accumulators.  The final normalisation uses the same
        // max, so the result is unchanged.
        if (__ballot(mt > m_run + 8.0f) != 0ull) {
            const float m_new = fmaxf(m_run, mt);
            const float alpha = (m_run == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
            l_run *= alpha;
#pragma unroll
            for (int n = 0; n < DTILES; ++n) acc[n] *= alpha;
            m_run = m_new;
        }
        float p[4];
#pragma unroll
        // (the select covers a tile whose tokens are all masked while the
        // running max is still -inf)
        for (int i = 0; i < 4; ++i) p[i] = (sc[i] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(sc[i] - m_run);
        l_run += (p[0] + p[1]) + (p[2] + p[3]);
        // P^T as the B operand (lane: tokens 4*g4 .. +3 of head r16).  bf16
        // pages take hi + lo bf16 halves (~16 mantissa bits); 1-byte pages,
        // whose V operand is already a bf16 rounding of code * scale, take
        // the hi half only.
        u32x2 p_hi, p_lo = {0, 0};
        if constexpr (QUANT) {
            p_hi = u32x2{bf16_pair(p[0], p[1]), bf16_pair(p[2], p[3])};
        } else {
            uint32_t h0, l0, h1, l1;
            split_pair(p[0], p[1], h0, l0);
            split_pair(p[2], p[3], h1, l1);
            p_hi = u32x2{h0, h1};
            p_lo = u32x2{l0, l1};
        }
        // V tile -> LDS as bf16 (token rows beyond the sequence are zeroed: p = 0
        // there, but stale page bytes may hold non-finite values)
        if constexpr (QUANT) {
            if constexpr (!APPEND) swap_lane_bit5(t.v[0], t.v[1]);
            const float vsc = __uint_as_float(t.vs);
            const bool live = full || vrow < nv;
            u32x2 *dst = reinterpret_cast<u32x2 *>(sv + vrow * PITCH);
            u32x2 x[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) x[i] = dequant4<DT>(t.v[i >> 2][i & 3], vsc);
            if (!full) {
#pragma unroll
                for (int i = 0; i < 8; ++i) x[i] = live ? x[i] : u32x2{0, 0};
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) dst[(vcol / 4 + i) ^ (vrow & 7)] = x[i];
        } else {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int row = v * 4 + vrow;
                u32x4 x = t.v[v];
                if (!full && row >= nv) x = u32x4{0, 0, 0, 0};
                u32x2 *dst = reinterpret_cast<u32x2 *>(sv + row * PITCH);
                dst[(vcol / 4) ^ (row & 7)] = u32x2{x[0], x[1]};
                dst[(vcol / 4 + 1) ^ (row & 7)] = u32x2{x[2], x[3]};
            }
        }
        // O^T[d][h] += V^T[d][t] P^T[t][h]; the A lane holds V[t = 4*g4 + jj][d =
        // 16n + r16], jj = 0..3.  V stays row-major in LDS and a transposing
        // read builds the operand: within each 16-lane group, lane j receives
        // element j % 4 of the 8 bytes addressed by lanes 4k + j / 4 (k =
        // 0..3), so lane 16*g4 + s points at V[4*g4 + s/4][16n + 4*(s%4)]
        // (chunk 4n + s%4 of that row, swizzled as stored).
        const int vr = 4 * g4 + (r16 >> 2);
        const uint16_t *vrow_p = sv + vr * PITCH;
#pragma unroll
        for (int n = 0; n < DTILES; ++n) {
            typedef short s16x4 __attribute__((ext_vector_type(4)));
            const s16x4 t4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) s16x4 *)(vrow_p + 4 * ((4 * n + (r16 & 3)) ^ (vr & 7))));
            const u32x2 av = __builtin_bit_cast(u32x2, t4);
            acc[n] = mfma_pv(av, p_hi, acc[n]);
            if constexpr (!QUANT) acc[n] = mfma_pv(av, p_lo, acc[n]);
        }
        if ((last_m >> idx) & 1) emit(bq);
    };

    for (int c0 = lo; c0 < hi; c0 += 64) {
        load_window(c0);
        if (c0 == lo) load_q(__builtin_amdgcn_readlane(seq_l, 0));
        const int n = hi - c0 < 64 ? hi - c0 : 64;
        // kRing register sets used in rotation: kRing - 1 tiles are in
        // flight while one is computed.  Loads are issued unconditionally
        // (past the end they re-read the last tile, an L2 hit) so no branch
        // joins paths with different loads in flight.
        constexpr int kRing = QUANT ? AIRKV_DECODE_QRING : AIRKV_DECODE_RING;
        auto clampi = [&](int i) { return i < n ? i : n - 1; };
        if constexpr (kRing == 3) {
            // written out: the compiler allocates this form in fewer
            // registers than the general ring below
            Tile<DT> ta, tb, tc;
            bool oka = load_tile(0, ta), okb = load_tile(clampi(1), tb), okc;
            for (int i = 0; i < n; i += 3) {
                okc = load_tile(clampi(i + 2), tc);
                compute_tile(c0 + i, i, ta, oka);
                if (i + 1 >= n) break;
                oka = load_tile(clampi(i + 3), ta);
                compute_tile(c0 + i + 1, i + 1, tb, okb);
                if (i + 2 >= n) break;
                okb = load_tile(clampi(i + 4), tb);
                compute_tile(c0 + i + 2, i + 2, tc, okc);
            }
        } else {
            Tile<DT> ring[kRing];
            bool ok[kRing];
#pragma unroll
            for (int j = 0; j < kRing - 1; ++j) ok[j] = load_tile(clampi(j), ring[j]);
            for (int i = 0; i < n; i += kRing) {
#pragma unroll
                for (int j = 0; j < kRing; ++j) {
                    if (i + j >= n) break;
                    const int jl = (j + kRing - 1) % kRing;      // the set freed by the previous tile
                    ok[jl] = load_tile(clampi(i + j + kRing - 1), ring[jl]);
                    // 1-byte pages: a tile's dequantization and products at
                    // raised wave priority, so a SIMD's computing wave issues
                    // ahead of one that is waiting to load (c4 ~2% faster;
                    // bf16 pages measured no change)
                    if constexpr (QUANT) __builtin_amdgcn_s_setprio(1);
                    compute_tile(c0 + i + j, i + j, ring[j], ok[j]);
                    if constexpr (QUANT) __builtin_amdgcn_s_setprio(0);
                }
            }
        }
    }
}

// Log-sum-exp merge of the pieces of one (sequence, kv head), lane l holding
// head_dim columns 2l and 2l + 1.  A wave loads the (max, sum) and partial
// outputs of kBatch pieces together and folds them with an online rescale,
// so it spends one memory round trip per kBatch pieces (16 when sequences
// average more than eight pieces, 8 when they average three to eight, 4 when
// about two: fewer registers, more resident waves).  The kernel is bound by those round trips and by how many waves it
// launches, not by bytes, so the host picks WH, the waves per query head:
// one wave per head when the
// batch's sequences have few pieces each (WH = 1, grid z covers groups above
// four heads), and four waves per head when they have many (WH = 4, one
// workgroup per head: wave w folds pieces w, w + 4, ... and the four parts
// are folded in LDS in wave order).  Also writes zeros for an empty sequence
// and counts sequence lengths outside [0, max_blocks * block_size].
struct MergeAcc {
    float m, l, o0, o1;
};

__device__ __forceinline__ void merge_fold(MergeAcc &c, float pm, float pl, float v0, float v1) {
    if (pm == -INFINITY) return;                         // past the last piece (or all masked)
    const float m_new = fmaxf(c.m, pm);
    const float sa = __builtin_amdgcn_exp2f(c.m - m_new), sb = __builtin_amdgcn_exp2f(pm - m_new);
    c.l = c.l * sa + pl * sb;
    c.o0 = c.o0 * sa + v0 * sb;
    c.o1 = c.o1 * sa + v1 * sb;
    c.m = m_new;
}

template <int D, int WH, int kBatch>
__global__ __launch_bounds__(kThreads) void decode_merge_kernel(DecodeArgs a) {
    static_assert(D == 128, "lane holds two head_dim columns");
    static_assert(WH == 1 || WH == kWaves, "one or all waves per head");
    constexpr int kHeadsPerGroup = kWaves / WH;          // query heads per workgroup
    __shared__ float s_ml[kWaves][2];
    __shared__ float2 s_o[kWaves][64];
    const int b = blockIdx.x, kh = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = a.group;
    const int64_t max_len = (int64_t)a.max_blocks * a.block_size;
    // every index the workgroup needs, loaded together (one round trip)
    const int p0 = a.prefix[b], p1 = a.prefix[b + 1], chunk = a.prefix[a.batch + 1];
    const int len = a.lens[b];
    if (tid == 0 && kh == 0 && blockIdx.z == 0 && (len < 0 || len > max_len)) atomicAdd(a.errors, 1ull);
    const int64_t obase = ((int64_t)b * a.n_q_heads + kh * G) * D;
    if (p0 == p1) {                                      // empty sequence: zeros
        if (blockIdx.z == 0)
            for (int idx = tid; idx < G * D; idx += kThreads) store_out(a, obase + idx, 0.0f);
        return;
    }
    const int w0 = p0 / chunk, w1 = (p1 - 1) / chunk;
    if (w0 == w1) return;                                // written by its slice
    const int n = w1 - w0 + 1;
    const int sub = wave % WH;                           // this wave's share of the head's pieces
    // row of (piece p, head h): row0 + p * G + h
    const int64_t row0 = ((int64_t)kh * a.slots + b + w0) * G;
    for (int h = blockIdx.z * kHeadsPerGroup + wave / WH; h < G; h += gridDim.z * kHeadsPerGroup) {
        MergeAcc c{-INFINITY, 0.0f, 0.0f, 0.0f};
        for (int q0 = sub; q0 < n; q0 += WH * kBatch) {
            float pm[kBatch], pl[kBatch];
            float2 pv[kBatch];
#pragma unroll
            for (int i = 0; i < kBatch; ++i) {
                const int p = q0 + WH * i < n ? q0 + WH * i : q0;
                const int64_t row = row0 + (int64_t)p * G + h;
                pm[i] = q0 + WH * i < n ? a.part_ml[row * 2] : -INFINITY;
                pl[i] = a.part_ml[row * 2 + 1];
                pv[i] = *reinterpret_cast<const float2 *>(a.part_o + row * D + 2 * lane);
            }
#pragma unroll
            for (int i = 0; i < kBatch; ++i) merge_fold(c, pm[i], pl[i], pv[i].x, pv[i].y);
        }
        if constexpr (WH > 1) {                          // fold the four waves' parts
            if (lane == 0) {
                s_ml[wave][0] = c.m;
                s_ml[wave][1] = c.l;
            }
            s_o[wave][lane] = float2{c.o0, c.o1};
            __syncthreads();
            if (sub != 0) continue;                      // one head per workgroup: loop ends
            c = MergeAcc{-INFINITY, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int w = 0; w < WH; ++w) merge_fold(c, s_ml[w][0], s_ml[w][1], s_o[w][lane].x, s_o[w][lane].y);
        }
        const float inv = 1.0f / c.l;
        const int64_t oi = obase + (int64_t)h * D + 2 * lane;
        if (a.out_dtype == AIR_KV_F32) {
            *reinterpret_cast<float2 *>((float *)a.out + oi) = float2{c.o0 * inv, c.o1 * inv};
        } else {
            *reinterpret_cast<uint32_t *>((uint16_t *)a.out + oi) =
                (uint32_t)bf16_rne(c.o0 * inv) | ((uint32_t)bf16_rne(c.o1 * inv) << 16);
        }
    }
}

template <int BS, bool QF32, int DT>
hipError_t launch_cfg(const DecodeArgs &a, hipStream_t s) {
    const int64_t waves = (int64_t)a.n_kv_heads * a.slices;
    const dim3 grid((unsigned)((waves + kWaves - 1) / kWaves));
    if (a.k_new)
        hipLaunchKernelGGL((decode_mfma_kernel<128, BS, QF32, DT, true>), grid, dim3(kThreads), 0, s, a);
    else
        hipLaunchKernelGGL((decode_mfma_kernel<128, BS, QF32, DT, false>), grid, dim3(kThreads), 0, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // Sequences average slices / batch pieces: past one round trip's worth,
    // four waves share each head.
    if (a.slices > 16 * a.batch) {
        hipLaunchKernelGGL((decode_merge_kernel<128, kWaves, 16>),
                           dim3((unsigned)a.batch, (unsigned)a.n_kv_heads, (unsigned)a.group), dim3(kThreads), 0,
                           s, a);
    } else if (a.slices > 8 * a.batch) {
        hipLaunchKernelGGL((decode_merge_kernel<128, 1, 16>),
                           dim3((unsigned)a.batch, (unsigned)a.n_kv_heads, (unsigned)((a.group + kWaves - 1) / kWaves)),
                           dim3(kThreads), 0, s, a);
    } else if (a.slices > 2 * a.batch) {        // about 3..8 pieces: eight per round trip
        hipLaunchKernelGGL((decode_merge_kernel<128, 1, 8>),
                           dim3((unsigned)a.batch, (unsigned)a.n_kv_heads, (unsigned)((a.group + kWaves - 1) / kWaves)),
                           dim3(kThreads), 0, s, a);
    } else {                    // about two pieces per sequence: fewer registers, more waves resident
        hipLaunchKernelGGL((decode_merge_kernel<128, 1, 4>),
                           dim3((unsigned)a.batch, (unsigned)a.n_kv_heads, (unsigned)((a.group + kWaves - 1) / kWaves)),
                           dim3(kThreads), 0, s, a);
    }
    return hipGetLastError();
}

template <int DT>
hipError_t launch_dt(const DecodeArgs &a, hipStream_t s) {
    if (a.block_size == 16)
        return a.q_dtype == AIR_KV_F32 ? launch_cfg<16, true, DT>(a, s) : launch_cfg<16, false, DT>(a, s);
    return a.q_dtype == AIR_KV_F32 ? launch_cfg<32, true, DT>(a, s) : launch_cfg<32, false, DT>(a, s);
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace

bool decode_mfma_supported(int dtype, int head_dim, int block_size, int group, int scale_group) {
    if (head_dim != 128 || (block_size != 16 && block_size != 32) || group < 1 || group > 16) return false;
    if (dtype == AIR_KV_BF16) return true;
    // 1-byte pages: a lane's 32 contiguous codes must share one scale
    return (dtype == AIR_KV_INT8 || dtype == AIR_KV_FP8) && scale_group >= 32;
}

// Slices per kv head: one wave for every wave slot of the GPU (4 SIMDs per
// compute unit x waves_per_simd), at most batch * max_splits.  The kernel
// widens the slices when the longest sequence would otherwise be cut into
// more than max_splits pieces (slice_chunk), leaving the rest of the waves
// idle.  The workspace holds the tile prefix and the chunk, then (slices +
// batch) partial rows per query head.
int plan_decode_mfma(const air_kv_pool &p, int32_t n_q_heads, int32_t batch, int32_t max_blocks,
                     int32_t max_splits, DecodePlan *plan) {
    const int nkv = p.desc.n_kv_heads, d = p.desc.head_dim, bs = p.desc.block_size;
    const int32_t nb = batch < kMaxBatch ? batch : kMaxBatch;
    const int64_t tiles_per_seq = ((int64_t)max_blocks * bs + 15) / 16;
    if ((int64_t)nb * tiles_per_seq > INT32_MAX)
        return fail(AIR_KV_E_INVALID_ARG, "batch x max_blocks too large for one decode launch");
    const int64_t cap = (int64_t)(nb > 0 ? nb : 1) * max_splits;
    auto slices_for = [&](int waves_per_simd) {
        const int64_t machine_waves = (int64_t)p.cus * 4 * waves_per_simd;
        const int64_t sl = (machine_waves + nkv - 1) / nkv;
        return sl > cap ? cap : sl;
    };
    const int64_t slices = slices_for(waves_per_simd(p.desc.dtype));
    plan->mfma = true;
    plan->dtype = p.desc.dtype;
    plan->part_tokens = plan->num_parts = 0;
    plan->slices = (int32_t)slices;
    // the f32-query build's slices (what is resident at once; the workspace,
    // sized for plan->slices, holds them whenever that build runs fewer waves)
    plan->slices_qf32 = (int32_t)slices_for(kernel_waves_per_simd(p.desc.dtype, false));
    plan->slices_append = (int32_t)slices_for(kernel_waves_per_simd(p.desc.dtype, true));
    plan->batch_per_launch = nb;
    plan->slots = (int32_t)(slices + nb);
    plan->ws_bytes = align256((size_t)(nb + 2) * 4) + align256((size_t)n_q_heads * plan->slots * 2 * 4) +
                     (size_t)n_q_heads * plan->slots * d * 4;
    return AIR_KV_OK;
}

hipError_t launch_decode_mfma(const DecodeArgs &base, const DecodePlan &plan, void *workspace,
                              hipStream_t s) {
    for (int32_t b0 = 0; b0 < base.batch; b0 += plan.batch_per_launch) {
        DecodeArgs a = base;
        a.batch = base.batch - b0 < plan.batch_per_launch ? base.batch - b0 : plan.batch_per_launch;
        // partial rows are laid out for plan.slots; fewer slices use a prefix of them
        a.slices = base.k_new ? plan.slices_append : base.q_dtype == AIR_KV_F32 ? plan.slices_qf32 : plan.slices;
        a.slots = a.slices + plan.batch_per_launch;
        const int64_t q_row = (int64_t)b0 * a.n_q_heads * 128;
        a.q = (const char *)base.q + q_row * (base.q_dtype == AIR_KV_F32 ? 4 : 2);
        a.out = (char *)base.out + q_row * (base.out_dtype == AIR_KV_F32 ? 4 : 2);
        a.tables = base.tables + (int64_t)b0 * a.max_blocks;
        a.lens = base.lens + b0;
        if (base.k_new) {
            const int64_t kv_row = (int64_t)b0 * a.n_kv_heads * 128;
            a.k_new = base.k_new + kv_row;
            a.v_new = base.v_new + kv_row;
        }
        char *ws = (char *)workspace;
        a.prefix = (int32_t *)ws;
        ws += align256((size_t)(plan.batch_per_launch + 2) * 4);
        a.part_ml = (float *)ws;
        ws += align256((size_t)a.n_q_heads * plan.slots * 2 * 4);
        a.part_o = (float *)ws;
        hipError_t e = plan.dtype == AIR_KV_BF16   ? launch_dt<AIR_KV_BF16>(a, s)
                       : plan.dtype == AIR_KV_INT8 ? launch_dt<AIR_KV_INT8>(a, s)
                                                   : launch_dt<AIR_KV_FP8>(a, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace airkv
