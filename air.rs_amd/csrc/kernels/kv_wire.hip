// KvBlock wire format (src/pd_disagg.rs:39-49) and its int8 transfer
// quantization (KvBlock::int8_quantize, :65-83).
//
// A wire block is the bf16 array [block_size][n_kv_heads][head_dim][2] of one
// page, K at index 0 and V at index 1 of the last axis.  One workgroup owns
// one block.  A thread takes 8 consecutive head_dim elements of one (token,
// head) row: 16 K and V bytes in from the two page slabs (any pool dtype,
// via load8), 32 interleaved wire bytes out, so reads and writes stay
// 16-byte coalesced.  The int8 variant rounds the values to bf16 (the wire
// element), reduces their absmax over the whole block in LDS, and writes
// round(x * (1 / scale)) codes in wire order with one f32 scale per block;
// blocks of up to 8 items per thread (bs 16, 8 heads, d 128 is exactly that)
// stay in registers between the two steps, larger ones are read twice.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "../pool.hpp"
#include "codecs.hpp"
#include "page_io.hpp"

namespace airkv {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;
constexpr int kHeldItems = 8;   // (token, head, 8-element) items a thread holds for the int8 pack

struct WireArgs {
    const int32_t *ids;
    int32_t n;
    int32_t n_kv_heads, head_dim, block_size, scale_group;
    int64_t num_blocks;
    void *k_pages, *v_pages;
    float *k_scales, *v_scales;
    void *wire;                    // bf16 wire blocks (pack out / unpack in)
    int8_t *codes;                 // int8 wire codes (pack_int8 out)
    float *wire_scales;            // one per block (pack_int8 out)
    unsigned long long *errors;
    uint32_t chunks_magic, heads_magic;   // ceil(2^32 / d) for d = head_dim / 8, n_kv_heads (0: d == 1)
};

// x / d for the small x of one block (x * d < 2^32) as one high multiply by
// m = ceil(2^32 / d): x * m / 2^32 = x / d + x * e / (d * 2^32) with e < d,
// so the floor is exact while x * e < 2^32.
__device__ __forceinline__ uint32_t div_magic(uint32_t x, uint32_t m) { return m ? __umulhi(x, m) : x; }

// bf16 pages: a wire element is the page element's bits (the f32 value of
// a bf16 rounds back to itself; a NaN gets its quiet bit, as bf16_rne gives
// it), so these kernels move bits with byte permutes instead of converting.
// Lane j of a pass owns item j = (token, head, 8-element chunk): 16 bytes
// from each slab, 32 wire bytes.  The pack stages each wave's 2 KB of wire
// bytes in its own LDS slice and stores them back as two 1 KB runs, so every
// store instruction writes whole cache lines (a lane's own 32 bytes would
// leave each instruction writing half of every line it touches).
constexpr int kItemsHeld = 8;   // items a lane loads before it stores (64 KB per 256 lanes)

// Both halves of a bf16 pair through bf16_rne(f32): NaN halves (magnitude
// above 0x7F80, which the add carries into bit 15) get bit 6 set.
__device__ __forceinline__ uint32_t quiet_bf16x2(uint32_t w) {
    const uint32_t t = (w & 0x7FFF7FFFu) + 0x007F007Fu;
    return w | ((t >> 9) & 0x00400040u);
}

// Page element of item `it` of block blk (item = (t * n_kv_heads + h) *
// chunks + c).
__device__ __forceinline__ int64_t item_elem(const WireArgs &a, int32_t blk, uint32_t it) {
    const uint32_t chunks = (uint32_t)a.head_dim / 8;
    const uint32_t r = div_magic(it, a.chunks_magic);              // t * n_kv_heads + h
    const uint32_t c = it - r * chunks;
    const uint32_t t = div_magic(r, a.heads_magic);
    const uint32_t h = r - t * (uint32_t)a.n_kv_heads;
    const int64_t row = ((int64_t)blk * a.n_kv_heads + h) * a.block_size + t;
    return row * a.head_dim + 8 * c;
}

__global__ __launch_bounds__(kThreads) void kv_pack_bf16_kernel(WireArgs a) {
    __shared__ __align__(16) u32x4 s_wire[kThreads / 64][2 * 64];   // per wave: 64 items x 32 bytes
    const int32_t blk = a.ids[blockIdx.x];
    if (blk < 0 || blk >= a.num_blocks) {
        if (threadIdx.x == 0) atomicAdd(a.errors, 1ull);
        return;
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t items = (uint32_t)a.block_size * a.n_kv_heads * a.head_dim / 8;
    u32x4 *out = reinterpret_cast<u32x4 *>(a.wire) + (int64_t)blockIdx.x * 2 * items;
    const uint16_t *kp = (const uint16_t *)a.k_pages, *vp = (const uint16_t *)a.v_pages;
    u32x4 *slice = s_wire[wave];
    for (uint32_t base = 0; base < items; base += kThreads * kItemsHeld) {
        u32x4 kw[kItemsHeld], vw[kItemsHeld];
#pragma unroll
        for (int u = 0; u < kItemsHeld; ++u) {
            const uint32_t it = base + u * kThreads + threadIdx.x;
            if (it < items) {
                const int64_t e = item_elem(a, blk, it);
                kw[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(kp + e));
                vw[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(vp + e));
            }
        }
#pragma unroll
        for (int u = 0; u < kItemsHeld; ++u) {
            // items [i0, i0 + 64) of this wave: wire segments 2 * i0 .. + 128
            const uint32_t i0 = base + u * kThreads + 64 * wave;
            if (i0 >= items) break;                      // uniform per wave
            u32x4 lo, hi;                                // k0 | v0 << 16, ...
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                lo[2 * j] = quiet_bf16x2(__builtin_amdgcn_perm(vw[u][j], kw[u][j], 0x05040100u));
                lo[2 * j + 1] = quiet_bf16x2(__builtin_amdgcn_perm(vw[u][j], kw[u][j], 0x07060302u));
                hi[2 * j] = quiet_bf16x2(__builtin_amdgcn_perm(vw[u][2 + j], kw[u][2 + j], 0x05040100u));
                hi[2 * j + 1] = quiet_bf16x2(__builtin_amdgcn_perm(vw[u][2 + j], kw[u][2 + j], 0x07060302u));
            }
            slice[2 * lane] = lo;
            slice[2 * lane + 1] = hi;
            __builtin_amdgcn_s_waitcnt(0xc07f);          // lgkmcnt(0): the slice is written
            __builtin_amdgcn_wave_barrier();
            const u32x4 a0 = slice[lane], a1 = slice[64 + lane];
            const uint32_t segs = 2 * (items - i0 < 64 ? items - i0 : 64);
            if ((uint32_t)lane < segs) __builtin_nontemporal_store(a0, out + 2 * i0 + lane);
            if ((uint32_t)(64 + lane) < segs) __builtin_nontemporal_store(a1, out + 2 * i0 + 64 + lane);
            __builtin_amdgcn_s_waitcnt(0xc07f);          // the slice is read before the next item
            __builtin_amdgcn_wave_barrier();
        }
    }
}

__global__ __launch_bounds__(kThreads) void kv_unpack_bf16_kernel(WireArgs a) {
    const int32_t blk = a.ids[blockIdx.x];
    if (blk < 0 || blk >= a.num_blocks) {
        if (threadIdx.x == 0) atomicAdd(a.errors, 1ull);
        return;
    }
    const uint32_t items = (uint32_t)a.block_size * a.n_kv_heads * a.head_dim / 8;
    const u32x4 *in = reinterpret_cast<const u32x4 *>(a.wire) + (int64_t)blockIdx.x * 2 * items;
    uint16_t *kp = (uint16_t *)a.k_pages, *vp = (uint16_t *)a.v_pages;
    // Each wave reads its 64 items' 2 KB of wire as two 1 KB runs (lane l:
    // segments l and 64 + l, so every load instruction reads whole lines)
    // and moves them through its own LDS slice to lane l's segments 2l and
    // 2l + 1.  Each lane loading its own two segments read half of every
    // line per load instruction.
    __shared__ __align__(16) u32x4 s_wire[kThreads / 64][2 * 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    u32x4 *slice = s_wire[wave];
    for (uint32_t base = 0; base < items; base += kThreads * kItemsHeld) {
        u32x4 w0[kItemsHeld], w1[kItemsHeld];
#pragma unroll
        for (int u = 0; u < kItemsHeld; ++u) {
            const uint32_t i0 = base + u * kThreads + 64 * wave;      // the wave's first item
            const uint32_t segs = i0 < items ? 2 * (items - i0 < 64 ? items - i0 : 64) : 0;
            w0[u] = (uint32_t)lane < segs ? __builtin_nontemporal_load(in + 2 * i0 + lane) : u32x4{0, 0, 0, 0};
            w1[u] = (uint32_t)(64 + lane) < segs ? __builtin_nontemporal_load(in + 2 * i0 + 64 + lane)
                                                  : u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < kItemsHeld; ++u) {
            const uint32_t it = base + u * kThreads + threadIdx.x;
            if (it - lane >= items) break;                 // uniform per wave
            slice[lane] = w0[u];
            slice[64 + lane] = w1[u];
            __builtin_amdgcn_s_waitcnt(0xc07f);          // lgkmcnt(0): the slice is written
            __builtin_amdgcn_wave_barrier();
            const u32x4 lo = slice[2 * lane], hi = slice[2 * lane + 1];
            __builtin_amdgcn_s_waitcnt(0xc07f);          // read before the next item rewrites it
            __builtin_amdgcn_wave_barrier();
            if (it >= items) continue;
            const int64_t e = item_elem(a, blk, it);
            u32x4 k, v;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                k[j] = quiet_bf16x2(__builtin_amdgcn_perm(lo[2 * j + 1], lo[2 * j], 0x05040100u));
                v[j] = quiet_bf16x2(__builtin_amdgcn_perm(lo[2 * j + 1], lo[2 * j], 0x07060302u));
                k[2 + j] = quiet_bf16x2(__builtin_amdgcn_perm(hi[2 * j + 1], hi[2 * j], 0x05040100u));
                v[2 + j] = quiet_bf16x2(__builtin_amdgcn_perm(hi[2 * j + 1], hi[2 * j], 0x07060302u));
            }
            // whole blocks are rewritten: streaming stores (4.95 against
            // 4.73 TB/s with plain ones for 4096 blocks of 64 KB)
            __builtin_nontemporal_store(k, reinterpret_cast<u32x4 *>(kp + e));
            __builtin_nontemporal_store(v, reinterpret_cast<u32x4 *>(vp + e));
        }
    }
}

// KvBlock::int8_quantize's code of y = x * inv when |y| <= 127.5 and y is
// finite: Rust's f32::round (half away from zero) is the truncation of
// y + copysign(0.49999997, y) (0.5 - 2^-25).  For 0.5 <= |y| < 2^22 the sum
// reaches the next integer exactly when |y| reaches the half (a tie lands on
// it; anything below stays at least an ulp short), and for |y| < 0.5 it
// stays below 1 (with 0.5 itself, 0.5 - 2^-25 would round up to 1.0).
// Blocks with a finite absmax whose scale (absmax / 127) is normal give
// |y| <= 127 * (1 + 2^-22): no clamp applies.
__device__ __forceinline__ uint32_t pd_code_finite(float y) {
    return (uint32_t)(int32_t)(y + __builtin_copysignf(0.49999997f, y));
}

// Magnitude bits of both halves of a bf16 pair with NaN halves (magnitude
// above 0x7F80, which the add carries into bit 15) set to 0.
__device__ __forceinline__ uint32_t mag_no_nan(uint32_t w) {
    const uint32_t t = w & 0x7FFF7FFFu;
    const uint32_t nan = ((t + 0x007F007Fu) >> 15) & 0x00010001u;
    return t & ~(nan * 0xFFFFu);
}

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t max_u16x2(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2, a),
                                                                  __builtin_bit_cast(u16x2, b)));
}

// Workgroup-wide max of one u32 per thread over NT threads; s holds NT / 64
// words that no thread reads until the barrier inside.
template <int NT>
__device__ __forceinline__ uint32_t block_max_u32(uint32_t m, uint32_t *s) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const uint32_t y = (uint32_t)__shfl_xor((int)m, o);
        m = y > m ? y : m;
    }
    if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = m;
    __syncthreads();
    uint32_t r = 0;
#pragma unroll
    for (int w = 0; w < NT / 64; ++w) r = s[w] > r ? s[w] : r;
    return r;
}

// Codes of 2 K and 2 V elements (K pair kp, V pair vp) in wire order k0 v0 k1 v1.
template <bool FAST>
__device__ __forceinline__ uint32_t codes4(uint32_t kp2, uint32_t vp2, float inv) {
    float y[4];
    {
#pragma clang fp contract(off)
        y[0] = __uint_as_float(kp2 << 16) * inv;
        y[1] = __uint_as_float(vp2 << 16) * inv;
        y[2] = __uint_as_float(kp2 & 0xFFFF0000u) * inv;
        y[3] = __uint_as_float(vp2 & 0xFFFF0000u) * inv;
    }
    uint32_t c[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        if constexpr (FAST) {
            c[e] = pd_code_finite(y[e]);
        } else {
            // the general rule on the value as pd_code takes it (x, then x * inv)
            const float x = e == 0 ? __uint_as_float(kp2 << 16) : e == 1 ? __uint_as_float(vp2 << 16)
                          : e == 2 ? __uint_as_float(kp2 & 0xFFFF0000u) : __uint_as_float(vp2 & 0xFFFF0000u);
            c[e] = (uint8_t)pd_code(x, inv);
        }
    }
    return __builtin_amdgcn_perm(c[1], c[0], 0x0c0c0400u) | __builtin_amdgcn_perm(c[3], c[2], 0x04000c0cu);
}

// KvBlock::int8_quantize fused with the pack for bf16 pools whose block fits
// one pass of 512 lanes x 4 items (2048 items: 64 KB of K and V).
// Workgroups are persistent:
// workgroup g takes blocks g, g + gridDim.x, ...; the page loads of its next
// block are issued before the codes of the current one are computed, so HBM
// reads continue while the vector ALUs work (with one workgroup per block,
// the resident blocks all load, then all compute).  The absmax runs on the
// bf16 magnitude bits (NaN halves dropped when the block holds one).
constexpr int kQThreads = 512, kQItems = 4;
__global__ __launch_bounds__(kQThreads) void kv_pack_int8_bf16_kernel(WireArgs a) {
    __shared__ uint32_t s_max[3][kQThreads / 64];
    const uint32_t items = (uint32_t)a.block_size * a.n_kv_heads * a.head_dim / 8;
    const uint16_t *kp = (const uint16_t *)a.k_pages, *vp = (const uint16_t *)a.v_pages;
    u32x4 kw[kQItems], vw[kQItems];
    auto block_of = [&](int64_t i) -> int32_t {
        if (i >= a.n) return -2;
        const int32_t b = a.ids[i];
        return b >= 0 && b < a.num_blocks ? b : -1;
    };
    auto load = [&](int32_t blk) {
#pragma unroll
        for (int u = 0; u < kQItems; ++u) {
            const uint32_t it = u * kQThreads + threadIdx.x;
            if (it < items) {
                const int64_t e = item_elem(a, blk, it);
                kw[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(kp + e));
                vw[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(vp + e));
            }
        }
    };
    int32_t blk = block_of(blockIdx.x);
    if (blk >= 0) load(blk);
    int par = 0;
    for (int64_t i = blockIdx.x; i < a.n; i += gridDim.x, par ^= 1) {
        const int32_t next = block_of(i + gridDim.x);
        if (blk < 0) {                                   // uniform: the id is shared
            if (threadIdx.x == 0) atomicAdd(a.errors, 1ull);
            if (next >= 0) load(next);
            blk = next;
            continue;
        }
        u32x4 ck[kQItems], cv[kQItems];             // this block's bits (out-of-range items 0)
        uint32_t m = 0;
#pragma unroll
        for (int u = 0; u < kQItems; ++u) {
            const bool in = u * kQThreads + threadIdx.x < items;
            ck[u] = in ? kw[u] : u32x4{0, 0, 0, 0};
            cv[u] = in ? vw[u] : u32x4{0, 0, 0, 0};
#pragma unroll
            for (int j = 0; j < 4; ++j) m = max_u16x2(m, max_u16x2(ck[u][j] & 0x7FFF7FFFu, cv[u][j] & 0x7FFF7FFFu));
        }
        if (next >= 0) load(next);                       // the next block's reads overlap the codes below
        uint32_t mb = block_max_u32<kQThreads>(max_u16x2(m, m >> 16) & 0xFFFFu, s_max[par]);
        const bool has_nan = mb > 0x7F80u;
        if (has_nan) {                                   // the max of the other values
            m = 0;
#pragma unroll
            for (int u = 0; u < kQItems; ++u)
#pragma unroll
                for (int j = 0; j < 4; ++j) m = max_u16x2(m, max_u16x2(mag_no_nan(ck[u][j]), mag_no_nan(cv[u][j])));
            mb = block_max_u32<kQThreads>(max_u16x2(m, m >> 16) & 0xFFFFu, s_max[2]);
        }
        float scale, inv;
        {
#pragma clang fp contract(off)
            const float max_val = __uint_as_float(mb << 16);
            scale = max_val > 0.0f ? max_val / 127.0f : 1.0f;
            inv = 1.0f / scale;
        }
        // no NaN, a finite absmax and a normal scale (1 / scale finite), or
        // all zeros: every |y| <= 127 * (1 + 2^-22)
        const bool fast = !has_nan && (mb == 0 || (mb < 0x7F80u && scale >= 1.17549435e-38f));
        int8_t *out = a.codes + i * (int64_t)items * 16;
        auto emit = [&](auto fast_tag) {
            constexpr bool F = decltype(fast_tag)::value;
#pragma unroll
            for (int u = 0; u < kQItems; ++u) {
                const uint32_t it = u * kQThreads + threadIdx.x;
                if (it >= items) break;
                const u32x4 q = {codes4<F>(ck[u][0], cv[u][0], inv), codes4<F>(ck[u][1], cv[u][1], inv),
                                 codes4<F>(ck[u][2], cv[u][2], inv), codes4<F>(ck[u][3], cv[u][3], inv)};
                __builtin_nontemporal_store(q, reinterpret_cast<u32x4 *>(out + (int64_t)it * 16));
            }
        };
        if (fast) emit(std::true_type{});
        else emit(std::false_type{});
        if (threadIdx.x == 0) a.wire_scales[i] = scale;
        blk = next;
    }
}

// wire bf16 pairs of 8 K and 8 V values: k0 v0 k1 v1 ...
__device__ __forceinline__ void interleave(const float (&k)[8], const float (&v)[8], u32x4 &lo, u32x4 &hi) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        lo[j] = (uint32_t)bf16_rne(k[j]) | ((uint32_t)bf16_rne(v[j]) << 16);
        hi[j] = (uint32_t)bf16_rne(k[4 + j]) | ((uint32_t)bf16_rne(v[4 + j]) << 16);
    }
}

// Block-wide absmax (NaN-ignoring fold, any order: max is order independent).
__device__ float block_absmax(float m, float *s_red) {
    for (int o = 32; o >= 1; o >>= 1) m = absmax_step(m, __shfl_xor(m, o));
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) s_red[wave] = m;
    __syncthreads();
    float r = 0.0f;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) r = absmax_step(r, s_red[w]);
    return r;
}

template <int DT, bool INT8>
__global__ __launch_bounds__(kThreads) void kv_pack_kernel(WireArgs a) {
    __shared__ float s_red[kThreads / 64];
    const int32_t blk = a.ids[blockIdx.x];
    if (blk < 0 || blk >= a.num_blocks) {
        if (threadIdx.x == 0) atomicAdd(a.errors, 1ull);
        return;
    }
    const int chunks = a.head_dim / 8;
    const int items = a.block_size * a.n_kv_heads * chunks;    // (t, h, chunk)
    const int ng = (DT == AIR_KV_INT8 || DT == AIR_KV_FP8) ? a.head_dim / a.scale_group : 1;
    const int sg = a.scale_group > 0 ? a.scale_group : 1;
    const int64_t wire_elems = (int64_t)a.block_size * a.n_kv_heads * a.head_dim * 2;
    auto load_item = [&](int it, float (&k)[8], float (&v)[8]) -> int64_t {
        const int t = it / (a.n_kv_heads * chunks);
        const int rem = it - t * a.n_kv_heads * chunks;
        const int h = rem / chunks, c = rem - h * chunks;
        const int64_t row = ((int64_t)blk * a.n_kv_heads + h) * a.block_size + t;
        const int64_t elem = row * a.head_dim + 8 * c;
        const int64_t sidx = row * ng + (8 * c) / sg;
        pio_u32x4 raw;
        load8<DT>(a.k_pages, a.k_scales, elem, sidx, k, &raw);
        load8<DT>(a.v_pages, a.v_scales, elem, sidx, v, &raw);
        return (((int64_t)t * a.n_kv_heads + h) * a.head_dim + 8 * c) * 2;   // wire element
    };
    if constexpr (!INT8) {
        // up to kHeldItems items per thread loaded before any is stored (the
        // compiler cannot move a load above a store it cannot prove disjoint)
        uint16_t *out = (uint16_t *)a.wire + (int64_t)blockIdx.x * wire_elems;
        for (int base = 0; base < items; base += kThreads * kHeldItems) {
            u32x4 lo[kHeldItems], hi[kHeldItems];
            int64_t we[kHeldItems];
#pragma unroll
            for (int u = 0; u < kHeldItems; ++u) {
                const int it = base + threadIdx.x + u * kThreads;
                we[u] = -1;
                if (it < items) {
                    float k[8], v[8];
                    we[u] = load_item(it, k, v);
                    interleave(k, v, lo[u], hi[u]);
                }
            }
#pragma unroll
            for (int u = 0; u < kHeldItems; ++u) {
                if (we[u] < 0) continue;
                __builtin_nontemporal_store(lo[u], reinterpret_cast<u32x4 *>(out + we[u]));
                __builtin_nontemporal_store(hi[u], reinterpret_cast<u32x4 *>(out + we[u] + 8));
            }
        }
    } else if (items <= kThreads * kHeldItems) {
        // the block held in registers as its bf16 wire pairs (k | v << 16):
        // one read of the pages, the absmax over the held values, then codes
        u32x4 wlo[kHeldItems], whi[kHeldItems];
        float m = 0.0f;
#pragma unroll
        for (int u = 0; u < kHeldItems; ++u) {
            const int it = threadIdx.x + u * kThreads;
            wlo[u] = whi[u] = u32x4{0, 0, 0, 0};
            if (it < items) {
                float k[8], v[8];
                (void)load_item(it, k, v);
                interleave(k, v, wlo[u], whi[u]);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    m = absmax_step(m, __uint_as_float(wlo[u][j] << 16));
                    m = absmax_step(m, __uint_as_float(wlo[u][j] & 0xFFFF0000u));
                    m = absmax_step(m, __uint_as_float(whi[u][j] << 16));
                    m = absmax_step(m, __uint_as_float(whi[u][j] & 0xFFFF0000u));
                }
            }
        }
        const float max_val = block_absmax(m, s_red);
        float scale, inv;
        {
#pragma clang fp contract(off)
            scale = max_val > 0.0f ? max_val / 127.0f : 1.0f;
            inv = 1.0f / scale;
        }
        int8_t *out = a.codes + (int64_t)blockIdx.x * wire_elems;
#pragma unroll
        for (int u = 0; u < kHeldItems; ++u) {
            const int it = threadIdx.x + u * kThreads;
            if (it >= items) break;
            const int t = it / (a.n_kv_heads * chunks);
            const int rem = it - t * a.n_kv_heads * chunks;
            const int h = rem / chunks, c = rem - h * chunks;
            const int64_t we = (((int64_t)t * a.n_kv_heads + h) * a.head_dim + 8 * c) * 2;
            u32x4 q;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t p0 = j < 2 ? wlo[u][2 * j] : whi[u][2 * j - 4];
                const uint32_t p1 = j < 2 ? wlo[u][2 * j + 1] : whi[u][2 * j - 3];
                const uint32_t c0 = (uint8_t)pd_code(__uint_as_float(p0 << 16), inv);
                const uint32_t c1 = (uint8_t)pd_code(__uint_as_float(p0 & 0xFFFF0000u), inv);
                const uint32_t c2 = (uint8_t)pd_code(__uint_as_float(p1 << 16), inv);
                const uint32_t c3 = (uint8_t)pd_code(__uint_as_float(p1 & 0xFFFF0000u), inv);
                q[j] = c0 | (c1 << 8) | (c2 << 16) | (c3 << 24);
            }
            __builtin_nontemporal_store(q, reinterpret_cast<u32x4 *>(out + we));
        }
        if (threadIdx.x == 0) a.wire_scales[blockIdx.x] = scale;
    } else {
        // larger blocks: pass 1 takes the absmax of the bf16 wire values,
        // pass 2 reads the pages again
        float m = 0.0f;
        for (int it = threadIdx.x; it < items; it += kThreads) {
            float k[8], v[8];
            (void)load_item(it, k, v);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                m = absmax_step(m, bf16_to_f32(bf16_rne(k[j])));
                m = absmax_step(m, bf16_to_f32(bf16_rne(v[j])));
            }
        }
        const float max_val = block_absmax(m, s_red);
        float scale, inv;
        {
#pragma clang fp contract(off)
            scale = max_val > 0.0f ? max_val / 127.0f : 1.0f;
            inv = 1.0f / scale;
        }
        int8_t *out = a.codes + (int64_t)blockIdx.x * wire_elems;
        for (int it = threadIdx.x; it < items; it += kThreads) {
            float k[8], v[8];
            const int64_t we = load_item(it, k, v);
            u32x4 q;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                uint32_t w = 0;
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const int i = 2 * j + e;
                    const uint32_t kc = (uint8_t)pd_code(bf16_to_f32(bf16_rne(k[i])), inv);
                    const uint32_t vc = (uint8_t)pd_code(bf16_to_f32(bf16_rne(v[i])), inv);
                    w |= (kc | (vc << 8)) << (16 * e);
                }
                q[j] = w;
            }
            __builtin_nontemporal_store(q, reinterpret_cast<u32x4 *>(out + we));
        }
        if (threadIdx.x == 0) a.wire_scales[blockIdx.x] = scale;
    }
}

template <int DT>
__global__ __launch_bounds__(kThreads) void kv_unpack_kernel(WireArgs a) {
    const int32_t blk = a.ids[blockIdx.x];
    if (blk < 0 || blk >= a.num_blocks) {
        if (threadIdx.x == 0) atomicAdd(a.errors, 1ull);
        return;
    }
    const int chunks = a.head_dim / 8;
    const int items = a.block_size * a.n_kv_heads * chunks;
    const int64_t wire_elems = (int64_t)a.block_size * a.n_kv_heads * a.head_dim * 2;
    const uint16_t *in = (const uint16_t *)a.wire + (int64_t)blockIdx.x * wire_elems;
    const int ng = (DT == AIR_KV_INT8 || DT == AIR_KV_FP8) ? a.head_dim / a.scale_group : 1;
    const int lanes = (DT == AIR_KV_INT8 || DT == AIR_KV_FP8) ? a.scale_group / 8 : 1;
    // items are walked in whole rounds so every lane of a scale group (which
    // share a row: chunks is a multiple of lanes) joins the shuffles; the
    // wire pieces of kHeldItems rounds are loaded before any is stored
    for (int base0 = 0; base0 < items; base0 += kThreads * kHeldItems) {
        u32x4 wlo[kHeldItems], whi[kHeldItems];
#pragma unroll
        for (int u = 0; u < kHeldItems; ++u) {
            const int it = base0 + u * kThreads + (int)threadIdx.x;
            const int itc = it < items ? it : 0;
            const int t = itc / (a.n_kv_heads * chunks);
            const int rem = itc - t * a.n_kv_heads * chunks;
            const int h = rem / chunks, c = rem - h * chunks;
            const int64_t we = (((int64_t)t * a.n_kv_heads + h) * a.head_dim + 8 * c) * 2;
            wlo[u] = *reinterpret_cast<const u32x4 *>(in + we);
            whi[u] = *reinterpret_cast<const u32x4 *>(in + we + 8);
        }
#pragma unroll
        for (int u = 0; u < kHeldItems; ++u) {
            const int base = base0 + u * kThreads;
            if (base >= items) break;
            const int it = base + (int)threadIdx.x;
            const bool valid = it < items;
            const int itc = valid ? it : 0;
            const int t = itc / (a.n_kv_heads * chunks);
            const int rem = itc - t * a.n_kv_heads * chunks;
            const int h = rem / chunks, c = rem - h * chunks;
            const u32x4 lo = wlo[u], hi = whi[u];
            float k[8], v[8];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                k[j] = __uint_as_float(lo[j] << 16);
                v[j] = __uint_as_float(lo[j] & 0xFFFF0000u);
                k[4 + j] = __uint_as_float(hi[j] << 16);
                v[4 + j] = __uint_as_float(hi[j] & 0xFFFF0000u);
            }
            const int64_t row = ((int64_t)blk * a.n_kv_heads + h) * a.block_size + t;
            const int64_t elem = row * a.head_dim + 8 * c;
            const int64_t sidx = row * ng + (8 * c) / (a.scale_group > 0 ? a.scale_group : 1);
            const bool lead = (c % lanes) == 0;
            store_row_chunk<DT>(k, a.k_pages, a.k_scales, elem, sidx, lead, lanes, valid);
            store_row_chunk<DT>(v, a.v_pages, a.v_scales, elem, sidx, lead, lanes, valid);
        }
    }
}

// KvBlock::int8_quantize over n wire blocks already in device memory.
__global__ __launch_bounds__(kThreads) void wire_int8_kernel(const uint16_t *wire, int64_t elems,
                                                              int8_t *codes, float *scales) {
    __shared__ float s_red[kThreads / 64];
    const uint16_t *in = wire + (int64_t)blockIdx.x * elems;
    int8_t *out = codes + (int64_t)blockIdx.x * elems;
    float m = 0.0f;
    for (int64_t i = threadIdx.x; i < elems; i += kThreads) m = absmax_step(m, bf16_to_f32(in[i]));
    const float max_val = block_absmax(m, s_red);
    float scale, inv;
    {
#pragma clang fp contract(off)
        scale = max_val > 0.0f ? max_val / 127.0f : 1.0f;
        inv = 1.0f / scale;
    }
    for (int64_t i = threadIdx.x; i < elems; i += kThreads) out[i] = pd_code(bf16_to_f32(in[i]), inv);
    if (threadIdx.x == 0) scales[blockIdx.x] = scale;
}

WireArgs wire_args(const air_kv_pool &p, const int32_t *ids, int32_t n) {
    WireArgs a;
    a.ids = ids; a.n = n;
    a.n_kv_heads = p.desc.n_kv_heads; a.head_dim = p.desc.head_dim;
    a.block_size = p.desc.block_size; a.scale_group = p.desc.scale_group;
    a.num_blocks = p.desc.num_blocks;
    a.k_pages = p.k_pages; a.v_pages = p.v_pages;
    a.k_scales = p.k_scales; a.v_scales = p.v_scales;
    a.wire = nullptr; a.codes = nullptr; a.wire_scales = nullptr;
    a.errors = p.errors;
    auto magic = [](uint32_t d) { return d <= 1 ? 0u : (uint32_t)(((1ull << 32) + d - 1) / d); };
    a.chunks_magic = magic((uint32_t)p.desc.head_dim / 8);
    a.heads_magic = magic((uint32_t)p.desc.n_kv_heads);
    return a;
}

// The bf16 kernels' divisions are exact while a block's item count times
// the divisor stays below 2^32 (any pool the allocator accepts).
bool segment_path(const air_kv_pool &p) {
    const uint64_t items = (uint64_t)p.desc.block_size * p.desc.n_kv_heads * (p.desc.head_dim / 8);
    const uint64_t d = (uint64_t)(p.desc.head_dim / 8 > p.desc.n_kv_heads ? p.desc.head_dim / 8 : p.desc.n_kv_heads);
    return p.desc.dtype == AIR_KV_BF16 && p.desc.head_dim % 8 == 0 && items * d < (1ull << 32);
}

template <bool INT8>
hipError_t pack_dt(const air_kv_pool &p, hipStream_t s, const WireArgs &a) {
    const dim3 grid((unsigned)a.n);
    if (!INT8 && segment_path(p)) {
        hipLaunchKernelGGL(kv_pack_bf16_kernel, grid, dim3(kThreads), 0, s, a);
        return hipGetLastError();
    }
    switch (p.desc.dtype) {
    case AIR_KV_F32: hipLaunchKernelGGL((kv_pack_kernel<AIR_KV_F32, INT8>), grid, dim3(kThreads), 0, s, a); break;
    case AIR_KV_BF16: hipLaunchKernelGGL((kv_pack_kernel<AIR_KV_BF16, INT8>), grid, dim3(kThreads), 0, s, a); break;
    case AIR_KV_INT8: hipLaunchKernelGGL((kv_pack_kernel<AIR_KV_INT8, INT8>), grid, dim3(kThreads), 0, s, a); break;
    default: hipLaunchKernelGGL((kv_pack_kernel<AIR_KV_FP8, INT8>), grid, dim3(kThreads), 0, s, a); break;
    }
    return hipGetLastError();
}

}  // namespace

size_t wire_block_bytes(const air_kv_pool &p) {
    return (size_t)p.desc.block_size * p.desc.n_kv_heads * p.desc.head_dim * 2 * 2;
}

hipError_t launch_pack_blocks(const air_kv_pool &p, hipStream_t s, const int32_t *ids, int32_t n,
                              void *out) {
    WireArgs a = wire_args(p, ids, n);
    a.wire = out;
    return pack_dt<false>(p, s, a);
}

hipError_t launch_pack_blocks_int8(const air_kv_pool &p, hipStream_t s, const int32_t *ids, int32_t n,
                                   int8_t *codes, float *scales) {
    WireArgs a = wire_args(p, ids, n);
    a.codes = codes;
    a.wire_scales = scales;
    const uint64_t items = (uint64_t)p.desc.block_size * p.desc.n_kv_heads * (p.desc.head_dim / 8);
    if (segment_path(p) && items <= (uint64_t)kQThreads * kQItems) {
        // persistent: two workgroups (16 waves) per CU
        const int64_t g = (int64_t)p.cus * 2;
        hipLaunchKernelGGL(kv_pack_int8_bf16_kernel, dim3((unsigned)(n < g ? n : g)), dim3(kQThreads), 0, s, a);
        return hipGetLastError();
    }
    return pack_dt<true>(p, s, a);
}

hipError_t launch_unpack_blocks(const air_kv_pool &p, hipStream_t s, const int32_t *ids, int32_t n,
                                const void *in) {
    WireArgs a = wire_args(p, ids, n);
    a.wire = const_cast<void *>(in);
    const dim3 grid((unsigned)n);
    if (segment_path(p)) {
        hipLaunchKernelGGL(kv_unpack_bf16_kernel, grid, dim3(kThreads), 0, s, a);
        return hipGetLastError();
    }
    switch (p.desc.dtype) {
    case AIR_KV_F32: hipLaunchKernelGGL((kv_unpack_kernel<AIR_KV_F32>), grid, dim3(kThreads), 0, s, a); break;
    case AIR_KV_BF16: hipLaunchKernelGGL((kv_unpack_kernel<AIR_KV_BF16>), grid, dim3(kThreads), 0, s, a); break;
    case AIR_KV_INT8: hipLaunchKernelGGL((kv_unpack_kernel<AIR_KV_INT8>), grid, dim3(kThreads), 0, s, a); break;
    default: hipLaunchKernelGGL((kv_unpack_kernel<AIR_KV_FP8>), grid, dim3(kThreads), 0, s, a); break;
    }
    return hipGetLastError();
}

hipError_t launch_wire_int8(hipStream_t s, const void *wire, int32_t n_blocks, int64_t elems,
                            int8_t *codes, float *scales) {
    hipLaunchKernelGGL(wire_int8_kernel, dim3((unsigned)n_blocks), dim3(kThreads), 0, s,
                       (const uint16_t *)wire, elems, codes, scales);
    return hipGetLastError();
}

}  // namespace airkv
