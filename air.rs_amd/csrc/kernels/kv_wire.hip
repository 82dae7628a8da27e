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

#include "../pool.hpp"
#include "codecs.hpp"
#include "page_io.hpp"

namespace airkv {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

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
};

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
    return a;
}

template <bool INT8>
hipError_t pack_dt(const air_kv_pool &p, hipStream_t s, const WireArgs &a) {
    const dim3 grid((unsigned)a.n);
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
    return pack_dt<true>(p, s, a);
}

hipError_t launch_unpack_blocks(const air_kv_pool &p, hipStream_t s, const int32_t *ids, int32_t n,
                                const void *in) {
    WireArgs a = wire_args(p, ids, n);
    a.wire = const_cast<void *>(in);
    const dim3 grid((unsigned)n);
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
