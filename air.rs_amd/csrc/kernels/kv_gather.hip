// Gather: pages -> one contiguous view per sequence (dequantizing INT8/FP8).
//
// Work is the flat list of (sequence, page) pairs of every live sequence, so
// variable lengths cost nothing: each workgroup builds the exclusive prefix
// sum of pages-per-sequence in LDS once, then walks the page list with a grid
// stride, finding a page's sequence by binary search.  A page is block_size
// rows of head_dim elements of K and of V for every kv head; each thread
// moves 8 elements (a 16-byte bf16 load) per tensor and head, so the 16 x 128
// rows of one head are one pass of 256 threads, four heads at a time.
#include <hip/hip_runtime.h>

#include "../pool.hpp"
#include "codecs.hpp"
#include "page_io.hpp"

#ifndef AIRKV_GATHER_WGS_PER_CU
#define AIRKV_GATHER_WGS_PER_CU 32         // build-time tuning knob: workgroups per CU in the grid (8 resident)
#endif

namespace airkv {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;
constexpr int kMaxSeqsPerLaunch = 4096;   // LDS prefix: 16 KB

struct GatherArgs {
    const int32_t *tables, *lens;
    const int64_t *out_offsets;
    int32_t batch, max_blocks;
    int32_t n_kv_heads, head_dim, block_size, scale_group;
    int64_t num_blocks;
    const void *k_pages, *v_pages;
    const float *k_scales, *v_scales;
    void *out_k, *out_v;
    int32_t layout;
    unsigned long long *errors;
};

template <int DT, int OUT>
__device__ __forceinline__ void store8(void *out, int64_t elem, const float (&x)[8], u32x4 raw) {
    if constexpr (OUT == AIR_KV_F32) {
        f32x4 *o = reinterpret_cast<f32x4 *>((float *)out + elem);
        __builtin_nontemporal_store(f32x4{x[0], x[1], x[2], x[3]}, o);
        __builtin_nontemporal_store(f32x4{x[4], x[5], x[6], x[7]}, o + 1);
    } else if constexpr (DT == AIR_KV_BF16) {
        // raw bits, no re-rounding
        __builtin_nontemporal_store(raw, reinterpret_cast<u32x4 *>((uint16_t *)out + elem));
    } else {
        u32x4 w;
        w[0] = (uint32_t)bf16_rne(x[0]) | ((uint32_t)bf16_rne(x[1]) << 16);
        w[1] = (uint32_t)bf16_rne(x[2]) | ((uint32_t)bf16_rne(x[3]) << 16);
        w[2] = (uint32_t)bf16_rne(x[4]) | ((uint32_t)bf16_rne(x[5]) << 16);
        w[3] = (uint32_t)bf16_rne(x[6]) | ((uint32_t)bf16_rne(x[7]) << 16);
        __builtin_nontemporal_store(w, reinterpret_cast<u32x4 *>((uint16_t *)out + elem));
    }
}

// Page -> 4 f32 (one 16-byte output store): 4 consecutive elements of one row,
// dequantized as load8 does (INT8/FP8: q as f32 * scale, src/kv_cache.rs:88,
// src/fp8.rs:263-264; BF16 widened exactly; F32 as stored).
template <int DT>
__device__ __forceinline__ f32x4 load4(const void *pages, const float *scales, int64_t elem, int64_t scale_idx) {
    if constexpr (DT == AIR_KV_F32) {
        return __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>((const float *)pages + elem));
    } else if constexpr (DT == AIR_KV_BF16) {
        const u32x2 w = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>((const uint16_t *)pages + elem));
        return f32x4{__uint_as_float(w[0] << 16), __uint_as_float(w[0] & 0xFFFF0000u),
                     __uint_as_float(w[1] << 16), __uint_as_float(w[1] & 0xFFFF0000u)};
    } else {
        const uint32_t w = __builtin_nontemporal_load((const uint32_t *)((const uint8_t *)pages + elem));
        const float sc = scales[scale_idx];
        f32x4 x;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t byte = (w >> (8 * j)) & 0xFFu;
            float val;
            if constexpr (DT == AIR_KV_INT8) val = (float)(int32_t)(int8_t)byte;
            else val = fp8_decode(byte);
            {
#pragma clang fp contract(off)
                x[j] = val * sc;
            }
        }
        return x;
    }
}

template <int DT, int OUT>
__global__ __launch_bounds__(kThreads) void kv_gather_kernel(GatherArgs a) {
    __shared__ int32_t s_prefix[kMaxSeqsPerLaunch + 1];
    __shared__ int32_t s_wave_tot[kThreads / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t max_len = (int64_t)a.max_blocks * a.block_size;

    // exclusive prefix of pages per sequence, kThreads sequences per round
    int32_t carry = 0;
    for (int base = 0; base < a.batch; base += kThreads) {
        const int b = base + tid;
        int32_t pages = 0;
        if (b < a.batch) {
            int64_t len = a.lens[b];
            len = len < 0 ? 0 : (len > max_len ? max_len : len);
            pages = (int32_t)((len + a.block_size - 1) / a.block_size);
        }
        int32_t incl = pages;
        for (int off = 1; off < 64; off <<= 1) {
            int32_t y = __shfl_up(incl, off);
            if (lane >= off) incl += y;
        }
        if (lane == 63) s_wave_tot[wave] = incl;
        __syncthreads();
        int32_t before = carry;
        for (int w = 0; w < wave; ++w) before += s_wave_tot[w];
        if (b < a.batch) s_prefix[b] = before + incl - pages;
        int32_t round_total = 0;
        for (int w = 0; w < kThreads / 64; ++w) round_total += s_wave_tot[w];
        carry += round_total;
        __syncthreads();
    }
    if (tid == 0) s_prefix[a.batch] = carry;
    __syncthreads();
    // count malformed lengths once
    if (blockIdx.x == 0) {
        for (int b = tid; b < a.batch; b += kThreads) {
            int32_t len = a.lens[b];
            if (len < 0 || len > max_len) atomicAdd(a.errors, 1ull);
        }
    }

    // One page of one sequence per step, all kv heads: the page's table
    // entry, length and output offset are looked up once, and each thread
    // keeps kHeadUnroll heads' K and V loads in flight before storing them.
    constexpr int kHeadUnroll = 4;
    const int rows = a.block_size, d = a.head_dim;
    const int tile_elems = rows * d;
    const int ng = DT == AIR_KV_INT8 || DT == AIR_KV_FP8 ? d / a.scale_group : 1;
    for (int64_t page_g = blockIdx.x; page_g < carry; page_g += gridDim.x) {
        // sequence owning global page index page_g: last b with prefix[b] <= page_g
        int lo = 0, hi = a.batch - 1;
        while (lo < hi) {
            int mid = (lo + hi + 1) >> 1;
            if (s_prefix[mid] <= page_g) lo = mid; else hi = mid - 1;
        }
        const int b = lo;
        const int32_t p = (int32_t)(page_g - s_prefix[b]);
        int64_t len = a.lens[b];
        len = len > max_len ? max_len : len;
        const int32_t blk = a.tables[(int64_t)b * a.max_blocks + p];
        if (blk < 0 || blk >= a.num_blocks) {     // one count per (page, kv head)
            if (tid == 0) atomicAdd(a.errors, (unsigned long long)a.n_kv_heads);
            continue;
        }
        const int64_t out_base = a.out_offsets[b];
        if constexpr (OUT == AIR_KV_F32) {
            // f32 outputs: lane l of a wave takes 4 elements at 4l and 4 at
            // 256 + 4l of the wave's 512, so each 16-byte store instruction
            // writes 1 KB of whole cache lines (8 elements per lane as two
            // stores 16 bytes apart left every instruction half of each line)
            const int wbase = (tid >> 6) * 512 + 4 * lane;
            for (int e0 = wbase; e0 < tile_elems; e0 += kThreads * 8) {
                for (int h0 = 0; h0 < a.n_kv_heads; h0 += kHeadUnroll) {
                    f32x4 xk[kHeadUnroll][2], xv[kHeadUnroll][2];
#pragma unroll
                    for (int half = 0; half < 2; ++half) {
                        const int e = e0 + 256 * half;
                        const int r = e / d, col = e - r * d;
#pragma unroll
                        for (int u = 0; u < kHeadUnroll; ++u) {
                            const int h = h0 + u < a.n_kv_heads ? h0 + u : a.n_kv_heads - 1;
                            const int64_t src_row = ((int64_t)blk * a.n_kv_heads + h) * rows + r;
                            const int64_t src = src_row * d + col;
                            const int64_t sidx = src_row * ng + col / (a.scale_group > 0 ? a.scale_group : 1);
                            xk[u][half] = load4<DT>(a.k_pages, a.k_scales, src, sidx);
                            xv[u][half] = load4<DT>(a.v_pages, a.v_scales, src, sidx);
                        }
                    }
#pragma unroll
                    for (int half = 0; half < 2; ++half) {
                        const int e = e0 + 256 * half;
                        const int r = e / d, col = e - r * d;
                        const int64_t t = (int64_t)p * rows + r;
                        if (e >= tile_elems || t >= len) continue;
#pragma unroll
                        for (int u = 0; u < kHeadUnroll; ++u) {
                            const int h = h0 + u;
                            if (h >= a.n_kv_heads) break;
                            const int64_t dst = out_base + (a.layout == AIR_KV_LAYOUT_HEAD_MAJOR
                                                                ? ((int64_t)h * len + t) * d + col
                                                                : (t * a.n_kv_heads + h) * d + col);
                            __builtin_nontemporal_store(xk[u][half], reinterpret_cast<f32x4 *>((float *)a.out_k + dst));
                            __builtin_nontemporal_store(xv[u][half], reinterpret_cast<f32x4 *>((float *)a.out_v + dst));
                        }
                    }
                }
            }
            continue;
        }
        for (int e = tid * 8; e < tile_elems; e += kThreads * 8) {
            const int r = e / d, col = e - r * d;
            const int64_t t = (int64_t)p * rows + r;
            if (t >= len) continue;
            for (int h0 = 0; h0 < a.n_kv_heads; h0 += kHeadUnroll) {
                float xk[kHeadUnroll][8], xv[kHeadUnroll][8];
                u32x4 rk[kHeadUnroll], rv[kHeadUnroll];
#pragma unroll
                for (int u = 0; u < kHeadUnroll; ++u) {
                    const int h = h0 + u < a.n_kv_heads ? h0 + u : a.n_kv_heads - 1;
                    const int64_t src_row = ((int64_t)blk * a.n_kv_heads + h) * rows + r;
                    const int64_t src = src_row * d + col;
                    const int64_t sidx = src_row * ng + col / (a.scale_group > 0 ? a.scale_group : 1);
                    rk[u] = rv[u] = u32x4{0, 0, 0, 0};
                    load8<DT>(a.k_pages, a.k_scales, src, sidx, xk[u], &rk[u]);
                    load8<DT>(a.v_pages, a.v_scales, src, sidx, xv[u], &rv[u]);
                }
#pragma unroll
                for (int u = 0; u < kHeadUnroll; ++u) {
                    const int h = h0 + u;
                    if (h >= a.n_kv_heads) break;
                    const int64_t dst = out_base + (a.layout == AIR_KV_LAYOUT_HEAD_MAJOR
                                                        ? ((int64_t)h * len + t) * d + col
                                                        : (t * a.n_kv_heads + h) * d + col);
                    store8<DT, OUT>(a.out_k, dst, xk[u], rk[u]);
                    store8<DT, OUT>(a.out_v, dst, xv[u], rv[u]);
                }
            }
        }
    }
}

template <int DT>
void dispatch_out(int out_dtype, dim3 grid, hipStream_t s, const GatherArgs &a) {
    if (out_dtype == AIR_KV_F32)
        hipLaunchKernelGGL((kv_gather_kernel<DT, AIR_KV_F32>), grid, dim3(kThreads), 0, s, a);
    else
        hipLaunchKernelGGL((kv_gather_kernel<DT, AIR_KV_BF16>), grid, dim3(kThreads), 0, s, a);
}

}  // namespace

hipError_t launch_gather(const air_kv_pool &p, hipStream_t s, const int32_t *tables,
                         const int32_t *lens, const int64_t *out_offsets, int32_t batch,
                         int32_t max_blocks, void *out_k, void *out_v, int32_t out_dtype,
                         int32_t out_layout) {
    const int cus = p.cus;
    for (int32_t b0 = 0; b0 < batch; b0 += kMaxSeqsPerLaunch) {
        const int32_t nb = batch - b0 < kMaxSeqsPerLaunch ? batch - b0 : kMaxSeqsPerLaunch;
        GatherArgs a;
        a.tables = tables + (int64_t)b0 * max_blocks;
        a.lens = lens + b0;
        a.out_offsets = out_offsets + b0;
        a.batch = nb;
        a.max_blocks = max_blocks;
        a.n_kv_heads = p.desc.n_kv_heads; a.head_dim = p.desc.head_dim;
        a.block_size = p.desc.block_size; a.scale_group = p.desc.scale_group;
        a.num_blocks = p.desc.num_blocks;
        a.k_pages = p.k_pages; a.v_pages = p.v_pages;
        a.k_scales = p.k_scales; a.v_scales = p.v_scales;
        a.out_k = out_k; a.out_v = out_v;
        a.layout = out_layout;
        a.errors = p.errors;
        dim3 grid((unsigned)(cus * AIRKV_GATHER_WGS_PER_CU));
        switch (p.desc.dtype) {
        case AIR_KV_F32: dispatch_out<AIR_KV_F32>(out_dtype, grid, s, a); break;
        case AIR_KV_BF16: dispatch_out<AIR_KV_BF16>(out_dtype, grid, s, a); break;
        case AIR_KV_INT8: dispatch_out<AIR_KV_INT8>(out_dtype, grid, s, a); break;
        default: dispatch_out<AIR_KV_FP8>(out_dtype, grid, s, a); break;
        }
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace airkv
