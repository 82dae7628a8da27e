// Reshape-and-cache: scatter new K/V rows into their pages, converting or
// quantizing on the way (the paged replacement of the Tensor::cat append at
// src/model.rs:569 and of save_layer's Q8 quantize, src/kv_cache.rs:307-315).
//
// One thread owns 8 consecutive head_dim elements of one (token, kv head) row
// and handles both K and V: two 32-byte f32 loads each, one 32/16/8-byte store
// each.  Consecutive threads cover a row, then the same head of the next
// token (four tokens per wave at head_dim 128), so a wave writes one
// contiguous run of page rows when its tokens share a block and reads four
// whole source rows.  For INT8/FP8 the
// scale_group/8 lanes of one scale group reduce their absmax with butterfly
// shuffles; the group's first lane stores the f32 scale.
#include <hip/hip_runtime.h>

#include "../pool.hpp"
#include "codecs.hpp"
#include "fastdiv.hpp"
#include "page_io.hpp"

namespace airkv {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;

struct AppendArgs {
    const float *k, *v;
    const int64_t *slots;
    int64_t n_tokens;
    int64_t num_slots;       // num_blocks * block_size
    int32_t n_kv_heads, head_dim, block_size, scale_group;
    void *k_pages, *v_pages;
    float *k_scales, *v_scales;
    unsigned long long *errors;
    // a launch's work-items count in 32 bits; its divisions by head_dim / 8
    // and n_kv_heads are invariant-divisor multiplies, the power-of-two
    // block size and scale group shifts
    FastDiv chunks_div, heads_div;
    int32_t bs_log2, sg_log2;
};

// F32 / BF16 pages, head_dim 128: each wave covers four consecutive tokens of
// one head as above, but lane l moves 4 elements at 4l and 4 at 256 + 4l of
// the wave's 512, so every 16-byte source load instruction reads two whole
// 512-byte rows and every page store instruction writes two whole page rows
// (8 consecutive elements per lane made each load instruction read half of
// every cache line it touched).
template <int DT>
__global__ __launch_bounds__(kThreads) void kv_append_rows_kernel(AppendArgs a) {
    static_assert(DT == AIR_KV_F32 || DT == AIR_KV_BF16, "unquantized pages");
    constexpr int D = 128;
    const int lane = threadIdx.x & 63;
    const uint32_t wave_g = (blockIdx.x * kThreads + threadIdx.x) >> 6;   // (token group of 4, head)
    const uint32_t tg = fast_div(wave_g, a.heads_div);
    const int h = (int)(wave_g - tg * (uint32_t)a.n_kv_heads);
    const int64_t t0 = (int64_t)tg * 4;
    f32x4 kx[2], vx[2];
    int64_t dst[2];
    bool ok[2];
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        const int e = 256 * half + 4 * lane;               // element of the wave's four rows
        const int64_t t = t0 + e / D;
        const int col = e % D;
        const bool active = t < a.n_tokens;
        const int64_t slot = active ? a.slots[t] : -1;
        ok[half] = slot >= 0 && slot < a.num_slots;
        if (active && slot >= a.num_slots && col == 0 && h == 0) atomicAdd(a.errors, 1ull);
        const int64_t src = (active ? t * a.n_kv_heads + h : 0) * D + col;
        kx[half] = active ? __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(a.k + src)) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        vx[half] = active ? __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(a.v + src)) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        const int64_t blk = ok[half] ? slot >> a.bs_log2 : 0;
        const int64_t off = ok[half] ? slot & (a.block_size - 1) : 0;
        dst[half] = ((blk * a.n_kv_heads + h) * a.block_size + off) * D + col;
    }
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        if (!ok[half]) continue;
        if constexpr (DT == AIR_KV_F32) {
            pio_store(kx[half], reinterpret_cast<f32x4 *>((float *)a.k_pages + dst[half]));
            pio_store(vx[half], reinterpret_cast<f32x4 *>((float *)a.v_pages + dst[half]));
        } else {
            const f32x4 k = kx[half], v = vx[half];
            pio_store(u32x2{(uint32_t)bf16_rne(k[0]) | ((uint32_t)bf16_rne(k[1]) << 16),
                            (uint32_t)bf16_rne(k[2]) | ((uint32_t)bf16_rne(k[3]) << 16)},
                      reinterpret_cast<u32x2 *>((uint16_t *)a.k_pages + dst[half]));
            pio_store(u32x2{(uint32_t)bf16_rne(v[0]) | ((uint32_t)bf16_rne(v[1]) << 16),
                            (uint32_t)bf16_rne(v[2]) | ((uint32_t)bf16_rne(v[3]) << 16)},
                      reinterpret_cast<u32x2 *>((uint16_t *)a.v_pages + dst[half]));
        }
    }
}

// The whole-line form of the source loads below (head_dim 128: a wave is
// four tokens of one head, lane 16 tl + c owning elements 8c .. 8c + 7 of
// token tl): load i gives lane l 16-byte piece 2 (l & 15) + (l >> 5) of token
// 2i + ((l >> 4) & 1)'s row, so each load instruction reads two whole
// 512-byte rows; exchanging lane bit 5 with the load index (the lane swap
// across the wave's halves) then leaves lane 16 tl + c holding pieces 2c and
// 2c + 1 of token tl, the layout the quantizer works on.  With each lane
// loading its own two pieces, every load instruction read half of every line
// it touched.
__device__ __forceinline__ void swap_halves(f32x4 &x0, f32x4 &x1) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x0[j]), __float_as_uint(x1[j]), false, false);
        x0[j] = __uint_as_float(r[0]);
        x1[j] = __uint_as_float(r[1]);
    }
}

template <int DT, bool LINES>
__global__ __launch_bounds__(kThreads) void kv_append_kernel(AppendArgs a) {
    // thread -> (chunk c, token t % 4, kv head h, token t / 4), chunk fastest:
    // 4 * chunks consecutive threads (a wave at head_dim 128) cover four
    // consecutive tokens of one head, whose page rows are one contiguous run
    // when the tokens share a block (prefill chunks)
    const uint32_t chunks = (uint32_t)a.head_dim >> 3;
    const uint32_t gid = blockIdx.x * kThreads + threadIdx.x;
    const uint32_t rest = fast_div(gid, a.chunks_div);
    const int c = (int)(gid - rest * chunks);
    const int tl = (int)(rest & 3);
    const uint32_t rest2 = rest >> 2;
    const uint32_t tq = fast_div(rest2, a.heads_div);
    const int h = (int)(rest2 - tq * (uint32_t)a.n_kv_heads);
    const int64_t t = (int64_t)tq * 4 + tl;
    const bool active = t < a.n_tokens;
    const int64_t row = t * a.n_kv_heads + h;
    const int64_t slot = active ? a.slots[t] : -1;
    const bool valid = slot >= 0 && slot < a.num_slots;
    if (active && slot >= a.num_slots && c == 0 && h == 0) atomicAdd(a.errors, 1ull);

    // the source rows are loaded whatever the slot turns out to be (every
    // token's row exists), so their loads overlap the slot load instead of
    // waiting for it
    float kx[8], vx[8];
    if constexpr (LINES) {
        // head_dim 128, whole-line loads (above); a lane loads for token
        // 2i + ((lane >> 4) & 1) of its wave's four, which may differ from
        // its own
        const int lane = threadIdx.x & 63;
        const int64_t tw = t - tl;                           // the wave's first token
        f32x4 kr[2], vr[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int64_t ts = tw + 2 * i + ((lane >> 4) & 1);
            const int64_t src = (ts * a.n_kv_heads + h) * 128 + 4 * (2 * (lane & 15) + (lane >> 5));
            kr[i] = ts < a.n_tokens ? __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(a.k + src))
                                    : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            vr[i] = ts < a.n_tokens ? __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(a.v + src))
                                    : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
        swap_halves(kr[0], kr[1]);
        swap_halves(vr[0], vr[1]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            kx[j] = valid ? kr[0][j] : 0.0f; kx[4 + j] = valid ? kr[1][j] : 0.0f;
            vx[j] = valid ? vr[0][j] : 0.0f; vx[4 + j] = valid ? vr[1][j] : 0.0f;
        }
    } else if (active) {
        const f32x4 *ks = reinterpret_cast<const f32x4 *>(a.k + row * a.head_dim + c * 8);
        const f32x4 *vs = reinterpret_cast<const f32x4 *>(a.v + row * a.head_dim + c * 8);
        const f32x4 k0 = __builtin_nontemporal_load(ks), k1 = __builtin_nontemporal_load(ks + 1);
        const f32x4 v0 = __builtin_nontemporal_load(vs), v1 = __builtin_nontemporal_load(vs + 1);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            kx[j] = valid ? k0[j] : 0.0f; kx[4 + j] = valid ? k1[j] : 0.0f;
            vx[j] = valid ? v0[j] : 0.0f; vx[4 + j] = valid ? v1[j] : 0.0f;
        }
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) kx[j] = vx[j] = 0.0f;
    }
    const int64_t blk = valid ? slot >> a.bs_log2 : 0;
    const int64_t off = valid ? slot & (a.block_size - 1) : 0;
    const int64_t dst_row = (blk * a.n_kv_heads + h) * a.block_size + off;
    const int64_t elem = dst_row * a.head_dim + c * 8;
    int lanes_per_group = 1;
    int64_t scale_idx = 0;
    bool lead = false;
    if constexpr (DT == AIR_KV_INT8 || DT == AIR_KV_FP8) {
        lanes_per_group = a.scale_group >> 3;
        scale_idx = dst_row * (a.head_dim >> a.sg_log2) + ((c * 8) >> a.sg_log2);
        lead = (c & (lanes_per_group - 1)) == 0;
    }
    store_row_chunk<DT>(kx, a.k_pages, a.k_scales, elem, scale_idx, lead, lanes_per_group, valid);
    store_row_chunk<DT>(vx, a.v_pages, a.v_scales, elem, scale_idx, lead, lanes_per_group, valid);
}

}  // namespace

hipError_t launch_append(const air_kv_pool &p, hipStream_t s, const float *k, const float *v,
                         const int64_t *slots, int32_t n_tokens) {
    AppendArgs a;
    a.k = k; a.v = v; a.slots = slots;
    a.n_tokens = n_tokens;
    a.num_slots = p.desc.num_blocks * p.desc.block_size;
    a.n_kv_heads = p.desc.n_kv_heads; a.head_dim = p.desc.head_dim;
    a.block_size = p.desc.block_size; a.scale_group = p.desc.scale_group;
    a.k_pages = p.k_pages; a.v_pages = p.v_pages;
    a.k_scales = p.k_scales; a.v_scales = p.v_scales;
    a.errors = p.errors;
    a.chunks_div = make_fast_div((uint32_t)p.desc.head_dim / 8);
    a.heads_div = make_fast_div((uint32_t)p.desc.n_kv_heads);
    a.bs_log2 = __builtin_ctz((unsigned)p.desc.block_size);              // 16 or 32
    a.sg_log2 = p.desc.scale_group > 0 ? __builtin_ctz((unsigned)p.desc.scale_group) : 0;   // a power of two
    // a dispatch counts its work-items in 32 bits: long appends take several
    // launches of at most kMaxBlocks workgroups, each a whole number of
    // four-token groups
    constexpr int64_t kMaxBlocks = ((int64_t)1 << 32) / kThreads - 1;
    const int64_t per_token = (int64_t)p.desc.n_kv_heads * (p.desc.head_dim / 8);
    const int64_t max_tokens = kMaxBlocks * kThreads / (4 * per_token) * 4;
    for (int64_t t0 = 0; t0 < n_tokens; t0 += max_tokens) {
        const int64_t nt = n_tokens - t0 < max_tokens ? n_tokens - t0 : max_tokens;
        AppendArgs c = a;
        c.k = k + t0 * per_token * 8;
        c.v = v + t0 * per_token * 8;
        c.slots = slots + t0;
        c.n_tokens = nt;
        const int64_t threads = (nt + 3) / 4 * 4 * per_token;
        dim3 grid((unsigned)((threads + kThreads - 1) / kThreads));
        const bool rows128 = p.desc.head_dim == 128;     // the whole-line form above
        switch (p.desc.dtype) {
        case AIR_KV_F32:
            if (rows128) hipLaunchKernelGGL(kv_append_rows_kernel<AIR_KV_F32>, grid, dim3(kThreads), 0, s, c);
            else hipLaunchKernelGGL((kv_append_kernel<AIR_KV_F32, false>), grid, dim3(kThreads), 0, s, c);
            break;
        case AIR_KV_BF16:
            if (rows128) hipLaunchKernelGGL(kv_append_rows_kernel<AIR_KV_BF16>, grid, dim3(kThreads), 0, s, c);
            else hipLaunchKernelGGL((kv_append_kernel<AIR_KV_BF16, false>), grid, dim3(kThreads), 0, s, c);
            break;
        case AIR_KV_INT8:
            if (rows128) hipLaunchKernelGGL((kv_append_kernel<AIR_KV_INT8, true>), grid, dim3(kThreads), 0, s, c);
            else hipLaunchKernelGGL((kv_append_kernel<AIR_KV_INT8, false>), grid, dim3(kThreads), 0, s, c);
            break;
        default:
            if (rows128) hipLaunchKernelGGL((kv_append_kernel<AIR_KV_FP8, true>), grid, dim3(kThreads), 0, s, c);
            else hipLaunchKernelGGL((kv_append_kernel<AIR_KV_FP8, false>), grid, dim3(kThreads), 0, s, c);
            break;
        }
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipGetLastError();
}

}  // namespace airkv
