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
// row and runs the folds in that order; rows reach the lanes through LDS:
// a wave stages 64 rows x 32 columns with coalesced loads (any pool dtype,
// dequantized by the shared page loader), then each lane reads its row back
// (row pitch 33 floats: conflict-free) and keeps it in registers.  Products
// and sums round separately (no contraction), as Rust's do.
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
constexpr int kWaves = kThreads / 64;
constexpr int kPitch = 33;          // floats per staged row (32 columns + 1: bank spread)
constexpr int kProjRows = 32;       // projection rows staged in LDS at a time

__device__ __forceinline__ float rust_min(float a, float b) {
    if (a != a) return b;
    if (b != b) return a;
    return a < b ? a : b;
}

__device__ __forceinline__ float rust_max(float a, float b) {
    if (a != a) return b;
    if (b != b) return a;
    return a > b ? a : b;
}

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

// The wave's 64 rows row0 .. row0 + 63 into registers: lane l gets row row0 + l
// in x.  Rows past n_rows and rows of out-of-pool blocks read as zeros; `live`
// tells the lane whether its row is real.  Every thread of the workgroup calls
// this the same number of times (it contains barriers).
template <int DT, int D>
__device__ void stage_rows(const RowSource &s, int64_t row0, int64_t n_rows, float *lds,
                           float (&x)[D], bool &live) {
    const int lane = threadIdx.x & 63;
    float *w_lds = lds + (threadIdx.x >> 6) * 64 * kPitch;
    {
        int64_t e;
        live = row0 + lane < n_rows && row_elem(s, row0 + lane, D, e);
    }
#pragma unroll
    for (int c = 0; c < D / 32; ++c) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int g = lane + 64 * i;          // 8-column group g % 4 of row g / 4
            const int rr = g >> 2, c8 = g & 3;
            float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            const int64_t r = row0 + rr;
            if (r < n_rows) {
                int64_t e;
                if (row_elem(s, r, D, e)) {
                    const int64_t el = e + 32 * c + 8 * c8;
                    pio_u32x4 raw;
                    load8<DT>(s.base, s.scales, el, s.scale_group ? el / s.scale_group : 0, v, &raw);
                }
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) w_lds[rr * kPitch + 8 * c8 + j] = v[j];
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < 32; ++j) x[32 * c + j] = w_lds[lane * kPitch + j];
        __syncthreads();
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
    __shared__ float lds[kWaves * 64 * kPitch];
    constexpr int W = (D + 63) / 64;
    const int lane = threadIdx.x & 63;
    for (int64_t base = (int64_t)blockIdx.x * kThreads; base < a.n_rows; base += (int64_t)gridDim.x * kThreads) {
        const int64_t row0 = base + (threadIdx.x & ~63);
        float x[D];
        bool live;
        stage_rows<DT, D>(a.src, row0, a.n_rows, lds, x, live);
        const int64_t r = row0 + lane;
        if (r >= a.n_rows) continue;
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

template <int DT, int D>
__global__ __launch_bounds__(kThreads) void value_compress_kernel(CompressArgs a) {
    __shared__ float lds[kWaves * 64 * kPitch];
    const int lane = threadIdx.x & 63;
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    for (int64_t base = (int64_t)blockIdx.x * kThreads; base < a.n_rows; base += (int64_t)gridDim.x * kThreads) {
        const int64_t row0 = base + (threadIdx.x & ~63);
        float x[D];
        bool live;
        stage_rows<DT, D>(a.src, row0, a.n_rows, lds, x, live);
        const int64_t r = row0 + lane;
        if (r >= a.n_rows) continue;
        if (!live && a.errors && (r % a.src.rows_per_block) == 0) atomicAdd(a.errors, 1ull);
        float lo = INFINITY, hi = -INFINITY;
#pragma unroll
        for (int j = 0; j < D; ++j) {                  // (:198-199)
            lo = rust_min(lo, x[j]);
            hi = rust_max(hi, x[j]);
        }
        float scale;
        uint32_t q[D / 4];
        {
#pragma clang fp contract(off)
            const float range = hi - lo;
            scale = range > 0.0f ? range / 255.0f : 1.0f;   // (:201-202)
#pragma unroll
            for (int j4 = 0; j4 < D / 4; ++j4) {
                uint32_t w = 0;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    float t = roundf((x[4 * j4 + k] - lo) / scale);   // (:204-209)
                    t = t < 0.0f ? 0.0f : t;
                    t = t > 255.0f ? 255.0f : t;
                    const uint32_t c = (t != t) ? 0u : (uint32_t)t;   // `as u8`: NaN -> 0
                    w |= c << (8 * k);
                }
                q[j4] = w;
            }
        }
        if (!live) { scale = 0.0f; lo = 0.0f; for (int j = 0; j < D / 4; ++j) q[j] = 0; }
        u32x4 *dst = reinterpret_cast<u32x4 *>(a.codes + r * D);
#pragma unroll
        for (int j = 0; j < D / 16; ++j) dst[j] = u32x4{q[4 * j], q[4 * j + 1], q[4 * j + 2], q[4 * j + 3]};
        a.f0[r] = scale;
        a.f1[r] = lo;
    }
}

template <int DT, int D>
__global__ __launch_bounds__(kThreads) void qjl_compress_kernel(CompressArgs a) {
    __shared__ float lds[kWaves * 64 * kPitch];
    __shared__ __align__(16) float proj[kProjRows * D];
    const int lane = threadIdx.x & 63;
    const int m = a.proj_dim, W = (m + 63) / 64;
    for (int64_t base = (int64_t)blockIdx.x * kThreads; base < a.n_rows; base += (int64_t)gridDim.x * kThreads) {
        const int64_t row0 = base + (threadIdx.x & ~63);
        float x[D];
        bool live;
        stage_rows<DT, D>(a.src, row0, a.n_rows, lds, x, live);
        const int64_t r = row0 + lane;
        const bool own = r < a.n_rows;
        if (own && !live && a.errors && (r % a.src.rows_per_block) == 0) atomicAdd(a.errors, 1ull);
        uint64_t word = 0;
        for (int i0 = 0; i0 < m; i0 += kProjRows) {
            // rows i0 .. i0 + 31 of R (zeros past m)
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
            __syncthreads();
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
    switch (kind) {
    case CompressKind::Key: AIRKV_LAUNCH_D(key_compress_kernel, a, s, grid) break;
    case CompressKind::Value: AIRKV_LAUNCH_D(value_compress_kernel, a, s, grid) break;
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
