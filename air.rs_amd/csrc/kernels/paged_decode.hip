// Split-K paged decode attention (one query token per sequence).
//
// The reference's flash_decode (src/flash_decode.rs:153-173) splits one
// head's contiguous KV into chunks, computes a normalised partial per chunk
// (:70-109) and merges the partials by log-sum-exp (:114-142).  Here the KV
// lives in pages: a workgroup owns one (partition, kv head, sequence) and the
// query heads that share the kv head (GQA, src/chunked_attn.rs:240-243), GC
// of them at a time: groups of up to 8 heads take one workgroup per kv head
// (GC the next power of two, heads past the group masked), so every K/V byte
// is read once for the whole group; larger groups (multi-query attention)
// take ceil(group / 8) workgroups of 8 heads each.  Within a partition the
// workgroup runs an online softmax over 64-token tiles; the partial output is
// left unnormalised together with its running max and sum (log2 domain), and
// a second kernel merges the partitions of each (sequence, query head).
//
// Thread mapping: head_dim/8 lanes cover one token row, 8 elements per lane,
// loaded with one 16-byte (bf16) or 8-byte (int8/fp8) access; a 64-lane wave
// covers 512/head_dim rows per pass.  Dot products reduce across the row's
// lanes with butterfly shuffles.  Quantized pages are dequantized in
// registers (code * group scale, as the oracle's dequantized cache).
#include <hip/hip_runtime.h>

#include <cmath>

#include "../host/status.hpp"
#include "../pool.hpp"
#include "codecs.hpp"
#include "decode_common.hpp"

namespace airkv {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kTile = 64;          // tokens per online-softmax step
#ifndef AIRKV_DECODE_PART
#define AIRKV_DECODE_PART 256      // build-time tuning knob: preferred tokens per partition
#endif
constexpr int kTargetPart = AIRKV_DECODE_PART;
constexpr int kCountNone = 0, kCountRows = 1, kCountBlocks = 2;   // out-of-pool entry counting

// Raw storage of 8 cache elements in registers.
template <int DT> struct Raw8;
template <> struct Raw8<AIR_KV_F32> { float4 a, b; };
template <> struct Raw8<AIR_KV_BF16> { uint4 w; };
template <> struct Raw8<AIR_KV_INT8> { uint2 w; float s; };
template <> struct Raw8<AIR_KV_FP8> { uint2 w; float s; };

template <int DT>
__device__ __forceinline__ void load_raw(const void *pages, const float *scales, int64_t elem,
                                         int64_t sidx, Raw8<DT> &r) {
    if constexpr (DT == AIR_KV_F32) {
        const float4 *p = reinterpret_cast<const float4 *>((const float *)pages + elem);
        r.a = p[0];
        r.b = p[1];
    } else if constexpr (DT == AIR_KV_BF16) {
        r.w = *reinterpret_cast<const uint4 *>((const uint16_t *)pages + elem);
    } else {
        r.w = *reinterpret_cast<const uint2 *>((const uint8_t *)pages + elem);
        r.s = scales[sidx];
    }
}

template <int DT>
__device__ __forceinline__ void zero_raw(Raw8<DT> &r) {
    if constexpr (DT == AIR_KV_F32) { r.a = make_float4(0, 0, 0, 0); r.b = r.a; }
    else if constexpr (DT == AIR_KV_BF16) { r.w = make_uint4(0, 0, 0, 0); }
    else { r.w = make_uint2(0, 0); r.s = 0.0f; }
}

template <int DT>
__device__ __forceinline__ void unpack(const Raw8<DT> &r, float (&x)[8]) {
    if constexpr (DT == AIR_KV_F32) {
        x[0] = r.a.x; x[1] = r.a.y; x[2] = r.a.z; x[3] = r.a.w;
        x[4] = r.b.x; x[5] = r.b.y; x[6] = r.b.z; x[7] = r.b.w;
    } else if constexpr (DT == AIR_KV_BF16) {
        const uint32_t u[4] = {r.w.x, r.w.y, r.w.z, r.w.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            x[2 * j] = __uint_as_float(u[j] << 16);
            x[2 * j + 1] = __uint_as_float(u[j] & 0xFFFF0000u);
        }
    } else {
        const uint32_t u[2] = {r.w.x, r.w.y};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t byte = (u[j >> 2] >> (8 * (j & 3))) & 0xFFu;
            float val;
            if constexpr (DT == AIR_KV_INT8) val = (float)(int32_t)(int8_t)byte;
            else val = fp8_decode(byte);
            x[j] = val * r.s;
        }
    }
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m));
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
    return v;
}

template <int DT, int G, int DP>
__global__ __launch_bounds__(kThreads) void decode_split_kernel(DecodeArgs a) {
    // DP: head_dim rounded up to 64, 128 or 256 (lanes past head_dim idle).
    // G: query heads per workgroup, the group's heads g0 .. g0 + gn - 1.
    constexpr int LPR = DP / 8;                 // lanes per token row
    constexpr int RPW = 64 / LPR;               // rows per wave per pass
    constexpr int RPP = RPW * kWaves;           // rows per workgroup pass
    constexpr int PASSES = kTile / RPP;
    constexpr bool QUANT = DT == AIR_KV_INT8 || DT == AIR_KV_FP8;
    static_assert(PASSES >= 1 && kTile % RPP == 0, "tile must cover whole passes");

    __shared__ float s_p[G * kTile];
    __shared__ float s_m[G], s_l[G], s_alpha[G];
    __shared__ float s_red[(kWaves - 1) * G * DP];

    const int d = a.head_dim;
    const int chunks = (a.group + G - 1) / G;
    const int kh = blockIdx.y / chunks, g0 = (blockIdx.y % chunks) * G;
    const int gn = a.group - g0 < G ? a.group - g0 : G;   // heads of the group in this workgroup
    const int64_t head0 = (int64_t)kh * a.group + g0;       // its first query head
    const int b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t max_len = (int64_t)a.max_blocks * a.block_size;
    const int chunk = lane % LPR;
    const bool cv = chunk * 8 < d;              // the lane's 8 elements lie inside head_dim
    const int row_in_pass = wave * RPW + lane / LPR;
    const int ng = QUANT ? d / a.scale_group : 1;
    // block sizes (16, 32) and scale groups are powers of two: the per-row
    // index arithmetic below shifts and masks instead of dividing
    const int bs_log2 = __builtin_ctz((unsigned)a.block_size);
    const int64_t bs_mask = a.block_size - 1;
    const int sg_log2 = QUANT ? __builtin_ctz((unsigned)a.scale_group) : 0;
    const int32_t *table = a.tables + (int64_t)b * a.max_blocks;

    float qr[G][8];                             // this lane's 8 elements of each query row, f32
    float acc[G][8];

    // q row `qrow` (zeros for heads past the group and lanes past head_dim)
    auto load_q = [&](int64_t qrow) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int64_t qoff = (qrow * a.n_q_heads + head0 + g) * d + chunk * 8;
            if (g >= gn || !cv) {
#pragma unroll
                for (int j = 0; j < 8; ++j) qr[g][j] = 0.0f;
            } else if (a.q_dtype == AIR_KV_F32) {
                const float4 *qp = reinterpret_cast<const float4 *>((const float *)a.q + qoff);
                float4 x0 = qp[0], x1 = qp[1];
                qr[g][0] = x0.x; qr[g][1] = x0.y; qr[g][2] = x0.z; qr[g][3] = x0.w;
                qr[g][4] = x1.x; qr[g][5] = x1.y; qr[g][6] = x1.z; qr[g][7] = x1.w;
            } else {
                uint4 w = *reinterpret_cast<const uint4 *>((const uint16_t *)a.q + qoff);
                const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    qr[g][2 * j] = __uint_as_float(u[j] << 16);
                    qr[g][2 * j + 1] = __uint_as_float(u[j] & 0xFFFF0000u);
                }
            }
        }
    };

    // Keys [start, end) of this workgroup's sequence: online softmax into
    // acc (unnormalised) and s_m / s_l, then acc summed over the rows of the
    // wave and over the waves, the total in wave 0's lanes < LPR.  An
    // out-of-pool table entry is counted (count) by every row that meets it
    // (kCountRows) or once, at its block's first token (kCountBlocks), or not
    // at all (kCountNone); its tokens are skipped (decode) or read as zero
    // keys and values (oob_zero: prefill, as the matrix-core prefill reads
    // them).
    auto attend = [&](int64_t start, int64_t end, int count, bool oob_zero) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[g][j] = 0.0f;
        __syncthreads();                        // the previous pass's readers of s_m / s_l / s_red
        if (tid < G) { s_m[tid] = -INFINITY; s_l[tid] = 0.0f; }
        __syncthreads();
        for (int64_t t0 = start; t0 < end; t0 += kTile) {
            Raw8<DT> vraw[PASSES];
            // ---- scores s = q . k (log2 units) for the tile's rows
#pragma unroll
            for (int ps = 0; ps < PASSES; ++ps) {
                const int r = ps * RPP + row_in_pass;
                const int64_t t = t0 + r;
                bool ok = t < end;
                int32_t blk = ok ? table[t >> bs_log2] : 0;
                bool in_pool = true;
                if (ok && (blk < 0 || blk >= a.num_blocks)) {
                    in_pool = false;
                    ok = oob_zero;
                    if (chunk == 0 && (count == kCountRows ||
                                       (count == kCountBlocks && ((t & bs_mask) == 0 || t == start))))
                        atomicAdd(a.errors, 1ull);
                }
                Raw8<DT> kraw;
                if (ok && cv && in_pool) {
                    const int64_t row = ((int64_t)blk * a.n_kv_heads + kh) * a.block_size + (t & bs_mask);
                    const int64_t sidx = row * ng + ((chunk * 8) >> sg_log2);
                    load_raw<DT>(a.k_pages, a.k_scales, row * d + chunk * 8, sidx, kraw);
                    load_raw<DT>(a.v_pages, a.v_scales, row * d + chunk * 8, sidx, vraw[ps]);
                } else {
                    zero_raw<DT>(kraw);
                    zero_raw<DT>(vraw[ps]);
                }
                float kx[8];
                unpack<DT>(kraw, kx);
                float sc[G];
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    float s = 0.0f;
#pragma unroll
                    for (int j = 0; j < 8; ++j) s += qr[g][j] * kx[j];
                    sc[g] = s;
                }
#pragma unroll
                for (int m = LPR / 2; m >= 1; m >>= 1)
#pragma unroll
                    for (int g = 0; g < G; ++g) sc[g] += __shfl_xor(sc[g], m);
                if (chunk == 0) {
#pragma unroll
                    for (int g = 0; g < G; ++g) s_p[g * kTile + r] = ok ? sc[g] * a.scale_log2 : -INFINITY;
                }
            }
            __syncthreads();
            // ---- online softmax update, one head per wave at a time
            for (int g = wave; g < G; g += kWaves) {
                const float s = s_p[g * kTile + lane];
                const float m_old = s_m[g];
                const float m_new = fmaxf(m_old, wave_max(s));
                const float p = (s == -INFINITY) ? 0.0f : exp2f(s - m_new);
                const float psum = wave_sum(p);
                s_p[g * kTile + lane] = p;
                if (lane == 0) {
                    const float alpha = (m_old == -INFINITY) ? 0.0f : exp2f(m_old - m_new);
                    s_alpha[g] = alpha;
                    s_l[g] = s_l[g] * alpha + psum;
                    s_m[g] = m_new;
                }
            }
            __syncthreads();
            // ---- acc = acc * alpha + p . V
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float al = s_alpha[g];
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[g][j] *= al;
            }
#pragma unroll
            for (int ps = 0; ps < PASSES; ++ps) {
                const int r = ps * RPP + row_in_pass;
                float vx[8];
                unpack<DT>(vraw[ps], vx);
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const float p = s_p[g * kTile + r];
#pragma unroll
                    for (int j = 0; j < 8; ++j) acc[g][j] += p * vx[j];
                }
            }
            __syncthreads();
        }
        // ---- reduce acc over the rows of the wave, then over the waves
#pragma unroll
        for (int m = LPR; m < 64; m <<= 1)
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[g][j] += __shfl_xor(acc[g][j], m);
        if (wave > 0 && lane < LPR) {
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
                for (int j = 0; j < 8; ++j) s_red[((wave - 1) * G + g) * DP + chunk * 8 + j] = acc[g][j];
        }
        __syncthreads();
        if (wave == 0 && lane < LPR) {
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    float v = acc[g][j];
#pragma unroll
                    for (int w = 0; w < kWaves - 1; ++w) v += s_red[(w * G + g) * DP + chunk * 8 + j];
                    acc[g][j] = v;
                }
        }
    };

    if (a.cu_q) {
        // Prefill rows: sequence b's query rows q0 .. q1 - 1, row r at
        // position len - q_len + r seeing keys 0 ..= that position, each a
        // single partition normalised here.  The consistency test and its
        // handling are the matrix-core prefill's: counted once, rows inside
        // [0, total_q] zero-filled.
        const int32_t q0 = a.cu_q[b], q1 = a.cu_q[b + 1];
        const int64_t len = a.lens[b];
        const bool rows_ok = q0 >= 0 && q1 >= q0 && q1 <= a.total_q;
        const int qlen = q1 - q0;
        if (!(rows_ok && len >= 0 && len <= max_len && (int64_t)qlen <= len)) {
            if (blockIdx.x == 0 && blockIdx.y == 0 && tid == 0) atomicAdd(a.errors, 1ull);
            if (!rows_ok) return;
            for (int r = blockIdx.x; r < qlen; r += gridDim.x)
                for (int i = tid; i < gn * d; i += kThreads) {
                    const int64_t oi = (((int64_t)q0 + r) * a.n_q_heads + head0 + i / d) * d + i % d;
                    if (a.out_dtype == AIR_KV_F32) ((float *)a.out)[oi] = 0.0f;
                    else ((uint16_t *)a.out)[oi] = 0;
                }
            return;
        }
        for (int r = blockIdx.x; r < qlen; r += gridDim.x) {
            const int64_t qrow = (int64_t)q0 + r;
            load_q(qrow);
            // the last row reads every key: its first head chunk counts each
            // out-of-pool entry once
            attend(0, len - qlen + r + 1, r == qlen - 1 && blockIdx.y == 0 ? kCountBlocks : kCountNone, true);
            if (wave == 0 && lane < LPR && cv) {
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    if (g >= gn) break;
                    const float inv = 1.0f / s_l[g];
                    const int64_t oi = (qrow * a.n_q_heads + head0 + g) * d + chunk * 8;
                    if (a.out_dtype == AIR_KV_F32) {
                        float4 *dst = reinterpret_cast<float4 *>((float *)a.out + oi);
                        dst[0] = make_float4(acc[g][0] * inv, acc[g][1] * inv, acc[g][2] * inv, acc[g][3] * inv);
                        dst[1] = make_float4(acc[g][4] * inv, acc[g][5] * inv, acc[g][6] * inv, acc[g][7] * inv);
                    } else {
                        uint32_t w[4];
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            w[j] = (uint32_t)bf16_rne(acc[g][2 * j] * inv) |
                                   ((uint32_t)bf16_rne(acc[g][2 * j + 1] * inv) << 16);
                        *reinterpret_cast<uint4 *>((uint16_t *)a.out + oi) = make_uint4(w[0], w[1], w[2], w[3]);
                    }
                }
            }
        }
        return;
    }

    // Decode: partition blockIdx.x of sequence b's keys
    const int part = blockIdx.x;
    int64_t len = a.lens[b];
    len = len < 0 ? 0 : (len > max_len ? max_len : len);
    const int64_t start = (int64_t)part * a.part_tokens;
    if (start >= len) return;
    const int64_t end = start + a.part_tokens < len ? start + a.part_tokens : len;
    load_q(b);
    attend(start, end, kCountRows, false);
    if (wave == 0 && lane < LPR && cv) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            if (g >= gn) break;
            const int64_t slot = ((int64_t)b * a.n_q_heads + head0 + g) * a.num_parts + part;
            float4 *dst = reinterpret_cast<float4 *>(a.part_o + slot * d + chunk * 8);
            dst[0] = make_float4(acc[g][0], acc[g][1], acc[g][2], acc[g][3]);
            dst[1] = make_float4(acc[g][4], acc[g][5], acc[g][6], acc[g][7]);
            if (chunk == 0) {
                a.part_ml[slot * 2] = s_m[g];
                a.part_ml[slot * 2 + 1] = s_l[g];
            }
        }
    }
}

// Log-sum-exp merge of the partitions (src/flash_decode.rs:114-142, with the
// partial outputs kept unnormalised): one workgroup per (query head, seq),
// one thread per head_dim element.
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeArgs a) {
    const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, d = a.head_dim;
    const int64_t max_len = (int64_t)a.max_blocks * a.block_size;
    int64_t len = a.lens[b];
    if (tid == 0 && (len < 0 || len > max_len) && h == 0) atomicAdd(a.errors, 1ull);
    len = len < 0 ? 0 : (len > max_len ? max_len : len);
    const int nparts = (int)((len + a.part_tokens - 1) / a.part_tokens);
    const int64_t base = ((int64_t)b * a.n_q_heads + h) * a.num_parts;
    float o = 0.0f;
    if (nparts > 0) {
        float m = -INFINITY;
        for (int p = 0; p < nparts; ++p) m = fmaxf(m, a.part_ml[(base + p) * 2]);
        float l = 0.0f, acc = 0.0f;
        for (int p = 0; p < nparts; ++p) {
            const float mp = a.part_ml[(base + p) * 2];
            const float w = (mp == -INFINITY) ? 0.0f : exp2f(mp - m);
            l += w * a.part_ml[(base + p) * 2 + 1];
            acc += w * a.part_o[(base + p) * d + tid];
        }
        o = l > 0.0f ? acc / l : 0.0f;
    }
    const int64_t oi = ((int64_t)b * a.n_q_heads + h) * d + tid;
    if (a.out_dtype == AIR_KV_F32) ((float *)a.out)[oi] = o;
    else ((uint16_t *)a.out)[oi] = bf16_rne(o);
}

template <int DT, int G, int DP>
hipError_t launch_typed(const DecodeArgs &a, hipStream_t s, int n_kv_heads) {
    // (partition or prefill row slot, head chunk, sequence)
    const int chunks = (a.group + G - 1) / G;
    dim3 grid((unsigned)a.num_parts, (unsigned)(n_kv_heads * chunks), (unsigned)a.batch);
    hipLaunchKernelGGL((decode_split_kernel<DT, G, DP>), grid, dim3(kThreads), 0, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.cu_q) return e;     // prefill rows are normalised in place
    hipLaunchKernelGGL(decode_merge_kernel, dim3((unsigned)a.n_q_heads, (unsigned)a.batch),
                       dim3((unsigned)a.head_dim), 0, s, a);
    return hipGetLastError();
}

// head_dim rounded up to 64, 128 or 256 lanes' worth of 8-element chunks
template <int DT, int G>
hipError_t launch_d(const DecodeArgs &a, hipStream_t s, int n_kv_heads, int d) {
    if (d <= 64) return launch_typed<DT, G, 64>(a, s, n_kv_heads);
    if (d <= 128) return launch_typed<DT, G, 128>(a, s, n_kv_heads);
    return launch_typed<DT, G, 256>(a, s, n_kv_heads);
}

// The decode step's append slot of each sequence on the vector path: token
// seq_lens[b] - 1 through its block table, or -1 (nothing appended) for an
// empty sequence, one longer than its table or a last block outside the
// pool -- the cases the decode itself counts.
__global__ __launch_bounds__(256) void step_slots_kernel(DecodeArgs a, int64_t *slots) {
    const int b = blockIdx.x * 256 + threadIdx.x;
    if (b >= a.batch) return;
    const int64_t len = a.lens[b], max_len = (int64_t)a.max_blocks * a.block_size;
    int64_t slot = -1;
    if (len > 0 && len <= max_len) {
        const int32_t blk = a.tables[(int64_t)b * a.max_blocks + (len - 1) / a.block_size];
        if (blk >= 0 && blk < a.num_blocks) slot = (int64_t)blk * a.block_size + (len - 1) % a.block_size;
    }
    slots[b] = slot;
}

// Heads per workgroup: the group rounded up to a power of two, at most 8.
template <int DT>
hipError_t launch_g(const DecodeArgs &a, hipStream_t s, int n_kv_heads, int d, int g) {
    if (g == 1) return launch_d<DT, 1>(a, s, n_kv_heads, d);
    if (g == 2) return launch_d<DT, 2>(a, s, n_kv_heads, d);
    if (g <= 4) return launch_d<DT, 4>(a, s, n_kv_heads, d);
    return launch_d<DT, 8>(a, s, n_kv_heads, d);
}

}  // namespace

// Byte offset of the vector path's append slots in its workspace.
static size_t step_slots_offset(int64_t batch, int64_t n_q_heads, int64_t parts, int64_t d) {
    return ((size_t)(batch * n_q_heads * parts * (d + 2)) * sizeof(float) + 255) & ~(size_t)255;
}

int plan_decode(const air_kv_pool &p, int32_t n_q_heads, int32_t batch, int32_t max_blocks,
                int32_t max_splits, DecodePlan *plan) {
    const int nkv = p.desc.n_kv_heads, d = p.desc.head_dim, bs = p.desc.block_size;
    if (n_q_heads <= 0 || n_q_heads % nkv)
        return fail(AIR_KV_E_INVALID_ARG, "n_q_heads %d is not a multiple of n_kv_heads %d", n_q_heads, nkv);
    const int g = n_q_heads / nkv;
    if (!decode_mfma_supported(p.desc.dtype, d, bs, g, p.desc.scale_group)) {
        if (d <= 0 || d % 8 || d > 256)
            return fail(AIR_KV_E_INVALID_ARG, "decode supports head_dim a multiple of 8 up to 256 (pool has %d)", d);
    }
    if (batch < 0 || batch > 65535) return fail(AIR_KV_E_INVALID_ARG, "batch %d out of range", batch);
    if (max_blocks <= 0) return fail(AIR_KV_E_INVALID_ARG, "max_blocks must be positive");
    if (max_splits < 1 || max_splits > 256)
        return fail(AIR_KV_E_INVALID_ARG, "max_splits %d outside 1..256", max_splits);
    plan->group = g;
    plan->max_splits = max_splits;
    if (decode_mfma_supported(p.desc.dtype, d, bs, g, p.desc.scale_group))
        return plan_decode_mfma(p, n_q_heads, batch, max_blocks, max_splits, plan);
    plan->mfma = false;
    plan->dtype = p.desc.dtype;
    plan->slices = plan->slices_qf32 = plan->batch_per_launch = plan->slots = 0;
    const int64_t max_ctx = (int64_t)max_blocks * bs;
    int64_t parts = (max_ctx + kTargetPart - 1) / kTargetPart;
    parts = parts < 1 ? 1 : (parts > max_splits ? max_splits : parts);
    int64_t part_tokens = (max_ctx + parts - 1) / parts;
    part_tokens = (part_tokens + bs - 1) / bs * bs;
    if (part_tokens > INT32_MAX) return fail(AIR_KV_E_INVALID_ARG, "max_blocks too large");
    parts = (max_ctx + part_tokens - 1) / part_tokens;
    plan->part_tokens = (int32_t)part_tokens;
    plan->num_parts = (int32_t)parts;
    // partial outputs and (max, sum), then the decode step's append slots
    plan->ws_bytes = step_slots_offset(batch, n_q_heads, parts, d) + (size_t)batch * sizeof(int64_t);
    return AIR_KV_OK;
}

hipError_t launch_decode(const air_kv_pool &p, hipStream_t s, const DecodePlan &plan, const void *q,
                         int32_t q_dtype, int32_t n_q_heads, const int32_t *tables,
                         const int32_t *lens, int32_t batch, int32_t max_blocks, float scale,
                         void *workspace, void *out, int32_t out_dtype, const float *k_new,
                         const float *v_new) {
    DecodeArgs a;
    a.k_new = plan.mfma ? k_new : nullptr;   // the vector path appends them before its kernels
    a.v_new = plan.mfma ? v_new : nullptr;
    a.q = q; a.q_dtype = q_dtype; a.n_q_heads = n_q_heads;
    a.tables = tables; a.lens = lens;
    a.batch = batch; a.max_blocks = max_blocks;
    a.part_tokens = plan.part_tokens; a.num_parts = plan.num_parts;
    a.slices = plan.slices; a.slots = plan.slots; a.max_splits = plan.max_splits;
    a.scale_log2 = scale * 1.4426950408889634f;
    a.n_kv_heads = p.desc.n_kv_heads; a.block_size = p.desc.block_size;
    a.scale_group = p.desc.scale_group; a.group = plan.group; a.num_blocks = p.desc.num_blocks;
    a.k_pages = p.k_pages; a.v_pages = p.v_pages;
    a.k_scales = p.k_scales; a.v_scales = p.v_scales;
    a.out = out; a.out_dtype = out_dtype;
    a.errors = p.errors;
    a.prefix = nullptr;
    a.head_dim = p.desc.head_dim;
    a.cu_q = nullptr;
    a.total_q = 0;
    if (plan.mfma) return launch_decode_mfma(a, plan, workspace, s);
    const size_t n_slots = (size_t)batch * n_q_heads * plan.num_parts;
    a.part_o = (float *)workspace;
    a.part_ml = a.part_o + n_slots * p.desc.head_dim;
    if (k_new && batch > 0) {
        // the decode step on the vector path: each sequence's new row
        // appended by air_kv_append's kernel at the slot its table gives
        // token seq_lens[b] - 1, then the decode
        int64_t *slots = (int64_t *)((char *)workspace +
                                     step_slots_offset(batch, n_q_heads, plan.num_parts, p.desc.head_dim));
        hipLaunchKernelGGL(step_slots_kernel, dim3((unsigned)((batch + 255) / 256)), dim3(256), 0, s, a, slots);
        hipError_t e = hipGetLastError();
        if (e == hipSuccess) e = launch_append(p, s, k_new, v_new, slots, batch);
        if (e != hipSuccess) return e;
    }
    const int d = p.desc.head_dim, g = plan.group, nkv = p.desc.n_kv_heads;
    switch (p.desc.dtype) {
    case AIR_KV_F32: return launch_g<AIR_KV_F32>(a, s, nkv, d, g);
    case AIR_KV_BF16: return launch_g<AIR_KV_BF16>(a, s, nkv, d, g);
    case AIR_KV_INT8: return launch_g<AIR_KV_INT8>(a, s, nkv, d, g);
    default: return launch_g<AIR_KV_FP8>(a, s, nkv, d, g);
    }
}

hipError_t launch_prefill_rows(const air_kv_pool &p, hipStream_t s, const void *q, int32_t q_dtype,
                               int32_t n_q_heads, const int32_t *cu_q, int32_t total_q, int32_t max_q_len,
                               const int32_t *tables, const int32_t *lens, int32_t batch, int32_t max_blocks,
                               float scale, void *out, int32_t out_dtype) {
    DecodeArgs a{};
    a.q = q; a.q_dtype = q_dtype; a.n_q_heads = n_q_heads;
    a.tables = tables; a.lens = lens;
    a.batch = batch; a.max_blocks = max_blocks;
    // row slots per sequence: one per query row up to max_q_len (longer
    // chunks stride over them)
    a.num_parts = max_q_len < 1 ? 1 : (max_q_len > 65535 ? 65535 : max_q_len);
    a.part_tokens = 0;
    a.scale_log2 = scale * 1.4426950408889634f;
    a.n_kv_heads = p.desc.n_kv_heads; a.block_size = p.desc.block_size;
    a.scale_group = p.desc.scale_group; a.group = n_q_heads / p.desc.n_kv_heads;
    a.head_dim = p.desc.head_dim; a.num_blocks = p.desc.num_blocks;
    a.k_pages = p.k_pages; a.v_pages = p.v_pages;
    a.k_scales = p.k_scales; a.v_scales = p.v_scales;
    a.out = out; a.out_dtype = out_dtype;
    a.errors = p.errors;
    a.cu_q = cu_q;
    a.total_q = total_q;
    const int d = p.desc.head_dim, g = a.group, nkv = p.desc.n_kv_heads;
    switch (p.desc.dtype) {
    case AIR_KV_F32: return launch_g<AIR_KV_F32>(a, s, nkv, d, g);
    case AIR_KV_BF16: return launch_g<AIR_KV_BF16>(a, s, nkv, d, g);
    case AIR_KV_INT8: return launch_g<AIR_KV_INT8>(a, s, nkv, d, g);
    default: return launch_g<AIR_KV_FP8>(a, s, nkv, d, g);
    }
}

}  // namespace airkv
