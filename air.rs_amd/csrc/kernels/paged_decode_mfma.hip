// Paged decode attention on the matrix cores (bf16 pages, head_dim 128).
//
// One workgroup owns one (split-K partition, kv head, sequence) and all G <= 16
// query heads of that kv head (GQA group), so each K/V byte is read from HBM
// once.  Its four waves take 16-token tiles of the partition round robin:
//
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
// Each wave reads the block ids of all its tiles with one vector load (lane k
// holds the id of the wave's k-th tile) and takes them with readlane, so tile
// addresses come from scalar registers and no load ever waits on another.  K
// and V of the next tile are in flight while the current tile is computed
// (two register sets, used alternately).  The four waves merge their
// (max, sum, O) through LDS; a sequence with a single partition writes its
// output directly, otherwise the partition stores an unnormalised partial that
// decode_merge_kernel combines by log-sum-exp (src/flash_decode.rs:114-142).
#include <hip/hip_runtime.h>

#include <cmath>

#include "../pool.hpp"
#include "codecs.hpp"
#include "decode_common.hpp"

namespace airkv {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxParts = 256;             // bound of max_splits

// Build-time tuning knobs (defaults are the shipped configuration).
#ifndef AIRKV_DECODE_WAVES_PER_EU
#define AIRKV_DECODE_WAVES_PER_EU 2        // register budget: waves per SIMD
#endif
#ifndef AIRKV_DECODE_NT_LOADS
#define AIRKV_DECODE_NT_LOADS 0            // non-temporal K/V loads
#endif

// Buffer descriptor word 3 for raw (untyped) buffer access on gfx9-class
// GPUs, and the cache-policy bits of the K/V loads (1 = glc... 2 = slc, i.e.
// streaming / non-temporal).
constexpr int kBufferWord3 = 0x00020000;
constexpr int kLoadAux = AIRKV_DECODE_NT_LOADS ? 2 : 0;

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

__device__ __forceinline__ void store_out(const DecodeArgs &a, int64_t idx, float v) {
    if (a.out_dtype == AIR_KV_F32) ((float *)a.out)[idx] = v;
    else ((uint16_t *)a.out)[idx] = bf16_rne(v);
}

template <int D, int BS, int GMAX, bool QF32>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(AIRKV_DECODE_WAVES_PER_EU)))
void decode_mfma_kernel(DecodeArgs a) {
    constexpr int KSTEPS = D / 32;            // QK k-steps
    constexpr int DTILES = D / 16;            // PV output tiles along head_dim
    constexpr int VCH = D / 8;                // 16-byte chunks per V row
    constexpr int VRPL = 64 / VCH;            // V rows per wave load
    constexpr int VLOADS = 16 / VRPL;         // V loads per 16-token tile
    constexpr int PITCH = D + 4;              // LDS row pitch in bf16 elements
    constexpr int VTILE = 16 * PITCH;         // bf16 elements per wave's V tile
    constexpr int MERGE_FLOATS = kWaves * GMAX * D;
    constexpr int SMEM = (VTILE * 2 * kWaves > MERGE_FLOATS * 4) ? VTILE * 2 * kWaves : MERGE_FLOATS * 4;
    static_assert(BS % 16 == 0, "a 16-token tile must not straddle pages");
    __shared__ __align__(16) unsigned char smem[SMEM];
    __shared__ float s_m[kWaves][16], s_l[kWaves][16];

    const int part = blockIdx.x, kh = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: scalar loop control
    const int g4 = lane >> 4, r16 = lane & 15;
    const int G = a.group;
    const int64_t max_len = (int64_t)a.max_blocks * BS;
    int64_t len = a.lens[b];
    len = len < 0 ? 0 : (len > max_len ? max_len : len);
    const int64_t start = (int64_t)part * a.part_tokens;
    if (start >= len) {
        if (len == 0 && part == 0)                      // empty sequence: zeros
            for (int idx = tid; idx < G * D; idx += kThreads)
                store_out(a, ((int64_t)b * a.n_q_heads + kh * G) * D + idx, 0.0f);
        return;
    }
    const int64_t end = start + a.part_tokens < len ? start + a.part_tokens : len;
    const int n_active = (int)((len + a.part_tokens - 1) / a.part_tokens);
    const int n_tiles = (int)((end - start + 15) / 16);
    const int my_tiles = wave < n_tiles ? (n_tiles - wave + kWaves - 1) / kWaves : 0;

    // Block ids of this wave's tiles, 64 at a time: lane k of `tbl` holds the id
    // of tile wave + 4 * (c0 + k).  The first chunk is requested before the Q
    // loads so both latencies overlap.
    const int32_t *table = a.tables + (int64_t)b * a.max_blocks;
    int32_t tbl = 0;
    int c0 = 0;
    auto load_table = [&](int first) {
        const int kk = first + lane;
        tbl = kk < my_tiles ? table[(start + 16 * (int64_t)(wave + kWaves * kk)) / BS] : 0;
    };
    load_table(0);

    // ---- Q^T in the B-operand layout: lane holds q[h = r16][8*g4 + 32*ks .. +8]
    u32x4 qhi[KSTEPS], qlo[KSTEPS];
    {
        const int64_t qrow = ((int64_t)b * a.n_q_heads + kh * G + r16) * D;
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
            const int d0 = 8 * g4 + 32 * ks;
            u32x4 hi = {0, 0, 0, 0}, lo = {0, 0, 0, 0};
            if (r16 < G) {
                if constexpr (QF32) {
                    const f32x4 *qp = reinterpret_cast<const f32x4 *>((const float *)a.q + qrow + d0);
                    const f32x4 x0 = qp[0], x1 = qp[1];
                    const float x[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
                    uint32_t h[8], l[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) split_bf16(x[j], h[j], l[j]);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        hi[j] = h[2 * j] | (h[2 * j + 1] << 16);
                        lo[j] = l[2 * j] | (l[2 * j + 1] << 16);
                    }
                } else {
                    hi = *reinterpret_cast<const u32x4 *>((const uint16_t *)a.q + qrow + d0);
                }
            }
            qhi[ks] = hi;
            qlo[ks] = lo;
        }
    }

    f32x4 acc[DTILES];
#pragma unroll
    for (int n = 0; n < DTILES; ++n) acc[n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float m_run = -INFINITY, l_run = 0.0f;

    const uint16_t *kp = (const uint16_t *)a.k_pages;
    const uint16_t *vp = (const uint16_t *)a.v_pages;
    uint16_t *sv = reinterpret_cast<uint16_t *>(smem) + wave * VTILE;
    const int vrow = lane / VCH, vch = lane % VCH;
    const int k_boff = (r16 * D + 8 * g4) * 2;          // lane's K byte offset in a tile
    const int v_boff = (vrow * D + vch * 8) * 2;        // lane's V byte offset in a tile

    // Tiles are loaded unconditionally (an id outside the pool reads block 0)
    // and skipped at compute time, so no branch ever merges freshly loaded
    // registers.
    auto load_tile = [&](int k, u32x4 (&kr)[KSTEPS], u32x4 (&vr)[VLOADS]) -> bool {
        int32_t blk = __builtin_amdgcn_readlane(tbl, k - c0);
        const bool ok = blk >= 0 && blk < a.num_blocks;
        blk = ok ? blk : 0;
        const int64_t t0 = start + 16 * (int64_t)(wave + kWaves * k);
        const int64_t base = (((int64_t)blk * a.n_kv_heads + kh) * BS + (t0 % BS)) * D;
        // Buffer loads: the tile's base lives in a scalar resource descriptor
        // and each lane's offset is a loop-invariant register, so no vector
        // address register is rewritten while earlier loads are in flight.
        // The descriptor also bounds the access to the 16-row tile.
        const __amdgpu_buffer_rsrc_t rk =
            __builtin_amdgcn_make_buffer_rsrc((void *)(kp + base), (short)0, 16 * D * 2, kBufferWord3);
        const __amdgpu_buffer_rsrc_t rv =
            __builtin_amdgcn_make_buffer_rsrc((void *)(vp + base), (short)0, 16 * D * 2, kBufferWord3);
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks)
            kr[ks] = __builtin_amdgcn_raw_buffer_load_b128(rk, k_boff + 64 * ks, 0, kLoadAux);
#pragma unroll
        for (int v = 0; v < VLOADS; ++v)
            vr[v] = __builtin_amdgcn_raw_buffer_load_b128(rv, v_boff + v * VRPL * D * 2, 0, kLoadAux);
        return ok;
    };

    auto compute_tile = [&](int k, const u32x4 (&kr)[KSTEPS], const u32x4 (&vr)[VLOADS], bool ok) {
        // A table entry outside the pool is counted and its tile masked out;
        // the tile still runs every instruction, so the loaded registers are
        // consumed on all paths and the loads in flight never need draining.
        if (!ok && lane == 0) atomicAdd(a.errors, 1ull);
        const int64_t t0 = start + 16 * (int64_t)(wave + kWaves * k);
        f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
            s = mfma_qk(kr[ks], qhi[ks], s);
            if constexpr (QF32) s = mfma_qk(kr[ks], qlo[ks], s);
        }
        // lane holds S[token 4*g4 + i][head r16]
        float sc[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) sc[i] = (ok && t0 + 4 * g4 + i < end) ? s[i] * a.scale_log2 : -INFINITY;
        float mt = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
        mt = fmaxf(mt, __shfl_xor(mt, 16));
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        // The running max is raised only when some head's tile max exceeds it
        // by more than 2^8 (and on the first tile): probabilities then stay
        // below 256, exact in the hi + lo split, and most tiles skip the
        // rescale of the accumulators.  The final normalisation uses the same
        // max, so the result is unchanged.
        if (__ballot(mt > m_run + 8.0f) != 0ull) {
            const float m_new = fmaxf(m_run, mt);
            const float alpha = (m_run == -INFINITY) ? 0.0f : exp2f(m_run - m_new);
            l_run *= alpha;
#pragma unroll
            for (int n = 0; n < DTILES; ++n) acc[n] *= alpha;
            m_run = m_new;
        }
        float p[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) p[i] = (sc[i] == -INFINITY) ? 0.0f : exp2f(sc[i] - m_run);
        l_run += (p[0] + p[1]) + (p[2] + p[3]);
        // P^T as the B operand (lane: tokens 4*g4 .. +3 of head r16), hi + lo halves
        uint32_t h[4], l[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) split_bf16(p[i], h[i], l[i]);
        const u32x2 p_hi = {h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
        const u32x2 p_lo = {l[0] | (l[1] << 16), l[2] | (l[3] << 16)};
        // V tile -> LDS (token rows beyond the sequence are zeroed: p = 0 there,
        // but stale page bytes may hold non-finite values)
#pragma unroll
        for (int v = 0; v < VLOADS; ++v) {
            const int row = v * VRPL + vrow;
            u32x4 w = vr[v];
            if (!ok || t0 + row >= end) w = u32x4{0, 0, 0, 0};
            u32x2 *dst = reinterpret_cast<u32x2 *>(sv + row * PITCH + vch * 8);
            dst[0] = u32x2{w[0], w[1]};
            dst[1] = u32x2{w[2], w[3]};
        }
        // O^T[d][h] += V^T[d][t] P^T[t][h]; A lane holds V[t = 4*g4 + jj][d = 16n + r16]
        const uint16_t *col = sv + (4 * g4) * PITCH + r16;
#pragma unroll
        for (int n = 0; n < DTILES; ++n) {
            const uint16_t *c = col + 16 * n;
            const u32x2 av = {(uint32_t)c[0] | ((uint32_t)c[PITCH] << 16),
                              (uint32_t)c[2 * PITCH] | ((uint32_t)c[3 * PITCH] << 16)};
            acc[n] = mfma_pv(av, p_hi, acc[n]);
            acc[n] = mfma_pv(av, p_lo, acc[n]);
        }
    };

    for (; c0 < my_tiles; c0 += 64) {
        const int c1 = my_tiles - c0 < 64 ? my_tiles : c0 + 64;
        if (c0 > 0) load_table(c0);
        // Three register sets used in rotation: two tiles are in flight while
        // the third is computed.  Loads are issued unconditionally (past the
        // end they re-read the last tile, an L2 hit) so no branch joins paths
        // with different loads in flight.
        auto clampk = [&](int k) { return k < c1 ? k : c1 - 1; };
        u32x4 ka[KSTEPS], va[VLOADS], kb[KSTEPS], vb[VLOADS], kc[KSTEPS], vc[VLOADS];
        bool oka = load_tile(c0, ka, va), okb = load_tile(clampk(c0 + 1), kb, vb), okc;
        for (int k = c0; k < c1; k += 3) {
            okc = load_tile(clampk(k + 2), kc, vc);
            compute_tile(k, ka, va, oka);
            if (k + 1 >= c1) break;
            oka = load_tile(clampk(k + 3), ka, va);
            compute_tile(k + 1, kb, vb, okb);
            if (k + 2 >= c1) break;
            okb = load_tile(clampk(k + 4), kb, vb);
            compute_tile(k + 2, kc, vc, okc);
        }
    }

    // ---- merge the four waves (head h = r16; lane holds O^T[d = 16n + 4*g4 + i][h])
    l_run += __shfl_xor(l_run, 16);
    l_run += __shfl_xor(l_run, 32);
    if (lane < 16) {
        s_m[wave][lane] = m_run;
        s_l[wave][lane] = l_run;
    }
    __syncthreads();                                   // V tiles are dead from here on
    float *so = reinterpret_cast<float *>(smem);       // [wave][GMAX][D]
    if (r16 < G) {
#pragma unroll
        for (int n = 0; n < DTILES; ++n)
#pragma unroll
            for (int i = 0; i < 4; ++i) so[(wave * GMAX + r16) * D + 16 * n + 4 * g4 + i] = acc[n][i];
    }
    __syncthreads();

    const int64_t slot_base = ((int64_t)b * a.n_q_heads + kh * G) * a.num_parts;
    for (int idx = tid; idx < G * D; idx += kThreads) {
        const int h = idx / D, d = idx - h * D;
        float m = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) m = fmaxf(m, s_m[w][h]);
        float wsum = 0.0f, o = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float f = exp2f(s_m[w][h] - m);       // a wave without tiles has m = -inf: f = 0
            wsum += f * s_l[w][h];
            o += f * so[(w * GMAX + h) * D + d];
        }
        if (n_active == 1) {
            store_out(a, ((int64_t)b * a.n_q_heads + kh * G + h) * D + d, o / wsum);
        } else {
            const int64_t slot = slot_base + (int64_t)h * a.num_parts + part;
            a.part_o[slot * D + d] = o;
            if (d == 0) {
                a.part_ml[slot * 2] = m;
                a.part_ml[slot * 2 + 1] = wsum;
            }
        }
    }
}

// Log-sum-exp merge of the partitions of one (sequence, kv head): the G x D
// outputs of its query heads.  Weights come from the partitions' (max, sum)
// staged in LDS; each thread then sums its output over the partitions with
// independent, unrolled loads.
template <int D, int GMAX>
__global__ __launch_bounds__(kThreads) void decode_merge_kernel(DecodeArgs a) {
    __shared__ float s_w[GMAX][kMaxParts];
    __shared__ float s_inv[GMAX];
    const int b = blockIdx.x, kh = blockIdx.y, tid = threadIdx.x;
    const int G = a.group;
    const int64_t max_len = (int64_t)a.max_blocks * a.block_size;
    int64_t len = a.lens[b];
    if (tid == 0 && kh == 0 && (len < 0 || len > max_len)) atomicAdd(a.errors, 1ull);
    len = len < 0 ? 0 : (len > max_len ? max_len : len);
    const int n_active = (int)((len + a.part_tokens - 1) / a.part_tokens);
    if (n_active <= 1) return;                          // written by the split kernel
    const int64_t slot_base = ((int64_t)b * a.n_q_heads + kh * G) * a.num_parts;
    // one wave per head: max over partitions, then weights exp2(m_p - m) / sum
    const int lane = tid & 63, wave = tid >> 6;
    for (int h = wave; h < G; h += kWaves) {
        const float *ml = a.part_ml + (slot_base + (int64_t)h * a.num_parts) * 2;
        float m = -INFINITY;
        for (int p = lane; p < n_active; p += 64) m = fmaxf(m, ml[2 * p]);
#pragma unroll
        for (int s = 32; s >= 1; s >>= 1) m = fmaxf(m, __shfl_xor(m, s));
        float l = 0.0f;
        for (int p = lane; p < n_active; p += 64) {
            const float w = exp2f(ml[2 * p] - m);
            s_w[h][p] = w;
            l += w * ml[2 * p + 1];
        }
#pragma unroll
        for (int s = 32; s >= 1; s >>= 1) l += __shfl_xor(l, s);
        if (lane == 0) s_inv[h] = 1.0f / l;
    }
    __syncthreads();
    for (int idx = tid; idx < G * D; idx += kThreads) {
        const int h = idx / D, d = idx - h * D;
        const float *po = a.part_o + (slot_base + (int64_t)h * a.num_parts) * D + d;
        float o = 0.0f;
#pragma unroll 8
        for (int p = 0; p < n_active; ++p) o += s_w[h][p] * po[(int64_t)p * D];
        store_out(a, ((int64_t)b * a.n_q_heads + kh * G + h) * D + d, o * s_inv[h]);
    }
}

template <int BS, int GMAX, bool QF32>
hipError_t launch_cfg(const DecodeArgs &a, hipStream_t s) {
    dim3 grid((unsigned)a.num_parts, (unsigned)a.n_kv_heads, (unsigned)a.batch);
    hipLaunchKernelGGL((decode_mfma_kernel<128, BS, GMAX, QF32>), grid, dim3(kThreads), 0, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.num_parts == 1) return e;
    hipLaunchKernelGGL((decode_merge_kernel<128, GMAX>), dim3((unsigned)a.batch, (unsigned)a.n_kv_heads),
                       dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

template <int BS, int GMAX>
hipError_t launch_q(const DecodeArgs &a, hipStream_t s) {
    return a.q_dtype == AIR_KV_F32 ? launch_cfg<BS, GMAX, true>(a, s) : launch_cfg<BS, GMAX, false>(a, s);
}

template <int BS>
hipError_t launch_bs(const DecodeArgs &a, hipStream_t s) {
    if (a.group <= 4) return launch_q<BS, 4>(a, s);
    if (a.group <= 8) return launch_q<BS, 8>(a, s);
    return launch_q<BS, 16>(a, s);
}

}  // namespace

bool decode_mfma_supported(int dtype, int head_dim, int block_size, int group) {
    return dtype == AIR_KV_BF16 && head_dim == 128 && (block_size == 16 || block_size == 32) &&
           group >= 1 && group <= 16;
}

hipError_t launch_decode_mfma(const DecodeArgs &a, hipStream_t s, int dtype, int head_dim) {
    (void)dtype;
    (void)head_dim;
    return a.block_size == 16 ? launch_bs<16>(a, s) : launch_bs<32>(a, s);
}

}  // namespace airkv
