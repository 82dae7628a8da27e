// Paged prefill attention (chunked, causal) on the matrix cores.
//
// For each sequence b, its q_len = cu_q[b + 1] - cu_q[b] newest tokens, whose
// K/V are already in the pages, attend causally over the sequence's seq_len
// cached tokens: query r sits at absolute position seq_len - q_len + r and
// sees keys 0 ..= that position.  This is blockwise_attention_head with
// q_offset = seq_len - q_len (src/chunked_attn.rs:114-213) per query head on
// kv head h / group (:240-243), i.e. the causal prefill branch of
// ops::attention with the mask of src/ops.rs:762-790, over paged storage.
//
// Work: a workgroup of four waves owns one (sequence, kv head) and four
// consecutive work items of it, item = token block * group + head of the
// group, a token block being 32 query rows.  With group 4 the four waves are
// the four query heads of one token block, so every K/V tile staged in LDS
// serves the whole GQA group.  Workgroups start in decreasing order of the
// keys their heaviest wave needs (prefill_slot below).
//
// Per 32-key tile, per wave (32 query rows):
//   S^T = K . Q^T   v_mfma_f32_32x32x16_bf16, M = 32 keys, N = 32 queries,
//                   K = head_dim in 8 steps of 16.  K is read from LDS in the
//                   A-operand layout (lane: key lane % 32, 8 contiguous
//                   head_dim elements at 16*step + 8*(lane / 32)); Q^T stays in
//                   registers in the matching B layout.  f32 queries are split
//                   into hi + lo bf16 halves and take two products per step.
//   online softmax in the log2 domain, one query per lane pair (lanes l and
//                   l + 32 hold 16 keys each); the running max is raised only
//                   when a tile exceeds it by 2^8, so probabilities stay below
//                   256 and most tiles skip rescaling the accumulators.
//   O^T += V^T . P^T  v_mfma_f32_32x32x16_f16, M = 32 head_dim rows (four
//                   tiles), N = 32 queries, K = 16 keys per step.  P^T is used
//                   where the S^T product left it: its B-operand keys are
//                   those of the C layout, keys (8*(i/4) + 4*(lane/32) + i%4)
//                   for registers i = 8*step .. +8.  V and P are f16 (11
//                   significant bits; bf16 probabilities alone leave ~3e-3
//                   relative error at these lengths).
//
// Two passes per work item.  The f16 pass above (1-byte pages: keys, values
// and queries dequantized or converted to f16 as well, one S^T product per
// step); a work item whose f16 result is not finite or whose every output of
// a query row lies below 2^-14 runs again with exact operands: V as bf16 and
// P as hi + lo bf16 halves (two PV products), 1-byte keys as hi + lo bf16
// halves (two S^T products) and values as one bf16 rounding with P's hi half.
//
// K and V tiles are staged row-major in three LDS stages (1-byte codes
// dequantized on the way); the V^T operand comes
// from two transposing reads (ds_read_b64_tr_b16) per 16 keys.  The loop is
// software-pipelined: the S^T product of tile t + 1 is issued before the
// softmax and PV products of tile t, tile t + 2 is written to LDS after them,
// and the page loads of tile t + 3 are in flight in registers, with one
// barrier per tile.
//
// Keys past the sequence and out-of-pool table entries are staged as zeros
// (stale page bytes may hold non-finite values).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "../host/status.hpp"
#include "../pool.hpp"
#include "codecs.hpp"
#include "prefill_common.hpp"

namespace airkv {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kRows = 32;                   // query rows per wave
constexpr int kKeys = 32;                   // keys per tile
constexpr int D = 128;                      // head_dim

#ifndef AIRKV_PREFILL_WAVES_PER_EU
#define AIRKV_PREFILL_WAVES_PER_EU 2        // register budget: waves per SIMD
#endif

__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x16 mfma32_f16(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// f16 pair (round to nearest even, element 0 in the low half).
__device__ __forceinline__ uint32_t f16_pair(float x, float y) {
    const f32x2 v = {x, y};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
}

// Eight bf16 values as f16: exact for magnitudes in [2^-17, 65504] (bf16's 8
// significant bits fit f16's 11, down into f16's subnormal range), rounded
// below that, and infinite above.
__device__ __forceinline__ u32x4 bf16x8_to_f16x8(u32x4 w) {
    u32x4 r;
#pragma unroll
    for (int j = 0; j < 4; ++j) r[j] = f16_pair(__uint_as_float(w[j] << 16), __uint_as_float(w[j] & 0xFFFF0000u));
    return r;
}

// bf16 bits (round to nearest even) of a finite f32.
__device__ __forceinline__ uint32_t bf16_bits(float x) {
    const uint32_t u = __float_as_uint(x);
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ void split_bf16(float x, uint32_t &hi, uint32_t &lo) {
    hi = bf16_bits(x);
    lo = bf16_bits(x - __uint_as_float(hi << 16));
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// (x, y) = hi + lo with both halves bf16 pairs (hardware round to nearest
// even): hi carries 8 significant bits, lo the next 8.
__device__ __forceinline__ void split_pair(float x, float y, uint32_t &hi, uint32_t &lo) {
    const f32x2 v = {x, y};
    const bf16x2 h = __builtin_convertvector(v, bf16x2);
    const f32x2 r = v - __builtin_convertvector(h, f32x2);
    hi = __builtin_bit_cast(uint32_t, h);
    lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(r, bf16x2));
}

// Eight cache elements of one row as bf16 (16 bytes).  bf16 pages are raw
// bits; int8 / fp8 pages are dequantized to the reference's f32 value
// (q as f32 * scale, src/kv_cache.rs:88; to_f32(code) * scale,
// src/fp8.rs:263-264) with one rounding, then rounded to bf16.  The fp8
// conversion is the hardware's OCP E4M3, which agrees with the reference
// decoder on every code its encoder emits.
template <int DT> struct Raw8;
template <> struct Raw8<AIR_KV_BF16> { u32x4 w; };
template <> struct Raw8<AIR_KV_INT8> { u32x2 w; float s; };
template <> struct Raw8<AIR_KV_FP8> { u32x2 w; float s; };

// Buffer descriptor word 3 for raw (untyped) buffer access on gfx9-class GPUs.
constexpr int kBufferWord3 = 0x00020000;

// One page slab (block_size rows of one kv head) as a buffer resource.  The
// tile's page bases are uniform, so the descriptors live in scalar registers
// and each thread's offsets inside a page stay constant across tiles.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t page_rsrc(const void *base, int64_t byte_off, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)((const char *)base + byte_off), (short)0, bytes,
                                             kBufferWord3);
}

// Unconditional load of 8 elements at byte offset `off` of a page (the page
// is always inside the pool: out-of-pool ids read block 0 and are zeroed
// when staged), plus the group scale for 1-byte pages.
template <int DT>
__device__ __forceinline__ void load_raw(__amdgpu_buffer_rsrc_t pg, __amdgpu_buffer_rsrc_t sc, int off,
                                         int soff, Raw8<DT> &r) {
    if constexpr (DT == AIR_KV_BF16) {
        r.w = __builtin_amdgcn_raw_buffer_load_b128(pg, off, 0, 0);
    } else {
        r.w = __builtin_amdgcn_raw_buffer_load_b64(pg, off, 0, 0);
        r.s = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(sc, soff, 0, 0));
    }
}

// Four 1-byte codes of word w times s as f32 pairs (elements 0, 1 and 2, 3):
// the reference's dequantized value with one rounding.  int8: the code
// biased to an unsigned byte (x ^ 0x80 = q + 128), and fma(q + 128, s, -128 s)
// is q * s rounded once; fp8: the hardware OCP E4M3 conversion.
template <int DT>
__device__ __forceinline__ void dequant4(uint32_t w, float s, f32x2 &lo, f32x2 &hi) {
    if constexpr (DT == AIR_KV_INT8) {
        const uint32_t u = w ^ 0x80808080u;
        const float off = -128.0f * s;
        lo = f32x2{__builtin_fmaf((float)(u & 0xFFu), s, off), __builtin_fmaf((float)((u >> 8) & 0xFFu), s, off)};
        hi = f32x2{__builtin_fmaf((float)((u >> 16) & 0xFFu), s, off), __builtin_fmaf((float)(u >> 24), s, off)};
    } else {
        lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false) * s;
        hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true) * s;
    }
}

template <int DT>
__device__ __forceinline__ u32x4 to_bf16x8(const Raw8<DT> &r) {
    if constexpr (DT == AIR_KV_BF16) {
        return r.w;
    } else {
        u32x4 o;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            f32x2 lo, hi;
            dequant4<DT>(r.w[h], r.s, lo, hi);
            o[2 * h] = __builtin_bit_cast(uint32_t, __builtin_convertvector(lo, bf16x2));
            o[2 * h + 1] = __builtin_bit_cast(uint32_t, __builtin_convertvector(hi, bf16x2));
        }
        return o;
    }
}

// Eight cache elements of one row as f16 (round to nearest even): bf16
// pages as bf16x8_to_f16x8 converts them; 1-byte pages dequantized as
// above and rounded once to f16's 11 significant bits (infinite beyond
// 65504).
template <int DT>
__device__ __forceinline__ u32x4 to_f16x8(const Raw8<DT> &r) {
    if constexpr (DT == AIR_KV_BF16) {
        return bf16x8_to_f16x8(r.w);
    } else {
        u32x4 o;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            f32x2 lo, hi;
            dequant4<DT>(r.w[h], r.s, lo, hi);
            o[2 * h] = f16_pair(lo[0], lo[1]);
            o[2 * h + 1] = f16_pair(hi[0], hi[1]);
        }
        return o;
    }
}

// Eight 1-byte codes dequantized as to_bf16x8 does, as hi + lo bf16 halves:
// hi the bf16 rounding of the f32 value x, lo that of x - hi (exact in f32),
// so hi + lo carries x to ~2^-17.
template <int DT>
__device__ __forceinline__ void to_bf16x8_split(const Raw8<DT> &r, u32x4 &hi, u32x4 &lo) {
    if constexpr (DT == AIR_KV_BF16) {
        hi = r.w;
        lo = u32x4{0, 0, 0, 0};
    } else {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            f32x2 a, b;
            dequant4<DT>(r.w[h], r.s, a, b);
            uint32_t h0, l0, h1, l1;
            split_pair(a[0], a[1], h0, l0);
            split_pair(b[0], b[1], h1, l1);
            hi[2 * h] = h0;
            lo[2 * h] = l0;
            hi[2 * h + 1] = h1;
            lo[2 * h + 1] = l1;
        }
    }
}

// Dispatch order.  The grid is one-dimensional: n_kv_heads workgroups for
// each of the batch * nz * ns_max (sequence, slot, piece) items, and the
// hardware starts workgroups in index order.  Slot z of sequence b serves
// that sequence's work group n_wg - 1 - z (and every nz-th one below it),
// whose heaviest wave needs the keys up to its last query row.
//
// Key split.  With a workspace (ns_max > 1), a slot that serves a single
// work group longer than the balanced load -- the batch's key tiles over the
// grid's resident workgroup slots, a.slots -- has its key tiles cut into
// ns = min(ns_max, ceil(tiles / T)) consecutive ranges, piece p taking range
// p; the pieces write unnormalised partial outputs (acc, running max, sum)
// to the workspace and prefill_merge_kernel combines them by log-sum-exp.
// Split slots get ordinals in index order; when more slots are that long
// than the workspace holds, T is raised until they fit.  Every workgroup
// derives the same T, pieces and ordinals from the lengths.
//
// Ranking.  Grid row r takes the item of rank r when items are ordered by
// the keys of their heaviest wave (a piece: its share), decreasing (in
// buckets of an eighth of an octave; ties by sequence, slot, piece), so long
// work starts first and short work fills the launch's tail.  Every item
// gets exactly one rank whatever the lengths hold.  Batches above kRankCap
// sequences or kRankItems items are taken slot by slot (slot slowest),
// without ranking or splitting.
constexpr int kRankCap = 2048;
constexpr int kRankItems = 64 * kThreads;
constexpr int kRankLdsBytes = (kThreads + kWaves + 8 + 2 * kRankCap) * 4;

struct PrefillSlot {
    int b, kh, z, nz;
    int p, ns, ord;            // piece, pieces of the slot (1: not split), split ordinal (-1: none)
};

__device__ __forceinline__ int len_bucket(int64_t len) {   // 0 .. 248, monotone in len
    if (len <= 0) return 0;
    const uint32_t x = len > 0x7fffffff ? 0x7fffffffu : (uint32_t)len;
    const int e = 31 - __builtin_clz(x);
    const int m = e >= 3 ? (int)(x >> (e - 3)) & 7 : (int)(x << (3 - e)) & 7;
    return 1 + 8 * e + m;
}

// Exclusive prefix sum over the workgroup's threads in thread order; wsum
// holds kWaves ints of LDS.  Contains barriers: every thread calls it.
__device__ __forceinline__ int block_exclusive_scan(int v, int *wsum) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int incl = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(incl, o);
        if (lane >= o) incl += y;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    int base = 0;
    for (int w = 0; w < wave; ++w) base += wsum[w];
    __syncthreads();
    return base + incl - v;
}

// Keys the heaviest wave of slot z of a sequence needs (0: no work).
__device__ __forceinline__ int64_t slot_keys(int64_t len, int64_t qlen, int G, int z) {
    if (qlen <= 0 || len < qlen) return 0;
    const int64_t n_items = (qlen + kRows - 1) / kRows * G;
    const int64_t n_wg = (n_items + kWaves - 1) / kWaves;
    if (z >= n_wg) return 0;
    const int64_t wi = n_wg - 1 - z;
    const int64_t last = wi * kWaves + kWaves - 1 < n_items ? wi * kWaves + kWaves - 1 : n_items - 1;
    const int64_t rows = (last / G + 1) * kRows;
    return len - qlen + (rows < qlen ? rows : qlen);
}

// Whether slot z of a sequence serves exactly one work group (splittable).
__device__ __forceinline__ bool single_unit(int64_t qlen, int G, int nz) {
    const int64_t n_items = (qlen + kRows - 1) / kRows * G;
    return (n_items + kWaves - 1) / kWaves <= nz;
}

__device__ __forceinline__ int slot_pieces(int64_t tiles, int64_t T, int ns_max) {
    if (tiles <= T) return 1;
    const int64_t n = (tiles + T - 1) / T;
    return (int)(n < ns_max ? n : ns_max);
}

// Whether sequence b's rows and length are consistent: 0 <= cu_q[b] <=
// cu_q[b + 1] <= total_q, 0 <= seq_len <= max_blocks * block_size and
// q_len <= seq_len.  The one test every prefill kernel applies: an
// inconsistent sequence is counted and zero-filled by its first workgroup,
// never split into pieces and never written by the merge.
__device__ __forceinline__ bool prefill_rows_ok(const PrefillArgs &a, int b) {
    const int32_t q0 = a.cu_q[b], q1 = a.cu_q[b + 1];
    return q0 >= 0 && q1 >= q0 && q1 <= a.total_q;
}
__device__ __forceinline__ bool prefill_seq_ok(const PrefillArgs &a, int b) {
    const int64_t len = a.lens[b];
    const int64_t qlen = (int64_t)a.cu_q[b + 1] - a.cu_q[b];
    return prefill_rows_ok(a, b) && len >= 0 && len <= a.max_len && qlen <= len;
}

// The plan of a split launch: one int2 per grid row {item, slot info}.
__device__ __forceinline__ int2 *prefill_plan_table(const PrefillArgs &a) {
    return reinterpret_cast<int2 *>((uint8_t *)a.ws + 64 + 16 * (int64_t)a.ws_units);
}

// Split launches (ns_max > 1) read their item from the plan that
// prefill_plan_kernel wrote to the workspace; others rank in every
// workgroup.  lds: at least kThreads + kWaves + 8 + 2 * kRankCap ints, free
// for the duration.
__device__ PrefillSlot prefill_slot(const PrefillArgs &a, int *lds) {
    const int tid = threadIdx.x;
    const int nz = a.nz, nsm = a.ns_max;
    const int row = (int)(blockIdx.x / (unsigned)a.n_kv_heads);
    PrefillSlot sl;
    sl.kh = (int)(blockIdx.x % (unsigned)a.n_kv_heads);
    sl.nz = nz;
    sl.p = 0;
    sl.ns = 1;
    sl.ord = -1;
    if (nsm > 1) {
        const int2 e = prefill_plan_table(a)[row];
        const int si = e.x / nsm;
        sl.p = e.x - si * nsm;
        sl.b = si / nz;
        sl.z = si - sl.b * nz;
        sl.ns = e.y & 15;
        sl.ord = (e.y >> 4) - 1;
        if (sl.p >= sl.ns) sl.b = -1;                   // no such piece: the workgroup exits
        return sl;
    }
    if (a.batch == 1 || a.batch > kRankCap || (int64_t)a.batch * nz > kRankItems) {
        // (one sequence: its slots are already in decreasing order)
        sl.b = row % a.batch;
        sl.z = row / a.batch;
        return sl;
    }
    int *hist = lds, *wsum = lds + kThreads, *sel = lds + kThreads + kWaves;
    int *slen = sel + 8, *sq = slen + kRankCap;
    hist[tid] = 0;
    for (int i = tid; i < a.batch; i += kThreads) {
        slen[i] = a.lens[i];
        const int64_t ql = (int64_t)a.cu_q[i + 1] - a.cu_q[i];
        sq[i] = ql < 0 ? 0 : ql > 0x7fffffff ? 0x7fffffff : (int)ql;
    }
    __syncthreads();
    const int n_it = a.batch * nz;
    const int chunk = (n_it + kThreads - 1) / kThreads;
    const int i0 = tid * chunk, i1 = i0 + chunk < n_it ? i0 + chunk : n_it;
    auto bucket_of = [&](int i) {
        const int bb = i / nz;
        return len_bucket(slot_keys(slen[bb], sq[bb], a.group, i - bb * nz));
    };
    for (int i = i0; i < i1; ++i) atomicAdd(&hist[bucket_of(i)], 1);
    __syncthreads();
    // buckets in decreasing order: thread t takes bucket kThreads - 1 - t
    const int bucket = kThreads - 1 - tid;
    const int cnt = hist[bucket];
    const int start = block_exclusive_scan(cnt, wsum);
    if (row >= start && row < start + cnt) {
        sel[0] = bucket;
        sel[1] = row - start;
    }
    __syncthreads();
    const int want = sel[0], j = sel[1];
    // the j-th item (index order) of bucket want: thread t scans its chunk
    int c = 0;
    for (int i = i0; i < i1; ++i) c += bucket_of(i) == want;
    const int before = block_exclusive_scan(c, wsum);
    if (j >= before && j < before + c) {
        int k = j - before;
        for (int i = i0; i < i1; ++i)
            if (bucket_of(i) == want && k-- == 0) sel[0] = i;
    }
    __syncthreads();
    const int item = sel[0];
    sl.b = item / nz;
    sl.z = item - sl.b * nz;
    __syncthreads();   // the caller reuses the LDS
    return sl;
}

// The plan of a split launch, once per launch (one workgroup of 256
// threads: split launches have few slots, and its barriers and scans cost
// less over four waves than sixteen, 6.9 -> 6.0 us): the split threshold T
// and each slot's pieces and ordinal (as above), every (sequence, slot,
// piece) item's rank by the keys of its heaviest wave (its share for a
// piece), decreasing in buckets of an eighth of an octave -- the order
// within a bucket is free, any order covers each item once -- and the
// descriptors of the split slots for the merge.
constexpr int kPlanThreads = 256;

__device__ __forceinline__ int plan_scan(int v, int *red, int &total) {   // exclusive, 1024 threads
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int incl = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(incl, o);
        if (lane >= o) incl += y;
    }
    if (lane == 63) red[wave] = incl;
    __syncthreads();
    int base = 0, tot = 0;
    for (int w = 0; w < kPlanThreads / 64; ++w) {
        base += w < wave ? red[w] : 0;
        tot += red[w];
    }
    __syncthreads();
    total = tot;
    return base + incl - v;
}

__global__ __launch_bounds__(kPlanThreads) void prefill_plan_kernel(PrefillArgs a) {
    __shared__ int slen[kRankCap], sq[kRankCap];
    __shared__ int info[kRankItems / 2];               // per slot: pieces | (ordinal + 1) << 4
    __shared__ int hist[256], cnt[256], red[kPlanThreads / 64];
    const int tid = threadIdx.x;
    const int nz = a.nz, nsm = a.ns_max;
    for (int i = tid; i < a.batch; i += kPlanThreads) {
        slen[i] = a.lens[i];
        // an inconsistent sequence plans as one with no rows: no keys, one
        // piece, never split (its first workgroup counts and zero-fills it)
        const int64_t ql = prefill_seq_ok(a, i) ? (int64_t)a.cu_q[i + 1] - a.cu_q[i] : 0;
        sq[i] = ql > 0x7fffffff ? 0x7fffffff : (int)ql;
    }
    if (tid < 256) hist[tid] = cnt[tid] = 0;
    __syncthreads();
    const int n_slots = a.batch * nz;
    auto tiles_of = [&](int si) -> int64_t {
        const int bb = si / nz;
        return (slot_keys(slen[bb], sq[bb], a.group, si - bb * nz) + kKeys - 1) / kKeys;
    };
    auto splittable = [&](int si) { return single_unit(sq[si / nz], a.group, nz); };
    // T: the balanced load (clamped terms: a balance target only), raised
    // until the split slots fit the workspace
    int part = 0, tot = 0;
    for (int si = tid; si < n_slots; si += kPlanThreads) {
        const int64_t t = tiles_of(si);
        part += (int)(t < (1 << 16) ? t : (1 << 16));
    }
    (void)plan_scan(part, red, tot);
    int64_t T = ((int64_t)tot * a.n_kv_heads + a.slots - 1) / a.slots;
    T = T < 8 ? 8 : T;                                  // pieces of at least 8 tiles
    for (;;) {
        int c = 0, n = 0;
        for (int si = tid; si < n_slots; si += kPlanThreads) c += splittable(si) && tiles_of(si) > T;
        (void)plan_scan(c, red, n);
        if (n <= a.ws_units) break;
        T += (T >> 2) + 1;
    }
    // pieces and ordinals (index order) of the slots: thread t owns a chunk
    const int chunk = (n_slots + kPlanThreads - 1) / kPlanThreads;
    const int s0 = tid * chunk, s1 = s0 + chunk < n_slots ? s0 + chunk : n_slots;
    int nsplit = 0;
    for (int si = s0; si < s1; ++si) {
        const int64_t t = tiles_of(si);
        const int ns = splittable(si) ? slot_pieces(t, T, nsm) : 1;
        info[si] = ns;
        nsplit += ns > 1;
    }
    int n_split = 0;
    int ord = plan_scan(nsplit, red, n_split);
    int32_t *hdr = reinterpret_cast<int32_t *>(a.ws);
    for (int si = s0; si < s1; ++si) {
        if (info[si] > 1) {
            int32_t *d = hdr + 16 + 4 * ord;
            d[0] = si / nz;
            d[1] = si % nz;
            d[2] = info[si];
            info[si] |= (ord + 1) << 4;
            ++ord;
        }
    }
    if (tid == 0) hdr[0] = n_split;
    __syncthreads();
    // rank every item: bucket histogram, descending starts, placement
    const int n_it = n_slots * nsm;
    auto bucket_of = [&](int i) {
        const int si = i / nsm, pp = i - si * nsm;
        const int ns = info[si] & 15;
        if (pp >= ns) return 0;
        if (ns == 1) {
            const int bb = si / nz;
            return len_bucket(slot_keys(slen[bb], sq[bb], a.group, si - bb * nz));
        }
        return len_bucket((tiles_of(si) + ns - 1) / ns * kKeys);
    };
    for (int i = tid; i < n_it; i += kPlanThreads) atomicAdd(&hist[bucket_of(i)], 1);
    __syncthreads();
    const int bk = tid < 256 ? 255 - tid : 0;           // thread t: bucket 255 - t (decreasing)
    int all = 0;
    const int st = plan_scan(tid < 256 ? hist[bk] : 0, red, all);
    if (tid < 256) cnt[bk] = st;
    __syncthreads();
    int2 *plan = prefill_plan_table(a);
    for (int i = tid; i < n_it; i += kPlanThreads) {
        const int r = atomicAdd(&cnt[bucket_of(i)], 1);
        plan[r] = int2{i, info[i / nsm]};
    }
}

// Per-(sequence, kv head) setup shared by the prefill kernels: reads the
// sequence's rows and length, counts (once) an inconsistent sequence and
// every out-of-pool table entry within its length, zero-fills the rows of an
// inconsistent sequence, and returns whether the workgroup has rows to
// compute.  Uniform per workgroup.
template <int BS>
__device__ bool prefill_begin(const PrefillArgs &a, const PrefillSlot &sl, int32_t &q0, int &qlen, int64_t &len) {
    const int b = sl.b, kh = sl.kh, tid = threadIdx.x;
    const int G = a.group;
    q0 = a.cu_q[b];
    len = a.lens[b];
    qlen = a.cu_q[b + 1] - q0;
    const bool rows_ok = prefill_rows_ok(a, b);
    const bool seq_ok = prefill_seq_ok(a, b);
    const int32_t *tbl = a.tables + (int64_t)b * a.max_blocks;
    if (sl.z == 0 && sl.p == 0 && kh == 0) {
        if (!seq_ok) {
            if (tid == 0) atomicAdd(a.errors, 1ull);
        } else if (qlen > 0) {
            for (int64_t j = tid; j < (len + BS - 1) / BS; j += kThreads) {
                const int32_t blk = tbl[j];
                if (blk < 0 || blk >= a.num_blocks) atomicAdd(a.errors, 1ull);
            }
        }
    }
    if (!seq_ok) {
        // rows of a sequence whose lengths are inconsistent become zeros
        if (rows_ok && sl.z == 0 && sl.p == 0) {
            const int64_t n = (int64_t)qlen * G * D;
            for (int64_t i = tid; i < n; i += kThreads) {
                const int64_t r = i / (G * D), e = i % (G * D);
                const int64_t idx = ((int64_t)(q0 + r) * a.n_q_heads + kh * G) * D + e;
                if (a.out_dtype == AIR_KV_F32) ((float *)a.out)[idx] = 0.0f;
                else ((uint16_t *)a.out)[idx] = 0;
            }
        }
        return false;
    }
    return qlen > 0;
}

// ---------------------------------------------------------------------------
// Three LDS stages and tiles software-pipelined inside each wave (every page
// dtype: 1-byte codes are dequantized to bf16 on their way to LDS).
//
// K and V tiles are staged row-major at padded pitches (below), which makes
// the K operand reads, the staging stores and the transposing V reads
// bank-conflict free.  The V^T operand comes from two transposing
// reads (ds_read_b64_tr_b16) per k-step: within each 16-lane group lane j
// receives element j % 4 of the 8 bytes addressed by lanes 4k + j / 4, so
// lane 16G + s points at V[kb + s/4][dblk + 4(s%4)] and receives V[kb + k][dblk
// + s], k = 0..3 -- four consecutive keys of one head_dim column, which are
// exactly the keys the S^T accumulator layout hands to P^T: keys 16 st + 4 hh
// + 0..3 and 16 st + 8 + 4 hh + 0..3 for lane half hh.
//
// Iteration t: the QK^T products of tile t + 1 are issued first (their K
// tile was staged an iteration earlier), then tile t's softmax runs on the
// vector ALUs while the matrix cores work, then tile t's PV products; tile
// t + 2 (loaded into registers an iteration earlier) is staged into the
// third LDS buffer and the loads of tile t + 3 are issued after the barrier.
// ---------------------------------------------------------------------------
constexpr int kStages = 3;
template <int N> struct Int { static constexpr int value = N; };
template <bool B> struct BoolC { static constexpr bool value = B; };
// Padded row pitches: K rows 272 bytes (consecutive rows start 4 banks
// apart, so the 16 rows of a K operand read hit 16 distinct 16-byte bank
// groups), V rows 320 bytes (rows start 16 banks apart, so the 4 rows x 64
// bytes of a transposing read cover the 64 banks once).  Every LDS address
// is then one per-lane register plus an immediate.
//
// 1-byte pages stage each dequantized key as two bf16 halves, hi + lo (hi the
// bf16 rounding of code * scale, lo that of the remainder: ~16 significant
// bits), in one 528-byte row (hi at 0, lo at 256; rows still 4 banks apart)
// and take a second QK^T product with the lo half.  One bf16 rounding of the
// keys moves logits by up to 2^-9 of each q_d * k_d term, which the outlier
// channels of quantized caches (20x the others) turn into >2e-2 output
// errors; the split leaves ~2^-17.  Three stages of the wider tile take
// 81408 bytes: two workgroups still fit a CU's 160 KB.
constexpr int VPITCH = D * 2 + 64;
constexpr int VTILE_BYTES = kKeys * VPITCH;
template <int DT> struct Lds {
    static constexpr bool kSplitK = DT != AIR_KV_BF16;
    static constexpr int KPITCH = D * 2 * (kSplitK ? 2 : 1) + 16;
    static constexpr int KTILE_BYTES = kKeys * KPITCH;
    static constexpr int STAGE_BYTES = KTILE_BYTES + VTILE_BYTES;   // K then V
    static constexpr int BYTES = kStages * STAGE_BYTES;
};
static_assert(2 * Lds<AIR_KV_INT8>::BYTES <= 160 * 1024, "two workgroups per CU");


// Partial output of piece p of split slot `ord`, kv head kh (layout in
// prefill_common.hpp).
__device__ __forceinline__ uint8_t *piece_base(const PrefillArgs &a, int ord, int kh, int p) {
    return (uint8_t *)a.ws + prefill_ws_header(a.ws_units, (int64_t)a.batch * a.nz * a.ns_max) +
           (((int64_t)ord * a.n_kv_heads + kh) * a.ns_max + p) * kPrefillPieceBytes;
}
__device__ __forceinline__ f32x4 *piece_acc(const PrefillArgs &a, int ord, int kh, int p, int wave) {
    return reinterpret_cast<f32x4 *>(piece_base(a, ord, kh, p)) + wave * 16 * 64;
}
__device__ __forceinline__ float *piece_ml(const PrefillArgs &a, int ord, int kh, int p) {
    return reinterpret_cast<float *>(piece_base(a, ord, kh, p) + kPrefillPieceAccBytes);
}

// One lane's 64 outputs (acc * inv) of query row r32, head_dim 32 n + 8 i4 +
// 4 hh + 0..3 (acc[n][4 * i4 .. + 4]), as out_dtype.
__device__ __forceinline__ void store_out(const PrefillArgs &a, const f32x16 (&acc)[D / 32], float inv,
                                          int64_t orow) {
    if (a.out_dtype == AIR_KV_F32) {
#pragma unroll
        for (int n = 0; n < D / 32; ++n)
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4)
                *reinterpret_cast<f32x4 *>((float *)a.out + orow + 32 * n + 8 * i4) =
                    f32x4{acc[n][4 * i4], acc[n][4 * i4 + 1], acc[n][4 * i4 + 2], acc[n][4 * i4 + 3]} * inv;
    } else {
#pragma unroll
        for (int n = 0; n < D / 32; ++n)
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                const f32x2 x = f32x2{acc[n][4 * i4], acc[n][4 * i4 + 1]} * inv;
                const f32x2 y = f32x2{acc[n][4 * i4 + 2], acc[n][4 * i4 + 3]} * inv;
                *reinterpret_cast<u32x2 *>((uint16_t *)a.out + orow + 32 * n + 8 * i4) =
                    u32x2{__builtin_bit_cast(uint32_t, __builtin_convertvector(x, bf16x2)),
                          __builtin_bit_cast(uint32_t, __builtin_convertvector(y, bf16x2))};
            }
    }
}

// store_out for the column blocks n = 2 half, 2 half + 1 of acc only.
__device__ __forceinline__ void store_out_half(const PrefillArgs &a, const f32x16 (&acc)[D / 32], int half,
                                               float inv, int64_t orow) {
#pragma unroll
    for (int nn = 0; nn < 2; ++nn) {
        const int n = 2 * half + nn;
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
            const f32x4 v = f32x4{acc[n][4 * i4], acc[n][4 * i4 + 1], acc[n][4 * i4 + 2], acc[n][4 * i4 + 3]} * inv;
            if (a.out_dtype == AIR_KV_F32) {
                *reinterpret_cast<f32x4 *>((float *)a.out + orow + 32 * n + 8 * i4) = v;
            } else {
                *reinterpret_cast<u32x2 *>((uint16_t *)a.out + orow + 32 * n + 8 * i4) =
                    u32x2{__builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{v[0], v[1]}, bf16x2)),
                          __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{v[2], v[3]}, bf16x2))};
            }
        }
    }
}

// Log-sum-exp merge of the pieces of split slot blockIdx.x / n_kv_heads, kv
// head blockIdx.x % n_kv_heads: lane for lane the partials the pieces wrote,
// folded in piece order with an online rescale by 2^(m_p - running max), then
// divided by the folded sum (the two lane halves of a query row hold halves
// of its keys).  Eight waves: wave w takes item wave w / 2 and half w % 2 of
// its lanes' 64 accumulators, and loads kMergeBatch pieces per round trip;
// the first batch is requested together with the slot's descriptor (piece
// addresses depend only on the slot, head, piece and wave), so a slot of up
// to kMergeBatch pieces costs one round trip before its output row.
constexpr int kMergeThreads = 512;
constexpr int kMergeBatch = 4;

__global__ __launch_bounds__(kMergeThreads) void prefill_merge_kernel(PrefillArgs a) {
    const int ord = (int)(blockIdx.x / (unsigned)a.n_kv_heads), kh = (int)(blockIdx.x % (unsigned)a.n_kv_heads);
    if (ord >= a.ws_units) return;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int iw = wave >> 1, half = wave & 1;          // item wave, half of its accumulators
    const int32_t *hdr = (const int32_t *)a.ws;
    const int32_t *d = hdr + 16 + 4 * ord;
    const int n_split = hdr[0];
    const int b = d[0], z = d[1], ns = d[2];
    float m = -INFINITY, l = 0.0f;
    f32x4 o[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) o[q] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int p0 = 0; p0 < a.ns_max; p0 += kMergeBatch) {
        // loads of pieces p0 .. p0 + kMergeBatch - 1 (within the slot's
        // ns_max workspace entries; pieces past ns are read but not folded)
        float pm[kMergeBatch], pl[kMergeBatch];
        f32x4 pv[kMergeBatch][8];
#pragma unroll
        for (int i = 0; i < kMergeBatch; ++i) {
            const int pp = p0 + i < a.ns_max ? p0 + i : p0;
            const float *ml = piece_ml(a, ord, kh, pp);
            pm[i] = ml[iw * 64 + lane];
            pl[i] = ml[kThreads + iw * 64 + lane];
            const f32x4 *pa = piece_acc(a, ord, kh, pp, iw) + 8 * half * 64 + lane;
#pragma unroll
            for (int q = 0; q < 8; ++q) pv[i][q] = pa[q * 64];
        }
        if (ord >= n_split || ns < 2 || ns > a.ns_max) return;   // uniform: an unused descriptor
#pragma unroll
        for (int i = 0; i < kMergeBatch; ++i) {
            // a piece past the slot's count, or with no visible key for this
            // row (running max -inf), adds nothing
            if (p0 + i >= ns || pm[i] == -INFINITY) continue;
            const float m_new = fmaxf(m, pm[i]);
            const float sa = __builtin_amdgcn_exp2f(m - m_new), sb = __builtin_amdgcn_exp2f(pm[i] - m_new);
            l = l * sa + pl[i] * sb;
#pragma unroll
            for (int q = 0; q < 8; ++q) o[q] = o[q] * sa + pv[i][q] * sb;
            m = m_new;
        }
        if (p0 + kMergeBatch >= ns) break;
    }
    if (b < 0 || b >= a.batch || z < 0 || z >= a.nz) return;
    if (!prefill_seq_ok(a, b)) return;                  // the plan never splits one: defence only
    const int G = a.group;
    const int32_t q0 = a.cu_q[b];
    const int qlen = a.cu_q[b + 1] - q0;
    const int n_items = (qlen + kRows - 1) / kRows * G;
    const int n_wg = (n_items + kWaves - 1) / kWaves;
    const int item = (n_wg - 1 - z) * kWaves + iw;
    const float L = l + __shfl_xor(l, 32);
    if (item >= n_items) return;                        // uniform per wave
    const int tb = item / G, h = kh * G + item % G, r0 = tb * kRows;
    const int r32 = lane & 31, hh = lane >> 5;
    if (r0 + r32 >= qlen) return;
    // this half's accumulators are acc[n][4 * i4 ..] for n = 2 half, 2 half + 1
    f32x16 acc[D / 32];
#pragma unroll
    for (int q = 0; q < 8; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[2 * half + q / 4][4 * (q % 4) + e] = o[q][e];
    store_out_half(a, acc, half, 1.0f / L, ((int64_t)(q0 + r0 + r32) * a.n_q_heads + h) * D + 4 * hh);
}

template <int BS, bool QF32, int DT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(AIRKV_PREFILL_WAVES_PER_EU)))
void prefill_pipe_kernel(PrefillArgs a) {
    constexpr int EB = DT == AIR_KV_BF16 ? 2 : 1;   // bytes per page element
    // Two passes.  First every work item runs with f16 operands (11
    // significant bits): V converted (bf16 pages) or dequantized (1-byte
    // pages) to f16 on its way to LDS and probabilities <= 2^8 rounded to
    // f16, one PV product per tile; 1-byte pages also take their keys
    // dequantized to f16 and the queries as f16 (f32 queries rounded once),
    // one S^T product per step instead of the key's bf16 hi + lo pair.  A work
    // item whose f16 result is not finite (a value beyond f16's 65504) or
    // whose every output of a query row is below 2^-14 in magnitude (values
    // so small that f16's subnormal spacing, 2^-24, would show) runs again
    // with the exact operands: bf16 pages V as bf16 and P as hi + lo bf16
    // halves (two products), 1-byte pages keys as hi + lo bf16 halves, V as
    // the bf16 rounding of code * scale and P's hi half.
    __shared__ int s_redo;
    if (threadIdx.x == 0) s_redo = 0;              // read only after barriers below
    constexpr bool kSplitK = Lds<DT>::kSplitK;
    constexpr int KPITCH = Lds<DT>::KPITCH, KTILE_BYTES = Lds<DT>::KTILE_BYTES;
    constexpr int STAGE_BYTES = Lds<DT>::STAGE_BYTES;
    __shared__ __align__(16) uint8_t smem[Lds<DT>::BYTES];
    static_assert(sizeof(smem) >= kRankLdsBytes, "dispatch ranking needs the tile LDS");
    PrefillSlot sl = prefill_slot(a, reinterpret_cast<int *>(smem));
    if (sl.b < 0) return;                               // a piece this launch does not use
    // uniform per workgroup: scalar registers
    sl.b = __builtin_amdgcn_readfirstlane(sl.b);
    sl.z = __builtin_amdgcn_readfirstlane(sl.z);
    sl.p = __builtin_amdgcn_readfirstlane(sl.p);
    sl.ns = __builtin_amdgcn_readfirstlane(sl.ns);
    sl.ord = __builtin_amdgcn_readfirstlane(sl.ord);
    const int b = sl.b, kh = sl.kh;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = a.group;
    int32_t q0;
    int qlen;
    int64_t len;
    if (!prefill_begin<BS>(a, sl, q0, qlen, len)) return;
    const int32_t *tbl = a.tables + (int64_t)b * a.max_blocks;
    const int q_offset = (int)(len - qlen);
    const int ntb = (qlen + kRows - 1) / kRows;
    const int n_items = ntb * G;
    const int n_wg = (n_items + kWaves - 1) / kWaves;
    const int r32 = lane & 31, hh = lane >> 5;

    // Staging: thread covers head_dim 8 * (tid % 16) .. + 8 of key rows
    // tid / 16 and 16 + tid / 16, for K and V alike (constant offsets inside
    // a page); 1-byte pages also load the f32 scale of that group.
    constexpr int PAGE_BYTES = BS * D * EB;
    const int n_sc = DT == AIR_KV_BF16 ? 1 : D / a.scale_group;
    int g_off[2], s_off[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int prow = ((tid >> 4) + 16 * i) % BS;
        g_off[i] = (prow * D + (tid & 15) * 8) * EB;
        s_off[i] = DT == AIR_KV_BF16 ? 0 : (prow * n_sc + ((tid & 15) * 8) / a.scale_group) * 4;
    }
    struct TileRegs {
        Raw8<DT> k[2], v[2];
        int kt;
        bool ok0, ok1;
    };
    int32_t nb0 = 0, nb1 = 0;          // block ids of the next tile to load (fetched a tile ahead)
    int tile0 = 0;                     // first key tile of the piece (0 unless split)
    auto fetch_ids = [&](int t, int kend) {
        const int last = (kend - 1) / BS;
        const int j0 = ((tile0 + t) * kKeys) / BS;
        nb0 = tbl[j0 < last ? j0 : last];
        if constexpr (BS == 16) nb1 = tbl[j0 + 1 < last ? j0 + 1 : last];
        else nb1 = nb0;
    };
    auto load_tile = [&](int t, TileRegs &R) {
        const int32_t b0 = __builtin_amdgcn_readfirstlane(nb0), b1 = __builtin_amdgcn_readfirstlane(nb1);
        R.kt = (tile0 + t) * kKeys;
        R.ok0 = b0 >= 0 && b0 < a.num_blocks;
        R.ok1 = b1 >= 0 && b1 < a.num_blocks;
        const int64_t row0 = ((int64_t)(R.ok0 ? b0 : 0) * a.n_kv_heads + kh) * BS;
        const int64_t row1 = ((int64_t)(R.ok1 ? b1 : 0) * a.n_kv_heads + kh) * BS;
        const __amdgpu_buffer_rsrc_t k0 = page_rsrc(a.k_pages, row0 * D * EB, PAGE_BYTES);
        const __amdgpu_buffer_rsrc_t v0 = page_rsrc(a.v_pages, row0 * D * EB, PAGE_BYTES);
        const __amdgpu_buffer_rsrc_t k1 = page_rsrc(a.k_pages, row1 * D * EB, PAGE_BYTES);
        const __amdgpu_buffer_rsrc_t v1 = page_rsrc(a.v_pages, row1 * D * EB, PAGE_BYTES);
        __amdgpu_buffer_rsrc_t ks0 = k0, vs0 = v0, ks1 = k1, vs1 = v1;   // unused for bf16
        if constexpr (DT != AIR_KV_BF16) {
            ks0 = page_rsrc(a.k_scales, row0 * n_sc * 4, BS * n_sc * 4);
            vs0 = page_rsrc(a.v_scales, row0 * n_sc * 4, BS * n_sc * 4);
            ks1 = page_rsrc(a.k_scales, row1 * n_sc * 4, BS * n_sc * 4);
            vs1 = page_rsrc(a.v_scales, row1 * n_sc * 4, BS * n_sc * 4);
        }
        load_raw<DT>(k0, ks0, g_off[0], s_off[0], R.k[0]);
        load_raw<DT>(v0, vs0, g_off[0], s_off[0], R.v[0]);
        load_raw<DT>(BS == 16 ? k1 : k0, BS == 16 ? ks1 : ks0, g_off[1], s_off[1], R.k[1]);
        load_raw<DT>(BS == 16 ? v1 : v0, BS == 16 ? vs1 : vs0, g_off[1], s_off[1], R.v[1]);
    };
    // Keys past the sequence and rows of out-of-pool blocks are staged as
    // zeros (stale page bytes may hold non-finite values); only the tiles
    // that hold such keys (a uniform test) pay for the selects.
    auto stage_tile = [&](auto f16v, int slot, TileRegs &R, int kend) {
        constexpr bool F16V = decltype(f16v)::value;    // V staged as f16 (bf16 pages)
        uint8_t *ks = smem + slot * STAGE_BYTES;
        uint8_t *vs = ks + KTILE_BYTES;
        u32x4 kb[2], vb[2];                       // as bf16 (1-byte pages dequantized)
        if constexpr (DT == AIR_KV_BF16) {
            // masked in the load registers themselves: no copies on the
            // common path
            if (!(R.ok0 && R.ok1 && R.kt + kKeys <= kend)) {
                const u32x4 zero = {0, 0, 0, 0};
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const bool okp = (BS == 16 && i == 1) ? R.ok1 : R.ok0;
                    const bool live = R.kt + (tid >> 4) + 16 * i < kend && okp;
                    R.k[i].w = live ? R.k[i].w : zero;
                    R.v[i].w = live ? R.v[i].w : zero;
                }
            }
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int row = (tid >> 4) + 16 * i;
                *reinterpret_cast<u32x4 *>(ks + row * KPITCH + (tid & 15) * 16) = R.k[i].w;
                *reinterpret_cast<u32x4 *>(vs + row * VPITCH + (tid & 15) * 16) =
                    F16V ? bf16x8_to_f16x8(R.v[i].w) : R.v[i].w;
            }
            return;
        }
        u32x4 kl[2];                              // lo halves of the keys (exact pass)
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            if constexpr (F16V) {
                kb[i] = to_f16x8<DT>(R.k[i]);
                kl[i] = u32x4{0, 0, 0, 0};
                vb[i] = to_f16x8<DT>(R.v[i]);
            } else {
                to_bf16x8_split<DT>(R.k[i], kb[i], kl[i]);
                vb[i] = to_bf16x8<DT>(R.v[i]);
            }
        }
        if (!(R.ok0 && R.ok1 && R.kt + kKeys <= kend)) {
            const u32x4 zero = {0, 0, 0, 0};
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const bool okp = (BS == 16 && i == 1) ? R.ok1 : R.ok0;
                const bool live = R.kt + (tid >> 4) + 16 * i < kend && okp;
                kb[i] = live ? kb[i] : zero;
                kl[i] = live ? kl[i] : zero;
                vb[i] = live ? vb[i] : zero;
            }
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int row = (tid >> 4) + 16 * i;
            *reinterpret_cast<u32x4 *>(ks + row * KPITCH + (tid & 15) * 16) = kb[i];
            if constexpr (!F16V) *reinterpret_cast<u32x4 *>(ks + row * KPITCH + D * 2 + (tid & 15) * 16) = kl[i];
            *reinterpret_cast<u32x4 *>(vs + row * VPITCH + (tid & 15) * 16) = vb[i];
        }
    };

    for (int w = sl.z; w < n_wg; w += sl.nz) {
        const int wi = n_wg - 1 - w;                   // heaviest work first
        const int item = wi * kWaves + wave;
        const bool wvalid = item < n_items;
        const int tb = (wvalid ? item : n_items - 1) / G;
        const int g = (wvalid ? item : n_items - 1) % G;
        const int h = kh * G + g;
        const int r0 = tb * kRows;
        const int last_item = (wi * kWaves + kWaves - 1 < n_items ? wi * kWaves + kWaves - 1 : n_items - 1);
        const int tb_last = last_item / G;
        const int rows_last = (tb_last + 1) * kRows < qlen ? (tb_last + 1) * kRows : qlen;
        const int kend = q_offset + rows_last;          // keys the workgroup needs (<= len)
        // uniform per workgroup / wave: kept in scalar registers so the
        // guards below are scalar branches
        // the piece's key tiles: [tile0, tile0 + nt) of the unit's nt_all
        const int nt_all = (kend + kKeys - 1) / kKeys;
        tile0 = __builtin_amdgcn_readfirstlane(sl.ns > 1 ? sl.p * nt_all / sl.ns : 0);
        const int nt = __builtin_amdgcn_readfirstlane(sl.ns > 1 ? (sl.p + 1) * nt_all / sl.ns - tile0 : nt_all);
        const int diag_kt = __builtin_amdgcn_readfirstlane(q_offset + r0 - kKeys + 1);   // first masked tile start

        const int qrow = r0 + r32 < qlen ? r0 + r32 : qlen - 1;
        const int qpos = q_offset + qrow;
        u32x4 qhi[D / 16], qlo[D / 16];
        // The query operands of a pass: bf16 (f32 queries as hi + lo bf16
        // halves), or for the f16 pass over 1-byte pages f16 (f32 queries as
        // hi + lo f16 halves, ~22 significant bits).
        auto load_q = [&](auto f16q) {
            constexpr bool F16Q = decltype(f16q)::value;
            const int64_t qbase = ((int64_t)(q0 + qrow) * a.n_q_heads + h) * D + 8 * hh;
#pragma unroll
            for (int ks = 0; ks < D / 16; ++ks) {
                if constexpr (QF32) {
                    const f32x4 *qp = reinterpret_cast<const f32x4 *>((const float *)a.q + qbase + 16 * ks);
                    const f32x4 x0 = qp[0], x1 = qp[1];
                    const float x[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        if constexpr (F16Q) {
                            // f16 pass, 1-byte pages: the query rounded to f16
                            // once (11 significant bits, finer than a bf16
                            // query, which the same pass takes exactly); a
                            // value beyond f16's range sends the work item to
                            // the exact pass, which splits it into hi + lo
                            qhi[ks][j] = f16_pair(x[2 * j], x[2 * j + 1]);
                            qlo[ks][j] = 0u;
                        } else {
                            uint32_t hb, lb;
                            split_pair(x[2 * j], x[2 * j + 1], hb, lb);
                            qhi[ks][j] = hb;
                            qlo[ks][j] = lb;
                        }
                    }
                } else {
                    qhi[ks] = *reinterpret_cast<const u32x4 *>((const uint16_t *)a.q + qbase + 16 * ks);
                    qlo[ks] = u32x4{0, 0, 0, 0};
                    if constexpr (F16Q) {              // bf16 -> f16, exact within f16's range
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            qhi[ks][j] = f16_pair(__uint_as_float(qhi[ks][j] << 16),
                                                  __uint_as_float(qhi[ks][j] & 0xFFFF0000u));
                    }
                }
            }
            // consumed here so no vector-memory wait lands inside the tile loop
#pragma unroll
            for (int ks = 0; ks < D / 16; ++ks) {
                asm volatile("" ::"v"(qhi[ks]));
                if constexpr (QF32 && !F16Q) asm volatile("" ::"v"(qlo[ks]));
            }
        };

        f32x16 acc[D / 32];
        float m_run = -INFINITY, l_run = 0.0f;

        auto qk = [&](auto f16k, int slot) {
            constexpr bool F16K = decltype(f16k)::value && DT != AIR_KV_BF16;   // f16 keys and queries
            const uint8_t *ks_ = smem + slot * STAGE_BYTES;
            f32x16 s;
#pragma unroll
            for (int i = 0; i < 16; ++i) s[i] = 0.0f;
#pragma unroll
            for (int ks = 0; ks < D / 16; ++ks) {
                const u32x4 kA = *reinterpret_cast<const u32x4 *>(ks_ + r32 * KPITCH + (2 * ks + hh) * 16);
                if constexpr (F16K) {
                    s = mfma32_f16(kA, qhi[ks], s);
                    continue;
                }
                s = mfma32(kA, qhi[ks], s);
                if constexpr (QF32) s = mfma32(kA, qlo[ks], s);
                if constexpr (kSplitK) {
                    const u32x4 kL =
                        *reinterpret_cast<const u32x4 *>(ks_ + r32 * KPITCH + D * 2 + (2 * ks + hh) * 16);
                    s = mfma32(kL, qhi[ks], s);
                }
            }
            return s;
        };
        // softmax of tile t (scores s, S^T layout), first half: causal mask,
        // tile max, lazy rescale
        auto softmax_head = [&](int t, f32x16 &sc) {
            const int kt = (tile0 + t) * kKeys;
            if (kt > diag_kt) {   // masked in place: keys past the query's position
                const int kq = qpos - kt - 4 * hh;
#pragma unroll
                for (int i = 0; i < 16; ++i) sc[i] = 8 * (i >> 2) + (i & 3) <= kq ? sc[i] : -INFINITY;
            }
            // a tree of three-input maxima, then the lane 32 apart through
            // the gfx950 lane swap (a VALU op; a shuffle is an LDS round trip
            // on the path to the exponentials)
            const float m0 = fmaxf(fmaxf(sc[0], sc[1]), sc[2]), m1 = fmaxf(fmaxf(sc[3], sc[4]), sc[5]);
            const float m2 = fmaxf(fmaxf(sc[6], sc[7]), sc[8]), m3 = fmaxf(fmaxf(sc[9], sc[10]), sc[11]);
            const float m4 = fmaxf(fmaxf(sc[12], sc[13]), sc[14]);
            float mt = fmaxf(fmaxf(fmaxf(m0, m1), m2), fmaxf(fmaxf(m3, m4), sc[15]));
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mt), __float_as_uint(mt), false, false);
            mt = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) * a.scale_log2;
            if (__ballot(mt > m_run + 8.0f) != 0ull) {
                const float m_new = fmaxf(m_run, mt);
                const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);   // 0 on the first tile
                l_run *= alpha;
#pragma unroll
                for (int n = 0; n < D / 32; ++n) acc[n] *= alpha;
                m_run = m_new;
            }
        };
        // second half: probabilities, their sum, and the PV products (f16,
        // bf16 hi + lo, or bf16 hi only)
        auto softmax_pv = [&](auto f16pv, int slot, const f32x16 &sc) {
            constexpr bool F16 = decltype(f16pv)::value;
            constexpr bool kSplitP = DT == AIR_KV_BF16 && !F16;
            float p[16];
#pragma unroll
            for (int i = 0; i < 16; ++i)   // masked: exp2(-inf) = 0
                p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[i], a.scale_log2, -m_run));
            float ls = p[0];
#pragma unroll
            for (int i = 1; i < 16; ++i) ls += p[i];
            l_run += ls;
            const uint8_t *vs_ = smem + slot * STAGE_BYTES + KTILE_BYTES;
            typedef short s16x4 __attribute__((ext_vector_type(4)));
            const int grp = lane >> 4, sl = lane & 15;
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                uint32_t hv[4], lv[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if constexpr (F16) {
                        hv[j] = f16_pair(p[8 * st + 2 * j], p[8 * st + 2 * j + 1]);
                        lv[j] = 0;
                    } else if constexpr (kSplitP) {
                        split_pair(p[8 * st + 2 * j], p[8 * st + 2 * j + 1], hv[j], lv[j]);
                    } else {
                        const f32x2 pv = {p[8 * st + 2 * j], p[8 * st + 2 * j + 1]};
                        hv[j] = __builtin_bit_cast(uint32_t, __builtin_convertvector(pv, bf16x2));
                        lv[j] = 0;
                    }
                }
                const u32x4 phi = {hv[0], hv[1], hv[2], hv[3]}, plo = {lv[0], lv[1], lv[2], lv[3]};
                const int vrow = 16 * st + 4 * hh + (sl >> 2);           // keys kb .. kb + 3, then + 8
#pragma unroll
                for (int n = 0; n < D / 32; ++n) {
                    const int col = 32 * n + 16 * (grp & 1) + 4 * (sl & 3);   // 16-bit column of the 8 bytes
                    const s16x4 t0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (__attribute__((address_space(3))) s16x4 *)(vs_ + vrow * VPITCH + col * 2));
                    const s16x4 t1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (__attribute__((address_space(3))) s16x4 *)(vs_ + (vrow + 8) * VPITCH + col * 2));
                    const u32x2 a0 = __builtin_bit_cast(u32x2, t0), a1 = __builtin_bit_cast(u32x2, t1);
                    const u32x4 va = {a0[0], a0[1], a1[0], a1[1]};
                    if constexpr (F16) {
                        acc[n] = mfma32_f16(va, phi, acc[n]);
                    } else {
                        acc[n] = mfma32(va, phi, acc[n]);
                        if constexpr (kSplitP) acc[n] = mfma32(va, plo, acc[n]);
                    }
                }
            }
        };

        // One pass over the item's key tiles: acc, m_run and l_run from
        // scratch, with the PV products of `f16pv`.
        auto run_pass = [&](auto f16pv) {
            constexpr bool F16 = decltype(f16pv)::value;
            constexpr bool kSplitP = DT == AIR_KV_BF16 && !F16;
            load_q(BoolC<F16 && DT != AIR_KV_BF16>{});
#pragma unroll
            for (int n = 0; n < D / 32; ++n)
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[n][i] = 0.0f;
            m_run = -INFINITY;
            l_run = 0.0f;
            TileRegs R;
            fetch_ids(0, kend);
            load_tile(0, R);
            fetch_ids(1, kend);
            stage_tile(f16pv, 0, R, kend);
            if (nt > 1) {
                load_tile(1, R);
                fetch_ids(2, kend);
                stage_tile(f16pv, 1, R, kend);
            }
            if (nt > 2) {
                load_tile(2, R);
                fetch_ids(3, kend);
            }
            __syncthreads();
            // One pipeline step for tile t, whose LDS slot S = t % 3 is a
            // compile-time constant (the loop is unrolled six times: three slots
            // times two score buffers), so every LDS address is a loop-invariant
            // register plus an immediate offset.
            auto step = [&](int t, auto slot, f32x16 &s_cur, f32x16 &s_next) {
                constexpr int S = decltype(slot)::value;
                // Unconditional: a wave past the last tile its own rows need sees
                // only keys beyond its rows, which the mask turns into zero
                // probabilities, and the S^T product of a slot past the last
                // tile reads stale but in-bounds LDS that is never used.  One
                // basic block then holds tile t + 1's S^T products and tile t's
                // exponentials and PV products, interleaved below.
                // The products and exponentials run at raised wave priority and
                // staging, the barrier and the page loads at the base one: when
                // both waves of a SIMD can issue, the one computing goes first
                // (measured 0-7% faster across chunk mixes, none slower).
                __builtin_amdgcn_s_setprio(1);
                softmax_head(t, s_cur);
                s_next = qk(f16pv, (S + 1) % kStages);
                softmax_pv(f16pv, S, s_cur);
                constexpr int kQk = (kSplitK && !F16) ? 16 : 8;      // K operand reads per tile
                __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
                for (int i = 0; i < kQk; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 48 / kQk, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
                constexpr int kPv = kSplitP ? 16 : 8;      // PV products per tile
#pragma unroll
                for (int i = 0; i < kPv; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x100, 16 / kPv, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
                }
                __builtin_amdgcn_s_setprio(0);
                if (t + 2 < nt) stage_tile(f16pv, (S + 2) % kStages, R, kend);
                __syncthreads();
                if (t + 3 < nt) {
                    load_tile(t + 3, R);
                    fetch_ids(t + 4, kend);
                }
            };
            f32x16 sa = qk(f16pv, 0), sb = sa;
            for (int t = 0; t < nt; t += 6) {
                step(t, Int<0>{}, sa, sb);
                if (t + 1 < nt) step(t + 1, Int<1>{}, sb, sa);
                if (t + 2 < nt) step(t + 2, Int<2>{}, sa, sb);
                if (t + 3 < nt) step(t + 3, Int<0>{}, sb, sa);
                if (t + 4 < nt) step(t + 4, Int<1>{}, sa, sb);
                if (t + 5 < nt) step(t + 5, Int<2>{}, sb, sa);
            }
        };

        // the sum of the query row's probabilities (its two lanes hold halves
        // of its keys)
        const bool row_live = wvalid && r0 + r32 < qlen;
        {
            run_pass(BoolC<true>{});
            // Checked on the row's unnormalised outputs: a non-finite sum, or
            // every |output| below 2^-14 (max |acc| < 2^-14 * l) on a row that
            // saw keys, sends the whole work item through the exact pass.
            float sum = 0.0f, mx = 0.0f;
#pragma unroll
            for (int n = 0; n < D / 32; ++n)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    sum += acc[n][i];
                    mx = fmaxf(mx, fabsf(acc[n][i]));
                }
            const float l = l_run + __shfl_xor(l_run, 32);
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const bool bad = row_live && (!__builtin_isfinite(sum) || (l > 0.0f && mx < 0x1p-14f * l));
            if (__ballot(bad) != 0ull && lane == 0) s_redo = 1;
            __syncthreads();
            const bool redo = s_redo != 0;
            __syncthreads();                           // every wave has read the flag
            if (redo) {
                if (tid == 0) s_redo = 0;              // next read after this pass's barriers
                run_pass(BoolC<false>{});
            }
        }

        if (sl.ns > 1) {
            // a piece of a split slot: the unnormalised partial (acc, running
            // max, this lane's sum) of every lane, in lane order
            f32x4 *pa = piece_acc(a, sl.ord, kh, sl.p, wave);
#pragma unroll
            for (int n = 0; n < D / 32; ++n)
#pragma unroll
                for (int i4 = 0; i4 < 4; ++i4)
                    pa[(4 * n + i4) * 64 + lane] =
                        f32x4{acc[n][4 * i4], acc[n][4 * i4 + 1], acc[n][4 * i4 + 2], acc[n][4 * i4 + 3]};
            float *pml = piece_ml(a, sl.ord, kh, sl.p);
            pml[wave * 64 + lane] = m_run;
            pml[kThreads + wave * 64 + lane] = l_run;
        } else if (row_live) {
            const float l = l_run + __shfl_xor(l_run, 32);
            store_out(a, acc, 1.0f / l, ((int64_t)(q0 + r0 + r32) * a.n_q_heads + h) * D + 4 * hh);
        }
        __syncthreads();      // the next work item restages every LDS buffer
    }
}

template <int BS, int DT>
hipError_t launch_dt(const PrefillArgs &a, hipStream_t s, dim3 grid) {
    if (a.q_dtype == AIR_KV_F32)
        hipLaunchKernelGGL((prefill_pipe_kernel<BS, true, DT>), grid, dim3(kThreads), 0, s, a);
    else
        hipLaunchKernelGGL((prefill_pipe_kernel<BS, false, DT>), grid, dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

template <int BS>
hipError_t launch_bs(const PrefillArgs &a, int dtype, hipStream_t s, dim3 grid) {
    switch (dtype) {
    case AIR_KV_BF16: return launch_dt<BS, AIR_KV_BF16>(a, s, grid);
    case AIR_KV_INT8: return launch_dt<BS, AIR_KV_INT8>(a, s, grid);
    default: return launch_dt<BS, AIR_KV_FP8>(a, s, grid);
    }
}

}  // namespace

bool prefill_supported(int dtype, int head_dim, int block_size, int scale_group) {
    if (head_dim != D || (block_size != 16 && block_size != 32)) return false;
    if (dtype == AIR_KV_BF16) return true;
    // 1-byte pages: a thread's 8 contiguous codes must share one scale
    return (dtype == AIR_KV_INT8 || dtype == AIR_KV_FP8) && scale_group >= 8;
}

PrefillPlan prefill_plan(int32_t batch, int32_t n_kv_heads, int32_t group, int32_t max_q_len, int cus) {
    PrefillPlan pl;
    // nz slots per sequence sized for max_q_len; the kernel strides over its
    // slots, so a sequence longer than max_q_len is still covered completely
    const int64_t ntb = ((int64_t)(max_q_len > 0 ? max_q_len : 1) + kRows - 1) / kRows;
    int64_t nz = (ntb * group + kWaves - 1) / kWaves;
    const int64_t units_all = (int64_t)batch * n_kv_heads * nz;
    const int64_t slots = 2 * (int64_t)cus;             // two resident workgroups per CU
    // The key split pays where the launch has fewer work groups than
    // resident workgroup slots (one 32K-token sequence: 274 -> 495 TFLOP/s;
    // two of 16K: +18%).  With more, the longest groups start first and the
    // tail runs them on emptier CUs: at the c5 chunk mix (1024 groups on 512
    // slots) splitting gained 6% in the main kernel and lost more to the plan
    // and the merge.  Pieces per slot: enough for one per resident slot, 2..8
    // (against two per resident slot: one 32K-token sequence 582 -> 736
    // TFLOP/s, two of 16K 680 -> 785, one 8K int8 sequence at the 70B
    // geometry 437 -> 521; half the partial outputs, and each piece's fixed
    // costs spread over twice the keys).
    int64_t ns = 1;
    if (units_all < slots) {
        ns = (slots + units_all - 1) / (units_all > 0 ? units_all : 1);
        ns = ns < 2 ? 2 : ns > 8 ? 8 : ns;
    }
    // a dispatch counts its work-items in 32 bits: at most 2^32 / 256 - 1
    // workgroups (fewer slots per sequence only lengthen each slot's stride)
    const int64_t cap = ((int64_t)0xffffffff / kThreads) / ((int64_t)batch * n_kv_heads * ns);
    nz = nz > cap ? cap : nz;
    pl.nz = (int32_t)nz;
    pl.ns_max = (int32_t)ns;
    // split slots are longer than the balanced load, so at most slots / n_kv_heads of them
    const int64_t units = std::min<int64_t>((int64_t)batch * nz, std::max<int64_t>(1, slots / n_kv_heads));
    const bool ranked = batch <= kRankCap && (int64_t)batch * nz * ns <= kRankItems &&
                        (int64_t)batch * nz <= kRankItems / 2;
    if (ns == 1 || !ranked) {                           // the key split rides on the ranked plan
        pl.ns_max = 1;
        pl.units = 0;
        pl.ws_bytes = 0;
        return pl;
    }
    pl.units = (int32_t)units;
    pl.ws_bytes = prefill_ws_header(units, (int64_t)batch * nz * ns) + units * n_kv_heads * ns * kPrefillPieceBytes;
    return pl;
}

hipError_t launch_prefill(PrefillArgs a, int dtype, int block_size, int32_t max_q_len, int cus,
                          hipStream_t s) {
    const PrefillPlan pl = prefill_plan(a.batch, a.n_kv_heads, a.group, max_q_len, cus);
    if (pl.nz < 1) return hipErrorInvalidConfiguration;
    a.nz = pl.nz;
    a.slots = 2 * cus;
    a.max_len = (int64_t)a.max_blocks * block_size;
    if (!a.ws || a.ws_units < 1 || pl.ns_max == 1) {
        a.ns_max = 1;
        a.ws = nullptr;
        a.ws_units = 0;
    } else {
        a.ns_max = pl.ns_max;
    }
    if (a.ns_max > 1) {
        hipLaunchKernelGGL(prefill_plan_kernel, dim3(1), dim3(kPlanThreads), 0, s, a);
        const hipError_t pe = hipGetLastError();
        if (pe != hipSuccess) return pe;
    }
    const dim3 grid((unsigned)((int64_t)a.batch * a.n_kv_heads * a.nz * a.ns_max));
    hipError_t e = block_size == 16 ? launch_bs<16>(a, dtype, s, grid) : launch_bs<32>(a, dtype, s, grid);
    if (e != hipSuccess || a.ns_max == 1) return e;
    hipLaunchKernelGGL(prefill_merge_kernel, dim3((unsigned)((int64_t)a.ws_units * a.n_kv_heads)),
                       dim3(kMergeThreads), 0, s, a);
    return hipGetLastError();
}

}  // namespace airkv
