// HBM ceiling kernels for the benchmark (not part of libairkv.so): what this
// GPU sustains for the access patterns of the paged-KV kernels, measured in
// the same run as them, so their rates can be read against an achievable
// bound as well as the 8 TB/s spec.
//
//   read      contiguous 16-byte loads, 64 bytes per thread (the decode's
//             byte stream without its page scatter)
//   page_read 4 KB pages in a shuffled order, one wave per page, K and V
//             pools: the decode's access pattern
//   write     contiguous 16-byte stores
//   copy      read + write of equal sizes: the gather's and block copies'
//             pattern (1 byte written per byte read)
//   mix21     two bytes read per byte written: the append's pattern (f32
//             rows in, bf16 page rows out)
//   page_copy 4 KB pages read in a shuffled order, written to consecutive
//             4 KB slots: the gather's pattern
//   page_mix21 8 KB of contiguous rows read per 4 KB page written in a
//             shuffled order: the append's pattern
//   copy / mix21 persistent: the same contiguous patterns as grid-stride
//             loops over 8 workgroups per CU with 128 or 256 bytes of loads
//             in flight per thread
//
// Each pattern has a plain and a non-temporal (`nt`: streaming) variant of
// its loads and of its stores; the bench reports the faster.  Every thread
// moves exactly 64 bytes of reads (and its share of writes) per launch, so a
// 1 GiB buffer is 65536 workgroups of 256 threads.  Loads feed a value that
// is stored only on an impossible condition, so nothing is optimised away.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kThreads = 256;

template <bool NT>
__device__ __forceinline__ u32x4 ld16(const u32x4 *p) {
    if constexpr (NT) return __builtin_nontemporal_load(p);
    return *p;
}

template <bool NT>
__device__ __forceinline__ void st16(u32x4 *p, u32x4 v) {
    if constexpr (NT) __builtin_nontemporal_store(v, p);
    else *p = v;
}

__device__ __forceinline__ uint32_t fold(u32x4 a, u32x4 b, u32x4 c, u32x4 d) {
    const u32x4 x = (a ^ b) + (c ^ d);
    return x[0] ^ x[1] ^ x[2] ^ x[3];
}

// Thread t reads 64 B as four 16-byte loads spread a wave apart (each load
// instruction of a wave covers 1 KB of consecutive lines).
template <bool NT>
__global__ __launch_bounds__(kThreads) void read_kernel(const u32x4 *src, int64_t n16, uint32_t *sink) {
    const int64_t base = (int64_t)blockIdx.x * kThreads * 4 + threadIdx.x;
    if (base + 3 * kThreads >= n16) return;
    const u32x4 a = ld16<NT>(src + base), b = ld16<NT>(src + base + kThreads);
    const u32x4 c = ld16<NT>(src + base + 2 * kThreads), d = ld16<NT>(src + base + 3 * kThreads);
    const uint32_t x = fold(a, b, c, d);
    if (x == 0x9E3779B9u && threadIdx.x == 7) sink[0] = x;
}

template <bool NT>
__global__ __launch_bounds__(kThreads) void write_kernel(u32x4 *dst, int64_t n16, uint32_t seed) {
    const int64_t base = (int64_t)blockIdx.x * kThreads * 4 + threadIdx.x;
    if (base + 3 * kThreads >= n16) return;
    const u32x4 v = {seed, seed ^ 1u, seed ^ 2u, (uint32_t)base};
#pragma unroll
    for (int i = 0; i < 4; ++i) st16<NT>(dst + base + i * kThreads, v);
}

// Every load of a thread is issued before its stores.
template <bool NTL, bool NTS>
__global__ __launch_bounds__(kThreads) void copy_kernel(const u32x4 *src, u32x4 *dst, int64_t n16) {
    const int64_t base = (int64_t)blockIdx.x * kThreads * 4 + threadIdx.x;
    if (base + 3 * kThreads >= n16) return;
    u32x4 v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = ld16<NTL>(src + base + i * kThreads);
#pragma unroll
    for (int i = 0; i < 4; ++i) st16<NTS>(dst + base + i * kThreads, v[i]);
}

// 64 B read, 32 B written per thread (contiguous both sides).
template <bool NTL, bool NTS>
__global__ __launch_bounds__(kThreads) void mix21_kernel(const u32x4 *src, u32x4 *dst, int64_t n16) {
    const int64_t base = (int64_t)blockIdx.x * kThreads * 4 + threadIdx.x;
    if (base + 3 * kThreads >= n16) return;
    u32x4 v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = ld16<NTL>(src + base + i * kThreads);
    const int64_t obase = (int64_t)blockIdx.x * kThreads * 2 + threadIdx.x;
    st16<NTS>(dst + obase, v[0] ^ v[1]);
    st16<NTS>(dst + obase + kThreads, v[2] ^ v[3]);
}

// One wave per (page, pool): a 4 KB page of K then the same page of V, 64 B
// per lane as four 16-byte loads 1 KB apart.  pages[] is a shuffled list of
// page indices into pools of n_pages pages each.
template <bool NT>
__global__ __launch_bounds__(kThreads) void page_read_kernel(const u32x4 *k, const u32x4 *v, const int32_t *pages,
                                                             int64_t n_list, int64_t pool_pages, uint32_t *sink) {
    const int64_t item = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    if (item >= 2 * n_list) return;
    const int lane = threadIdx.x & 63;
    const int64_t pg = pages[item >> 1];
    if (pg < 0 || pg >= pool_pages) return;
    const u32x4 *base = ((item & 1) ? v : k) + pg * 256 + lane;
    const u32x4 a = ld16<NT>(base), b = ld16<NT>(base + 64), c = ld16<NT>(base + 128), d = ld16<NT>(base + 192);
    const uint32_t x = fold(a, b, c, d);
    if (x == 0x9E3779B9u && lane == 7) sink[0] = x;
}

// 2 KB pages (the int8 decode's per-head run at block size 16): one wave per
// page, 32 B per lane.  GROUP = 1: pages[] lists 2 KB pages in a shuffled
// order; GROUP = 8: pages[] lists 16 KB blocks in a shuffled order and eight
// consecutive waves read the block's eight 2 KB pieces (as the decode's
// waves read the kv heads of one block).  HALF: each load instruction reads
// half of every 128-byte line it touches (lane (r, g) = (lane & 15, lane >> 4)
// reads row r's bytes 16 g and 64 + 16 g), as a 1-byte decode tile whose
// lane holds the MFMA operand layout directly would; else lane l reads bytes
// 16 l and 1024 + 16 l (whole lines per instruction).
template <bool NT, int GROUP, bool HALF = false>
__global__ __launch_bounds__(kThreads) void page_read2k_kernel(const u32x4 *k, const u32x4 *v, const int32_t *pages,
                                                               int64_t n_list, int64_t pool_pages2k, uint32_t *sink) {
    const int64_t item = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);   // (entry, piece, K|V)
    if (item >= 2 * GROUP * n_list) return;
    const int lane = threadIdx.x & 63;
    const int64_t e = item / (2 * GROUP);
    const int piece = (int)((item >> 1) % GROUP);
    const int64_t pg = (int64_t)pages[e] * GROUP + piece;          // 2 KB page index
    if (pg < 0 || pg >= pool_pages2k) return;
    const u32x4 *base = ((item & 1) ? v : k) + pg * 128 + (HALF ? (lane & 15) * 8 + (lane >> 4) : lane);
    const u32x4 a = ld16<NT>(base), b = ld16<NT>(base + (HALF ? 4 : 64));
    const uint32_t x = fold(a, b, a, b) ^ a[0];
    if (x == 0x9E3779B9u && lane == 7) sink[0] = x;
}

// The gather's pattern: 4 KB pages read in a shuffled order and written to
// consecutive 4 KB slots of an output, one wave per page (K pool pages to
// the first half of `out`, V pool pages to the second half).
template <bool NTL, bool NTS>
__global__ __launch_bounds__(kThreads) void page_copy_kernel(const u32x4 *k, const u32x4 *v, const int32_t *pages,
                                                             int64_t n_list, int64_t pool_pages, u32x4 *out) {
    const int64_t item = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    if (item >= 2 * n_list) return;
    const int lane = threadIdx.x & 63;
    const int64_t pg = pages[item >> 1];
    if (pg < 0 || pg >= pool_pages) return;
    const u32x4 *src = ((item & 1) ? v : k) + pg * 256 + lane;
    u32x4 *dst = out + ((item & 1) * n_list + (item >> 1)) * 256 + lane;
    u32x4 x[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = ld16<NTL>(src + 64 * i);
#pragma unroll
    for (int i = 0; i < 4; ++i) st16<NTS>(dst + 64 * i, x[i]);
}

// The append's pattern: 8 KB of contiguous rows read per 4 KB page written,
// the pages in a shuffled order, one wave per page (K pool pages from the
// first half of `src`'s rows, V from the second).
template <bool NTL, bool NTS>
__global__ __launch_bounds__(kThreads) void page_mix21_kernel(const u32x4 *src, u32x4 *k, u32x4 *v,
                                                              const int32_t *pages, int64_t n_list,
                                                              int64_t pool_pages) {
    const int64_t item = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    if (item >= 2 * n_list) return;
    const int lane = threadIdx.x & 63;
    const int64_t pg = pages[item >> 1];
    if (pg < 0 || pg >= pool_pages) return;
    const u32x4 *in = src + ((item & 1) * n_list + (item >> 1)) * 512 + lane;
    u32x4 *dst = ((item & 1) ? v : k) + pg * 256 + lane;
    u32x4 x[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = ld16<NTL>(in + 64 * i);
#pragma unroll
    for (int i = 0; i < 4; ++i) st16<NTS>(dst + 64 * i, x[2 * i] ^ x[2 * i + 1]);
}

// Persistent grid-stride forms of copy and mix21: a grid of 8 workgroups per
// CU, each thread keeping U 16-byte loads in flight (U = 8: 128 B, U = 16:
// 256 B) before its stores, the loads of one step a grid apart so each wave
// instruction still covers 1 KB of consecutive lines.
template <bool NTL, bool NTS, int U>
__global__ __launch_bounds__(kThreads) void copy_persist_kernel(const u32x4 *src, u32x4 *dst, int64_t n16) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t base = (int64_t)blockIdx.x * kThreads + threadIdx.x; base + (U - 1) * stride < n16;
         base += U * stride) {
        u32x4 v[U];
#pragma unroll
        for (int i = 0; i < U; ++i) v[i] = ld16<NTL>(src + base + i * stride);
#pragma unroll
        for (int i = 0; i < U; ++i) st16<NTS>(dst + base + i * stride, v[i]);
    }
}

// U loads in flight, U / 2 stores (two bytes read per byte written).
template <bool NTL, bool NTS, int U>
__global__ __launch_bounds__(kThreads) void mix21_persist_kernel(const u32x4 *src, u32x4 *dst, int64_t n16) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    int64_t obase = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    for (int64_t base = obase; base + (U - 1) * stride < n16; base += U * stride, obase += U / 2 * stride) {
        u32x4 v[U];
#pragma unroll
        for (int i = 0; i < U; ++i) v[i] = ld16<NTL>(src + base + i * stride);
#pragma unroll
        for (int i = 0; i < U / 2; ++i) st16<NTS>(dst + obase + i * stride, v[2 * i] ^ v[2 * i + 1]);
    }
}

// One-shot forms with other bytes per thread: U 16-byte loads a wave apart
// (U = 2: 32 B, 8: 128 B, 16: 256 B), then the thread's stores -- U for
// copy, U / 2 for mix21 -- or U stores alone (write).
template <bool NTL, bool NTS, int U, int MODE>   // MODE 0 copy, 1 mix21, 2 write
__global__ __launch_bounds__(kThreads) void wide_kernel(const u32x4 *src, u32x4 *dst, int64_t n16) {
    const int64_t base = (int64_t)blockIdx.x * kThreads * U + threadIdx.x;
    if (base + (U - 1) * kThreads >= n16) return;
    if constexpr (MODE == 2) {
        const u32x4 v = {0x5bd1e995u, (uint32_t)base, 7u, 11u};
#pragma unroll
        for (int i = 0; i < U; ++i) st16<NTS>(dst + base + i * kThreads, v);
        return;
    }
    u32x4 v[U];
#pragma unroll
    for (int i = 0; i < U; ++i) v[i] = ld16<NTL>(src + base + i * kThreads);
    if constexpr (MODE == 0) {
#pragma unroll
        for (int i = 0; i < U; ++i) st16<NTS>(dst + base + i * kThreads, v[i]);
    } else {
        const int64_t obase = (int64_t)blockIdx.x * kThreads * (U / 2) + threadIdx.x;
#pragma unroll
        for (int i = 0; i < U / 2; ++i) st16<NTS>(dst + obase + i * kThreads, v[2 * i] ^ v[2 * i + 1]);
    }
}

template <int U, int MODE>
void launch_wide(bool ntl, bool nts, hipStream_t s, const u32x4 *in, u32x4 *out, int64_t n16) {
    const dim3 g((unsigned)(n16 / (kThreads * U))), b(kThreads);
#define AIRKV_WIDE(L, S) hipLaunchKernelGGL((wide_kernel<L, S, U, MODE>), g, b, 0, s, in, out, n16)
    if (ntl && nts) AIRKV_WIDE(true, true);
    else if (ntl) AIRKV_WIDE(true, false);
    else if (nts) AIRKV_WIDE(false, true);
    else AIRKV_WIDE(false, false);
#undef AIRKV_WIDE
}

template <int U>
void launch_persist(bool mix, bool ntl, bool nts, dim3 g, dim3 b, hipStream_t s, const u32x4 *in, u32x4 *out,
                    int64_t n16) {
#define AIRKV_PERSIST(K, L, S) hipLaunchKernelGGL((K<L, S, U>), g, b, 0, s, in, out, n16)
    if (mix) {
        if (ntl && nts) AIRKV_PERSIST(mix21_persist_kernel, true, true);
        else if (ntl) AIRKV_PERSIST(mix21_persist_kernel, true, false);
        else if (nts) AIRKV_PERSIST(mix21_persist_kernel, false, true);
        else AIRKV_PERSIST(mix21_persist_kernel, false, false);
    } else {
        if (ntl && nts) AIRKV_PERSIST(copy_persist_kernel, true, true);
        else if (ntl) AIRKV_PERSIST(copy_persist_kernel, true, false);
        else if (nts) AIRKV_PERSIST(copy_persist_kernel, false, true);
        else AIRKV_PERSIST(copy_persist_kernel, false, false);
    }
#undef AIRKV_PERSIST
}

dim3 grid_for(int64_t n16) { return dim3((unsigned)(n16 / (kThreads * 4))); }

}  // namespace

extern "C" {

// kind: 0 read, 1 write, 2 copy, 3 mix21 (bytes = bytes read), 4 page_read
// (src = K pool, dst = V pool, bytes = one pool's bytes, pages / n_pages =
// the page list), 5 page_copy (as page_read, written to `sink`, which holds
// 2 * n_pages * 4 KB), 6 page_mix21 (src holds 2 * n_pages * 8 KB of rows,
// dst = K pool, sink = V pool), 7 / 8 persistent copy with 128 / 256 B in
// flight per thread, 9 / 10 persistent mix21 likewise, 11 / 12 / 13 one-shot
// copy with 32 / 128 / 256 B per thread, 14 one-shot mix21 with 128 B read
// per thread, 15 / 16 write with 32 / 128 B per thread, 17 page_read of
// 2 KB pages (pages: a shuffled list of the pools' 2 KB pages), 18 the same
// pages read eight at a time from shuffled 16 KB blocks (pages: a shuffled
// list of blocks), 19 kind 17 with each load instruction reading half of
// every line it touches.  nt_load / nt_store pick the non-temporal variants.
// Returns 0 or the hipError_t of the launch.
int air_ceiling_launch(int kind, int nt_load, int nt_store, const void *src, void *dst, int64_t bytes,
                       const int32_t *pages, int64_t n_pages, void *sink, void *stream) {
    hipStream_t s = (hipStream_t)stream;
    const int64_t n16 = bytes / 16;
    const u32x4 *in = (const u32x4 *)src;
    u32x4 *out = (u32x4 *)dst;
    uint32_t *sk = (uint32_t *)sink;
    if (n16 < kThreads * 4) return (int)hipErrorInvalidValue;
    const dim3 g = grid_for(n16), b(kThreads);
    switch (kind) {
    case 0:
        if (nt_load) hipLaunchKernelGGL(read_kernel<true>, g, b, 0, s, in, n16, sk);
        else hipLaunchKernelGGL(read_kernel<false>, g, b, 0, s, in, n16, sk);
        break;
    case 1:
        if (nt_store) hipLaunchKernelGGL(write_kernel<true>, g, b, 0, s, out, n16, 0x5bd1e995u);
        else hipLaunchKernelGGL(write_kernel<false>, g, b, 0, s, out, n16, 0x5bd1e995u);
        break;
    case 2:
        if (nt_load && nt_store) hipLaunchKernelGGL((copy_kernel<true, true>), g, b, 0, s, in, out, n16);
        else if (nt_load) hipLaunchKernelGGL((copy_kernel<true, false>), g, b, 0, s, in, out, n16);
        else if (nt_store) hipLaunchKernelGGL((copy_kernel<false, true>), g, b, 0, s, in, out, n16);
        else hipLaunchKernelGGL((copy_kernel<false, false>), g, b, 0, s, in, out, n16);
        break;
    case 3:
        if (nt_load && nt_store) hipLaunchKernelGGL((mix21_kernel<true, true>), g, b, 0, s, in, out, n16);
        else if (nt_load) hipLaunchKernelGGL((mix21_kernel<true, false>), g, b, 0, s, in, out, n16);
        else if (nt_store) hipLaunchKernelGGL((mix21_kernel<false, true>), g, b, 0, s, in, out, n16);
        else hipLaunchKernelGGL((mix21_kernel<false, false>), g, b, 0, s, in, out, n16);
        break;
    case 4: {
        if (!pages || n_pages <= 0 || n_pages * 4096 > bytes) return (int)hipErrorInvalidValue;
        const dim3 gp((unsigned)((2 * n_pages + kThreads / 64 - 1) / (kThreads / 64)));
        const int64_t pool_pages = bytes / 4096;
        if (nt_load)
            hipLaunchKernelGGL(page_read_kernel<true>, gp, b, 0, s, in, (const u32x4 *)dst, pages, n_pages, pool_pages, sk);
        else
            hipLaunchKernelGGL(page_read_kernel<false>, gp, b, 0, s, in, (const u32x4 *)dst, pages, n_pages, pool_pages, sk);
        break;
    }
    case 5: {
        // src = K pool, dst = V pool (bytes each), sink = output of 2 * n_pages * 4 KB
        if (!pages || n_pages <= 0 || n_pages * 4096 > bytes) return (int)hipErrorInvalidValue;
        const dim3 gp((unsigned)((2 * n_pages + kThreads / 64 - 1) / (kThreads / 64)));
        const int64_t pool_pages = bytes / 4096;
        u32x4 *o = (u32x4 *)sink;
        const u32x4 *vv = (const u32x4 *)dst;
        if (nt_load && nt_store)
            hipLaunchKernelGGL((page_copy_kernel<true, true>), gp, b, 0, s, in, vv, pages, n_pages, pool_pages, o);
        else if (nt_load)
            hipLaunchKernelGGL((page_copy_kernel<true, false>), gp, b, 0, s, in, vv, pages, n_pages, pool_pages, o);
        else if (nt_store)
            hipLaunchKernelGGL((page_copy_kernel<false, true>), gp, b, 0, s, in, vv, pages, n_pages, pool_pages, o);
        else
            hipLaunchKernelGGL((page_copy_kernel<false, false>), gp, b, 0, s, in, vv, pages, n_pages, pool_pages, o);
        break;
    }
    case 6: {
        // src = 2 * n_pages * 8 KB of rows, dst = K pool, sink = V pool (bytes each)
        if (!pages || n_pages <= 0 || n_pages * 4096 > bytes) return (int)hipErrorInvalidValue;
        const dim3 gp((unsigned)((2 * n_pages + kThreads / 64 - 1) / (kThreads / 64)));
        const int64_t pool_pages = bytes / 4096;
        u32x4 *vp = (u32x4 *)sink;
        if (nt_load && nt_store)
            hipLaunchKernelGGL((page_mix21_kernel<true, true>), gp, b, 0, s, in, out, vp, pages, n_pages, pool_pages);
        else if (nt_load)
            hipLaunchKernelGGL((page_mix21_kernel<true, false>), gp, b, 0, s, in, out, vp, pages, n_pages, pool_pages);
        else if (nt_store)
            hipLaunchKernelGGL((page_mix21_kernel<false, true>), gp, b, 0, s, in, out, vp, pages, n_pages, pool_pages);
        else
            hipLaunchKernelGGL((page_mix21_kernel<false, false>), gp, b, 0, s, in, out, vp, pages, n_pages, pool_pages);
        break;
    }
    case 7:    // copy, persistent, 128 B in flight per thread
    case 8:    // copy, persistent, 256 B
    case 9:    // mix21, persistent, 128 B (bytes = bytes read)
    case 10: { // mix21, persistent, 256 B
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            return (int)hipErrorInvalidValue;
        const dim3 gp((unsigned)(cus * 8));
        const bool mix = kind >= 9;
        if (kind == 7 || kind == 9) launch_persist<8>(mix, nt_load, nt_store, gp, b, s, in, out, n16);
        else launch_persist<16>(mix, nt_load, nt_store, gp, b, s, in, out, n16);
        break;
    }
    case 17:   // 2 KB pages (pages / n_pages: a shuffled list of 2 KB pages)
    case 18:   // 16 KB blocks (pages / n_pages: a shuffled list of blocks), 8 waves a block
    case 19: { // kind 17 with half of every line per load instruction
        const int grp = kind == 18 ? 8 : 1;
        if (!pages || n_pages <= 0 || n_pages * 2048 * grp > bytes) return (int)hipErrorInvalidValue;
        const dim3 gp((unsigned)((2 * grp * n_pages + kThreads / 64 - 1) / (kThreads / 64)));
        const int64_t pool2k = bytes / 2048;
        const u32x4 *vv = (const u32x4 *)dst;
        if (kind == 17) {
            if (nt_load) hipLaunchKernelGGL((page_read2k_kernel<true, 1>), gp, b, 0, s, in, vv, pages, n_pages, pool2k, sk);
            else hipLaunchKernelGGL((page_read2k_kernel<false, 1>), gp, b, 0, s, in, vv, pages, n_pages, pool2k, sk);
        } else if (kind == 19) {
            if (nt_load)
                hipLaunchKernelGGL((page_read2k_kernel<true, 1, true>), gp, b, 0, s, in, vv, pages, n_pages, pool2k, sk);
            else
                hipLaunchKernelGGL((page_read2k_kernel<false, 1, true>), gp, b, 0, s, in, vv, pages, n_pages, pool2k, sk);
        } else {
            if (nt_load) hipLaunchKernelGGL((page_read2k_kernel<true, 8>), gp, b, 0, s, in, vv, pages, n_pages, pool2k, sk);
            else hipLaunchKernelGGL((page_read2k_kernel<false, 8>), gp, b, 0, s, in, vv, pages, n_pages, pool2k, sk);
        }
        break;
    }
    case 11: launch_wide<2, 0>(nt_load, nt_store, s, in, out, n16); break;
    case 12: launch_wide<8, 0>(nt_load, nt_store, s, in, out, n16); break;
    case 13: launch_wide<16, 0>(nt_load, nt_store, s, in, out, n16); break;
    case 14: launch_wide<8, 1>(nt_load, nt_store, s, in, out, n16); break;
    case 15: launch_wide<2, 2>(nt_load, nt_store, s, in, out, n16); break;
    case 16: launch_wide<8, 2>(nt_load, nt_store, s, in, out, n16); break;
    default:
        return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

}  // extern "C"
