// Whole-block copies inside a pool: the page copy that copy-on-write needs
// (BlockAllocator::cow_write only copies metadata, src/paged_attention.rs:160),
// and the moves between pages and a contiguous staging buffer that let the
// host swap copies (KvSwapManager's closures, src/kv_swap.rs:55-98) travel as
// one large transfer.  Each (block, tensor) slab is split over kSplit
// workgroups (16 KB each for the 32 KB slabs of a bs 16, 8-head, d 128 bf16
// pool: 5.09 against 5.00 TB/s with one workgroup per slab), and the grid
// holds scale slabs only for pools that have them; 16-byte non-temporal
// pieces, every load of a thread issued before its stores.
#include <hip/hip_runtime.h>

#include "../pool.hpp"

namespace airkv {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;   // 16-byte pieces in flight per thread: 16 KB per pass
constexpr int kSplit = 2;    // workgroups per slab

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// bytes (a multiple of 16) from in to out.  The loads of a pass are all
// issued before its stores: in and out are never proven disjoint, so a
// load-store loop would wait for each store before the next load.
__device__ __forceinline__ void move_slab(const uint8_t *in, uint8_t *out, uint64_t bytes) {
    const u32x4 *src = reinterpret_cast<const u32x4 *>(in);
    u32x4 *dst = reinterpret_cast<u32x4 *>(out);
    const uint64_t n16 = bytes / 16;
    for (uint64_t base = 0; base < n16; base += (uint64_t)kThreads * kUnroll) {
        u32x4 v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const uint64_t i = base + (uint64_t)u * kThreads + threadIdx.x;
            if (i < n16) v[u] = __builtin_nontemporal_load(src + i);
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const uint64_t i = base + (uint64_t)u * kThreads + threadIdx.x;
            if (i < n16) __builtin_nontemporal_store(v[u], dst + i);
        }
    }
}

struct CopyArgs {
    const int32_t *src, *dst;
    int64_t num_blocks;
    uint8_t *bases[4];       // k pages, v pages, k scales, v scales
    uint64_t slab_bytes[4];  // bytes of one block in each tensor (multiples of 16)
    unsigned long long *errors;
};

// Part `part` of kSplit of a slab: 16-byte pieces [part * n16 / kSplit, (part + 1) * n16 / kSplit).
__device__ __forceinline__ void move_part(const uint8_t *in, uint8_t *out, uint64_t bytes, int part) {
    const uint64_t n16 = bytes / 16, p0 = n16 * part / kSplit, p1 = n16 * (part + 1) / kSplit;
    move_slab(in + 16 * p0, out + 16 * p0, 16 * (p1 - p0));
}

__global__ __launch_bounds__(kThreads) void copy_blocks_kernel(CopyArgs a) {
    const int pair = blockIdx.x, which = blockIdx.y / kSplit, part = blockIdx.y % kSplit;
    const uint64_t bytes = a.slab_bytes[which];
    if (bytes == 0) return;
    const int32_t s = a.src[pair], d = a.dst[pair];
    if (s < 0 || d < 0 || s >= a.num_blocks || d >= a.num_blocks) {
        if (threadIdx.x == 0 && which == 0 && part == 0) atomicAdd(a.errors, 1ull);
        return;
    }
    move_part(a.bases[which] + (uint64_t)s * bytes, a.bases[which] + (uint64_t)d * bytes, bytes, part);
}

// Block i of the list <-> staging + i * block_bytes, laid out as the host
// buffers of air_kv_read_blocks / air_kv_write_blocks: K slab, V slab, K
// scales, V scales.  The ids were checked on the host.
struct StageArgs {
    const int32_t *ids;
    uint8_t *bases[4];
    uint64_t slab_bytes[4];
    uint8_t *staging;
    uint64_t block_bytes;
    int to_staging;
};

__global__ __launch_bounds__(kThreads) void stage_blocks_kernel(StageArgs a) {
    const int i = blockIdx.x, which = blockIdx.y / kSplit, part = blockIdx.y % kSplit;
    const uint64_t bytes = a.slab_bytes[which];
    if (bytes == 0) return;
    uint64_t off = 0;
    for (int j = 0; j < which; ++j) off += a.slab_bytes[j];
    uint8_t *st = a.staging + (uint64_t)i * a.block_bytes + off;
    uint8_t *pg = a.bases[which] + (uint64_t)a.ids[i] * bytes;
    if (a.to_staging) move_part(pg, st, bytes, part);
    else move_part(st, pg, bytes, part);
}

}  // namespace

hipError_t launch_copy_blocks(const air_kv_pool &p, hipStream_t s, const int32_t *src,
                              const int32_t *dst, int32_t n) {
    CopyArgs a;
    a.src = src; a.dst = dst; a.num_blocks = p.desc.num_blocks;
    a.bases[0] = (uint8_t *)p.k_pages; a.bases[1] = (uint8_t *)p.v_pages;
    a.bases[2] = (uint8_t *)p.k_scales; a.bases[3] = (uint8_t *)p.v_scales;
    a.slab_bytes[0] = a.slab_bytes[1] = p.page_slab_bytes;
    a.slab_bytes[2] = a.slab_bytes[3] = p.scale_slab_bytes;
    a.errors = p.errors;
    const unsigned slabs = p.scale_slab_bytes ? 4 : 2;
    hipLaunchKernelGGL(copy_blocks_kernel, dim3((unsigned)n, slabs * kSplit), dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_stage_blocks(const air_kv_pool &p, hipStream_t s, const int32_t *ids, int32_t n,
                               void *staging, bool to_staging) {
    if (n <= 0) return hipSuccess;
    StageArgs a;
    a.ids = ids;
    a.bases[0] = (uint8_t *)p.k_pages; a.bases[1] = (uint8_t *)p.v_pages;
    a.bases[2] = (uint8_t *)p.k_scales; a.bases[3] = (uint8_t *)p.v_scales;
    a.slab_bytes[0] = a.slab_bytes[1] = p.page_slab_bytes;
    a.slab_bytes[2] = a.slab_bytes[3] = p.scale_slab_bytes;
    a.staging = (uint8_t *)staging;
    a.block_bytes = p.block_bytes;
    a.to_staging = to_staging ? 1 : 0;
    const unsigned slabs = p.scale_slab_bytes ? 4 : 2;
    hipLaunchKernelGGL(stage_blocks_kernel, dim3((unsigned)n, slabs * kSplit), dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

}  // namespace airkv
