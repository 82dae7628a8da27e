// Whole-block copies inside a pool: the page copy that copy-on-write needs
// (BlockAllocator::cow_write only copies metadata, src/paged_attention.rs:160).
// One workgroup per (pair, tensor); 16-byte vector copies.
#include <hip/hip_runtime.h>

#include "../pool.hpp"

namespace airkv {
namespace {

constexpr int kThreads = 256;

struct CopyArgs {
    const int32_t *src, *dst;
    int64_t num_blocks;
    uint8_t *bases[4];       // k pages, v pages, k scales, v scales
    uint64_t slab_bytes[4];  // bytes of one block in each tensor (multiples of 16)
    unsigned long long *errors;
};

__global__ __launch_bounds__(kThreads) void copy_blocks_kernel(CopyArgs a) {
    const int pair = blockIdx.x, which = blockIdx.y;
    const uint64_t bytes = a.slab_bytes[which];
    if (bytes == 0) return;
    const int32_t s = a.src[pair], d = a.dst[pair];
    if (s < 0 || d < 0 || s >= a.num_blocks || d >= a.num_blocks) {
        if (threadIdx.x == 0 && which == 0) atomicAdd(a.errors, 1ull);
        return;
    }
    const uint4 *in = reinterpret_cast<const uint4 *>(a.bases[which] + (uint64_t)s * bytes);
    uint4 *out = reinterpret_cast<uint4 *>(a.bases[which] + (uint64_t)d * bytes);
    for (uint64_t i = threadIdx.x; i < bytes / 16; i += kThreads) out[i] = in[i];
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
    hipLaunchKernelGGL(copy_blocks_kernel, dim3((unsigned)n, 4), dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

}  // namespace airkv
