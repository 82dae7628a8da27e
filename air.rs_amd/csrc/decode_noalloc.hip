// air_paged_decode_noalloc: the split-K paged decode with its workspace in a
// file-scope device array instead of caller memory, for callers that cannot
// allocate (code under HIP graph capture, tight serving loops, harnesses
// that forbid hipMalloc).  It runs the same plan and kernels as
// air_paged_decode; only the workspace pointer differs.
//
// `scratch` below is a device symbol: in host code its name is a host-side
// stand-in, not a device address.  The device address is looked up once per
// device with hipGetSymbolAddress (with that device current) and kept in
// g_scratch; only that pointer is ever handed to a kernel.  Each device holds
// its own copy of the array until the process ends.
#include <hip/hip_runtime.h>

#include <mutex>

#include "air_kv.h"
#include "host/status.hpp"
#include "pool.hpp"

using airkv::fail;

namespace {

constexpr size_t kScratchBytes = (size_t)AIR_KV_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

__device__ __align__(256) char scratch[kScratchBytes];

std::mutex g_mu;
void *g_scratch[kMaxDevices] = {};

int hip_fail(hipError_t e, const char *what) {
    return fail(AIR_KV_E_HIP, "%s: %s", what, hipGetErrorString(e));
}

// The device address of `scratch` on `device` (looked up on first use).
int scratch_on(int device, void **out) {
    if (device < 0 || device >= kMaxDevices) return fail(AIR_KV_E_INVALID_ARG, "device %d out of range", device);
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_scratch[device]) {
        int prev = 0;
        hipError_t e = hipGetDevice(&prev);
        if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
        if (prev != device && (e = hipSetDevice(device)) != hipSuccess) return hip_fail(e, "hipSetDevice");
        void *ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (prev != device) (void)hipSetDevice(prev);
        if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
        if (!ptr) return fail(AIR_KV_E_HIP, "hipGetSymbolAddress(scratch) gave NULL");
        g_scratch[device] = ptr;
    }
    *out = g_scratch[device];
    return AIR_KV_OK;
}

}  // namespace

extern "C" {

int air_paged_decode_noalloc(air_kv_pool *p, void *stream, const void *q, int32_t q_dtype,
                             int32_t n_q_heads, const int32_t *block_tables, const int32_t *seq_lens,
                             int32_t batch, int32_t max_blocks, float scale, int32_t max_splits, void *out,
                             int32_t out_dtype) {
    if (!p) return fail(AIR_KV_E_INVALID_ARG, "pool is NULL");
    airkv::DecodePlan plan;
    if (int rc = airkv::plan_decode(*p, n_q_heads, batch, max_blocks, max_splits, &plan)) return rc;
    if (plan.ws_bytes > kScratchBytes)
        return fail(AIR_KV_E_INVALID_ARG,
                    "air_paged_decode_noalloc: this launch needs %zu bytes of workspace, above the %zu-byte "
                    "scratch array (use air_paged_decode with a workspace)",
                    plan.ws_bytes, kScratchBytes);
    if (batch == 0) return AIR_KV_OK;
    void *ws = nullptr;
    if (int rc = scratch_on(p->device, &ws)) return rc;
    // The workspace needs no initialisation (every call rewrites what it
    // reads), so nothing is cleared here.
    return air_paged_decode(p, stream, q, q_dtype, n_q_heads, block_tables, seq_lens, batch, max_blocks, scale,
                            max_splits, ws, kScratchBytes, out, out_dtype);
}

}  // extern "C"
