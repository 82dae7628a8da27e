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
//
// Calls on one GPU share that GPU's array, so they are ordered: each call
// records an event on its stream after its launch, and a call on another
// stream first makes its stream wait for that event (calls on one stream
// are ordered by the stream itself).  The event is created with the
// symbol lookup, once per device; nothing is allocated per call.
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

std::mutex g_mu;                       // guards the per-device state and orders the launches
void *g_scratch[kMaxDevices] = {};
hipEvent_t g_done[kMaxDevices] = {};   // recorded after the device's latest call
hipStream_t g_last[kMaxDevices] = {};  // the stream of that call
bool g_any[kMaxDevices] = {};          // a call has been recorded

int hip_fail(hipError_t e, const char *what) {
    return fail(AIR_KV_E_HIP, "%s: %s", what, hipGetErrorString(e));
}

// The device address of `scratch` on `device` and the device's ordering
// event (set up on first use).  The caller holds g_mu.
int scratch_on(int device, void **out) {
    if (device < 0 || device >= kMaxDevices) return fail(AIR_KV_E_INVALID_ARG, "device %d out of range", device);
    if (!g_scratch[device]) {
        int prev = 0;
        hipError_t e = hipGetDevice(&prev);
        if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
        if (prev != device && (e = hipSetDevice(device)) != hipSuccess) return hip_fail(e, "hipSetDevice");
        void *ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        hipEvent_t ev = nullptr;
        if (e == hipSuccess) e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
        if (prev != device) (void)hipSetDevice(prev);
        if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch) / hipEventCreate");
        if (!ptr) return fail(AIR_KV_E_HIP, "hipGetSymbolAddress(scratch) gave NULL");
        g_done[device] = ev;
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
    const int dev = p->device;
    std::lock_guard<std::mutex> lock(g_mu);
    void *ws = nullptr;
    if (int rc = scratch_on(dev, &ws)) return rc;
    hipStream_t s = (hipStream_t)stream;
    // a call on another stream than the device's latest waits for that call
    if (g_any[dev] && g_last[dev] != s) {
        hipError_t e = hipStreamWaitEvent(s, g_done[dev], 0);
        if (e != hipSuccess) return hip_fail(e, "hipStreamWaitEvent (ordering after the previous no-alloc call)");
    }
    // The workspace needs no initialisation (every call rewrites what it
    // reads), so nothing is cleared here.
    const int rc = air_paged_decode(p, stream, q, q_dtype, n_q_heads, block_tables, seq_lens, batch, max_blocks,
                                    scale, max_splits, ws, kScratchBytes, out, out_dtype);
    if (rc != AIR_KV_OK) return rc;
    hipError_t e = hipEventRecord(g_done[dev], s);
    if (e != hipSuccess) return hip_fail(e, "hipEventRecord (after the no-alloc call)");
    g_last[dev] = s;
    g_any[dev] = true;
    return AIR_KV_OK;
}

}  // extern "C"
