// extern "C" entry points for the device pool (air_kv.h, "Device side").
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>
#include <new>
#include <vector>

#include "host/status.hpp"
#include "kernels/prefill_common.hpp"
#include "pool.hpp"

using airkv::fail;

namespace {

int hip_fail(hipError_t e, const char *what) {
    return fail(AIR_KV_E_HIP, "%s: %s", what, hipGetErrorString(e));
}

bool pow2(int x) { return x > 0 && (x & (x - 1)) == 0; }

}  // namespace

extern "C" {

int air_kv_pool_create(const air_kv_pool_desc *desc, air_kv_pool **out) {
    if (!desc || !out) return fail(AIR_KV_E_INVALID_ARG, "desc or out is NULL");
    const air_kv_pool_desc d = *desc;
    if (d.num_blocks <= 0 || d.num_blocks > (int64_t)INT32_MAX)
        return fail(AIR_KV_E_INVALID_ARG, "num_blocks %lld out of range", (long long)d.num_blocks);
    if (d.block_size != 16 && d.block_size != 32)
        return fail(AIR_KV_E_INVALID_ARG, "block_size must be 16 or 32 (got %d)", d.block_size);
    if (d.n_kv_heads <= 0 || d.n_kv_heads > 256)
        return fail(AIR_KV_E_INVALID_ARG, "n_kv_heads %d out of range", d.n_kv_heads);
    if (d.head_dim <= 0 || d.head_dim % 32 || d.head_dim > 256)
        return fail(AIR_KV_E_INVALID_ARG, "head_dim must be a multiple of 32 up to 256 (got %d)", d.head_dim);
    if (d.dtype < AIR_KV_F32 || d.dtype > AIR_KV_FP8)
        return fail(AIR_KV_E_INVALID_ARG, "unknown dtype %d", d.dtype);
    if (airkv::dtype_quantized(d.dtype) &&
        (!pow2(d.scale_group) || d.scale_group < 8 || d.head_dim % d.scale_group))
        return fail(AIR_KV_E_INVALID_ARG,
                    "scale_group must be a power of two >= 8 dividing head_dim (got %d)", d.scale_group);

    auto *p = new (std::nothrow) air_kv_pool();
    if (!p) return fail(AIR_KV_E_OOM, "host allocation failed");
    p->desc = d;
    if (!airkv::dtype_quantized(d.dtype)) p->desc.scale_group = 0;
    p->elem_bytes = airkv::dtype_bytes(d.dtype);
    const size_t rows = (size_t)d.n_kv_heads * d.block_size;
    p->page_slab_bytes = rows * d.head_dim * p->elem_bytes;
    p->scale_slab_bytes = airkv::dtype_quantized(d.dtype) ? rows * (d.head_dim / d.scale_group) * 4 : 0;
    p->block_bytes = 2 * (p->page_slab_bytes + p->scale_slab_bytes);

    hipError_t e = hipGetDevice(&p->device);
    if (e != hipSuccess) { delete p; return hip_fail(e, "hipGetDevice"); }
    if (hipDeviceGetAttribute(&p->cus, hipDeviceAttributeMultiprocessorCount, p->device) != hipSuccess ||
        p->cus <= 0)
        p->cus = 256;
    const size_t pages = p->page_slab_bytes * (size_t)d.num_blocks;
    const size_t scales = p->scale_slab_bytes * (size_t)d.num_blocks;
    auto cleanup = [&](hipError_t err, const char *what) {
        (void)hipFree(p->k_pages); (void)hipFree(p->v_pages);
        (void)hipFree(p->k_scales); (void)hipFree(p->v_scales);
        (void)hipFree(p->errors);
        delete p;
        return err == hipErrorOutOfMemory ? fail(AIR_KV_E_OOM, "%s: out of device memory", what)
                                          : hip_fail(err, what);
    };
    if ((e = hipMalloc(&p->k_pages, pages)) != hipSuccess) return cleanup(e, "hipMalloc(k_pages)");
    if ((e = hipMalloc(&p->v_pages, pages)) != hipSuccess) return cleanup(e, "hipMalloc(v_pages)");
    if (scales) {
        if ((e = hipMalloc((void **)&p->k_scales, scales)) != hipSuccess) return cleanup(e, "hipMalloc(k_scales)");
        if ((e = hipMalloc((void **)&p->v_scales, scales)) != hipSuccess) return cleanup(e, "hipMalloc(v_scales)");
    }
    if ((e = hipMalloc((void **)&p->errors, sizeof(unsigned long long))) != hipSuccess)
        return cleanup(e, "hipMalloc(errors)");
    if ((e = hipMemset(p->k_pages, 0, pages)) != hipSuccess) return cleanup(e, "hipMemset");
    if ((e = hipMemset(p->v_pages, 0, pages)) != hipSuccess) return cleanup(e, "hipMemset");
    if (scales) {
        if ((e = hipMemset(p->k_scales, 0, scales)) != hipSuccess) return cleanup(e, "hipMemset");
        if ((e = hipMemset(p->v_scales, 0, scales)) != hipSuccess) return cleanup(e, "hipMemset");
    }
    if ((e = hipMemset(p->errors, 0, sizeof(unsigned long long))) != hipSuccess) return cleanup(e, "hipMemset");
    if ((e = hipDeviceSynchronize()) != hipSuccess) return cleanup(e, "hipDeviceSynchronize");
    *out = p;
    return AIR_KV_OK;
}

int air_kv_pool_destroy(air_kv_pool *p) {
    if (!p) return AIR_KV_OK;
    int dev_prev = 0;
    (void)hipGetDevice(&dev_prev);
    (void)hipSetDevice(p->device);
    (void)hipFree(p->k_pages); (void)hipFree(p->v_pages);
    (void)hipFree(p->k_scales); (void)hipFree(p->v_scales);
    (void)hipFree(p->errors);
    (void)hipFree(p->stage);
    (void)hipSetDevice(dev_prev);
    delete p;
    return AIR_KV_OK;
}

int air_kv_pool_info(const air_kv_pool *p, air_kv_pool_desc *desc, void **k_pages, void **v_pages,
                     void **k_scales, void **v_scales, size_t *block_bytes) {
    if (!p) return fail(AIR_KV_E_INVALID_ARG, "pool is NULL");
    if (desc) *desc = p->desc;
    if (k_pages) *k_pages = p->k_pages;
    if (v_pages) *v_pages = p->v_pages;
    if (k_scales) *k_scales = p->k_scales;
    if (v_scales) *v_scales = p->v_scales;
    if (block_bytes) *block_bytes = p->block_bytes;
    return AIR_KV_OK;
}

int air_kv_append(air_kv_pool *p, void *stream, const float *k, const float *v,
                  const int64_t *slot_mapping, int32_t n_tokens) {
    if (!p) return fail(AIR_KV_E_INVALID_ARG, "pool is NULL");
    if (n_tokens < 0) return fail(AIR_KV_E_INVALID_ARG, "n_tokens < 0");
    if (n_tokens == 0) return AIR_KV_OK;
    if (!k || !v || !slot_mapping) return fail(AIR_KV_E_INVALID_ARG, "k, v or slot_mapping is NULL");
    hipError_t e = airkv::launch_append(*p, (hipStream_t)stream, k, v, slot_mapping, n_tokens);
    return e == hipSuccess ? AIR_KV_OK : hip_fail(e, "air_kv_append launch");
}

int air_kv_gather(air_kv_pool *p, void *stream, const int32_t *block_tables, const int32_t *seq_lens,
                  const int64_t *out_offsets, int32_t batch, int32_t max_blocks, void *out_k,
                  void *out_v, int32_t out_dtype, int32_t out_layout) {
    if (!p) return fail(AIR_KV_E_INVALID_ARG, "pool is NULL");
    if (batch < 0 || max_blocks <= 0) return fail(AIR_KV_E_INVALID_ARG, "bad batch / max_blocks");
    if (batch == 0) return AIR_KV_OK;
    if (!block_tables || !seq_lens || !out_offsets || !out_k || !out_v)
        return fail(AIR_KV_E_INVALID_ARG, "NULL gather buffer");
    if (out_dtype != AIR_KV_F32 && out_dtype != AIR_KV_BF16)
        return fail(AIR_KV_E_INVALID_ARG, "gather out_dtype must be F32 or BF16");
    if (out_dtype == AIR_KV_BF16 && p->desc.dtype == AIR_KV_F32)
        return fail(AIR_KV_E_INVALID_ARG, "an F32 pool gathers to F32 only");
    if (out_layout != AIR_KV_LAYOUT_HEAD_MAJOR && out_layout != AIR_KV_LAYOUT_TOKEN_MAJOR)
        return fail(AIR_KV_E_INVALID_ARG, "unknown out_layout %d", out_layout);
    hipError_t e = airkv::launch_gather(*p, (hipStream_t)stream, block_tables, seq_lens, out_offsets,
                                        batch, max_blocks, out_k, out_v, out_dtype, out_layout);
    return e == hipSuccess ? AIR_KV_OK : hip_fail(e, "air_kv_gather launch");
}

int air_paged_decode_workspace_size(const air_kv_pool *p, int32_t n_q_heads, int32_t batch,
                                    int32_t max_blocks, int32_t max_splits, size_t *bytes) {
    if (!p || !bytes) return fail(AIR_KV_E_INVALID_ARG, "pool or bytes is NULL");
    airkv::DecodePlan plan;
    if (int rc = airkv::plan_decode(*p, n_q_heads, batch, max_blocks, max_splits, &plan)) return rc;
    *bytes = plan.ws_bytes;
    return AIR_KV_OK;
}

int air_paged_decode(air_kv_pool *p, void *stream, const void *q, int32_t q_dtype, int32_t n_q_heads,
                     const int32_t *block_tables, const int32_t *seq_lens, int32_t batch,
                     int32_t max_blocks, float scale, int32_t max_splits, void *workspace,
                     size_t ws_bytes, void *out, int32_t out_dtype) {
    if (!p) return fail(AIR_KV_E_INVALID_ARG, "pool is NULL");
    airkv::DecodePlan plan;
    if (int rc = airkv::plan_decode(*p, n_q_heads, batch, max_blocks, max_splits, &plan)) return rc;
    if (batch == 0) return AIR_KV_OK;
    if (!q || !block_tables || !seq_lens || !out || !workspace)
        return fail(AIR_KV_E_INVALID_ARG, "NULL decode buffer");
    if (ws_bytes < plan.ws_bytes)
        return fail(AIR_KV_E_INVALID_ARG, "workspace %zu bytes < %zu needed", ws_bytes, plan.ws_bytes);
    if (q_dtype != AIR_KV_F32 && q_dtype != AIR_KV_BF16)
        return fail(AIR_KV_E_INVALID_ARG, "q_dtype must be F32 or BF16");
    if (out_dtype != AIR_KV_F32 && out_dtype != AIR_KV_BF16)
        return fail(AIR_KV_E_INVALID_ARG, "out_dtype must be F32 or BF16");
    if (!(scale == scale)) return fail(AIR_KV_E_INVALID_ARG, "scale is NaN");
    hipError_t e = airkv::launch_decode(*p, (hipStream_t)stream, plan, q, q_dtype, n_q_heads,
                                        block_tables, seq_lens, batch, max_blocks, scale, workspace,
                                        out, out_dtype);
    return e == hipSuccess ? AIR_KV_OK : hip_fail(e, "air_paged_decode launch");
}

int air_paged_decode_append(air_kv_pool *p, void *stream, const void *q, int32_t q_dtype, int32_t n_q_heads,
                            const float *k_new, const float *v_new, const int32_t *block_tables,
                            const int32_t *seq_lens, int32_t batch, int32_t max_blocks, float scale,
                            int32_t max_splits, void *workspace, size_t ws_bytes, void *out,
                            int32_t out_dtype) {
    if (!p) return fail(AIR_KV_E_INVALID_ARG, "pool is NULL");
    airkv::DecodePlan plan;
    if (int rc = airkv::plan_decode(*p, n_q_heads, batch, max_blocks, max_splits, &plan)) return rc;
    if (batch == 0) return AIR_KV_OK;
    if (!q || !k_new || !v_new || !block_tables || !seq_lens || !out || !workspace)
        return fail(AIR_KV_E_INVALID_ARG, "NULL decode buffer");
    if ((uintptr_t)k_new % 16 || (uintptr_t)v_new % 16)   // read as 16-byte vectors
        return fail(AIR_KV_E_INVALID_ARG, "k_new and v_new must be 16-byte aligned");
    if (ws_bytes < plan.ws_bytes)
        return fail(AIR_KV_E_INVALID_ARG, "workspace %zu bytes < %zu needed", ws_bytes, plan.ws_bytes);
    if (q_dtype != AIR_KV_F32 && q_dtype != AIR_KV_BF16)
        return fail(AIR_KV_E_INVALID_ARG, "q_dtype must be F32 or BF16");
    if (out_dtype != AIR_KV_F32 && out_dtype != AIR_KV_BF16)
        return fail(AIR_KV_E_INVALID_ARG, "out_dtype must be F32 or BF16");
    if (!(scale == scale)) return fail(AIR_KV_E_INVALID_ARG, "scale is NaN");
    hipError_t e = airkv::launch_decode(*p, (hipStream_t)stream, plan, q, q_dtype, n_q_heads,
                                        block_tables, seq_lens, batch, max_blocks, scale, workspace,
                                        out, out_dtype, k_new, v_new);
    return e == hipSuccess ? AIR_KV_OK : hip_fail(e, "air_paged_decode_append launch");
}

int air_paged_prefill_workspace_size(const air_kv_pool *p, int32_t n_q_heads, int32_t batch,
                                     int32_t max_q_len, size_t *bytes) {
    if (!p || !bytes) return fail(AIR_KV_E_INVALID_ARG, "pool or bytes is NULL");
    if (n_q_heads <= 0 || n_q_heads % p->desc.n_kv_heads)
        return fail(AIR_KV_E_INVALID_ARG, "n_q_heads %d is not a multiple of n_kv_heads %d", n_q_heads,
                    p->desc.n_kv_heads);
    if (batch < 0 || max_q_len < 0) return fail(AIR_KV_E_INVALID_ARG, "negative batch or max_q_len");
    const air_kv_pool_desc &d = p->desc;
    if (batch == 0 || !airkv::prefill_supported(d.dtype, d.head_dim, d.block_size, d.scale_group)) {
        *bytes = 0;             // the vector prefill splits nothing
        return AIR_KV_OK;
    }
    const airkv::PrefillPlan pl =
        airkv::prefill_plan(batch, p->desc.n_kv_heads, n_q_heads / p->desc.n_kv_heads, max_q_len, p->cus);
    *bytes = (size_t)pl.ws_bytes;
    return AIR_KV_OK;
}

int air_paged_prefill(air_kv_pool *p, void *stream, const void *q, int32_t q_dtype, int32_t n_q_heads,
                      const int32_t *cu_q, int32_t total_q, int32_t max_q_len,
                      const int32_t *block_tables, const int32_t *seq_lens, int32_t batch,
                      int32_t max_blocks, float scale, void *workspace, size_t ws_bytes, void *out,
                      int32_t out_dtype) {
    if (!p) return fail(AIR_KV_E_INVALID_ARG, "pool is NULL");
    const air_kv_pool_desc &d = p->desc;
    if (n_q_heads <= 0 || n_q_heads % d.n_kv_heads)
        return fail(AIR_KV_E_INVALID_ARG, "n_q_heads %d is not a multiple of n_kv_heads %d", n_q_heads,
                    d.n_kv_heads);
    if (batch < 0 || total_q < 0 || max_q_len < 0 || max_blocks < 0)
        return fail(AIR_KV_E_INVALID_ARG, "negative batch, total_q, max_q_len or max_blocks");
    if (batch == 0 || total_q == 0) return AIR_KV_OK;
    if (!q || !cu_q || !block_tables || !seq_lens || !out)
        return fail(AIR_KV_E_INVALID_ARG, "NULL prefill buffer");
    if (q_dtype != AIR_KV_F32 && q_dtype != AIR_KV_BF16)
        return fail(AIR_KV_E_INVALID_ARG, "q_dtype must be F32 or BF16");
    if (out_dtype != AIR_KV_F32 && out_dtype != AIR_KV_BF16)
        return fail(AIR_KV_E_INVALID_ARG, "out_dtype must be F32 or BF16");
    if (!(scale > 0.0f && scale < INFINITY))
        return fail(AIR_KV_E_INVALID_ARG, "prefill scale must be finite and > 0");
    if ((int64_t)max_blocks * d.block_size > INT32_MAX)
        return fail(AIR_KV_E_INVALID_ARG, "max_blocks * block_size exceeds int32");
    if (!airkv::prefill_supported(d.dtype, d.head_dim, d.block_size, d.scale_group)) {
        // F32 pages, head_dim other than 128, small scale groups: the
        // vector kernel, one query row per workgroup and head chunk
        if (batch > 65535) return fail(AIR_KV_E_INVALID_ARG, "batch %d above 65535 for this pool", batch);
        hipError_t e = airkv::launch_prefill_rows(*p, (hipStream_t)stream, q, q_dtype, n_q_heads, cu_q, total_q,
                                                  max_q_len, block_tables, seq_lens, batch, max_blocks, scale,
                                                  out, out_dtype);
        return e == hipSuccess ? AIR_KV_OK : hip_fail(e, "air_paged_prefill launch");
    }
    airkv::PrefillArgs a;
    a.q = q; a.q_dtype = q_dtype; a.n_q_heads = n_q_heads;
    a.cu_q = cu_q; a.tables = block_tables; a.lens = seq_lens;
    a.batch = batch; a.max_blocks = max_blocks; a.total_q = total_q;
    a.scale_log2 = scale * 1.4426950408889634f;
    a.n_kv_heads = d.n_kv_heads; a.group = n_q_heads / d.n_kv_heads; a.scale_group = d.scale_group;
    a.num_blocks = d.num_blocks;
    a.k_pages = p->k_pages; a.v_pages = p->v_pages; a.k_scales = p->k_scales; a.v_scales = p->v_scales;
    a.out = out; a.out_dtype = out_dtype;
    a.errors = p->errors;
    a.ws = nullptr;
    a.ws_units = 0;
    const airkv::PrefillPlan pl =
        airkv::prefill_plan(batch, d.n_kv_heads, n_q_heads / d.n_kv_heads, max_q_len, p->cus);
    if (workspace && pl.ws_bytes > 0) {
        if (ws_bytes < (size_t)pl.ws_bytes)
            return fail(AIR_KV_E_INVALID_ARG, "prefill workspace of %zu bytes, %lld needed", ws_bytes,
                        (long long)pl.ws_bytes);
        if ((uintptr_t)workspace % 16) return fail(AIR_KV_E_INVALID_ARG, "prefill workspace must be 16-byte aligned");
        a.ws = workspace;
        a.ws_units = pl.units;
    }
    hipError_t e = airkv::launch_prefill(a, d.dtype, d.block_size, max_q_len, p->cus, (hipStream_t)stream);
    return e == hipSuccess ? AIR_KV_OK : hip_fail(e, "air_paged_prefill launch");
}

int air_kv_copy_blocks(air_kv_pool *p, void *stream, const int32_t *src, const int32_t *dst, int32_t n) {
    if (!p) return fail(AIR_KV_E_INVALID_ARG, "pool is NULL");
    if (n < 0) return fail(AIR_KV_E_INVALID_ARG, "n < 0");
    if (n == 0) return AIR_KV_OK;
    if (!src || !dst) return fail(AIR_KV_E_INVALID_ARG, "NULL block list");
    hipError_t e = airkv::launch_copy_blocks(*p, (hipStream_t)stream, src, dst, n);
    return e == hipSuccess ? AIR_KV_OK : hip_fail(e, "air_kv_copy_blocks launch");
}

int air_kv_block_wire_bytes(const air_kv_pool *p, size_t *bytes) {
    if (!p || !bytes) return fail(AIR_KV_E_INVALID_ARG, "pool or bytes is NULL");
    *bytes = airkv::wire_block_bytes(*p);
    return AIR_KV_OK;
}

int air_kv_pack_blocks(air_kv_pool *p, void *stream, const int32_t *ids, int32_t n, void *out) {
    if (!p) return fail(AIR_KV_E_INVALID_ARG, "pool is NULL");
    if (n < 0) return fail(AIR_KV_E_INVALID_ARG, "n < 0");
    if (n == 0) return AIR_KV_OK;
    if (!ids || !out) return fail(AIR_KV_E_INVALID_ARG, "NULL ids or out");
    hipError_t e = airkv::launch_pack_blocks(*p, (hipStream_t)stream, ids, n, out);
    return e == hipSuccess ? AIR_KV_OK : hip_fail(e, "air_kv_pack_blocks launch");
}

int air_kv_pack_blocks_int8(air_kv_pool *p, void *stream, const int32_t *ids, int32_t n,
                            int8_t *codes, float *scales) {
    if (!p) return fail(AIR_KV_E_INVALID_ARG, "pool is NULL");
    if (n < 0) return fail(AIR_KV_E_INVALID_ARG, "n < 0");
    if (n == 0) return AIR_KV_OK;
    if (!ids || !codes || !scales) return fail(AIR_KV_E_INVALID_ARG, "NULL ids, codes or scales");
    hipError_t e = airkv::launch_pack_blocks_int8(*p, (hipStream_t)stream, ids, n, codes, scales);
    return e == hipSuccess ? AIR_KV_OK : hip_fail(e, "air_kv_pack_blocks_int8 launch");
}

int air_kv_unpack_blocks(air_kv_pool *p, void *stream, const int32_t *ids, int32_t n, const void *in) {
    if (!p) return fail(AIR_KV_E_INVALID_ARG, "pool is NULL");
    if (n < 0) return fail(AIR_KV_E_INVALID_ARG, "n < 0");
    if (n == 0) return AIR_KV_OK;
    if (!ids || !in) return fail(AIR_KV_E_INVALID_ARG, "NULL ids or in");
    hipError_t e = airkv::launch_unpack_blocks(*p, (hipStream_t)stream, ids, n, in);
    return e == hipSuccess ? AIR_KV_OK : hip_fail(e, "air_kv_unpack_blocks launch");
}

int air_kv_wire_int8_quantize(void *stream, const void *wire, int32_t n_blocks, size_t elems_per_block,
                              int8_t *codes, float *scales) {
    if (n_blocks < 0) return fail(AIR_KV_E_INVALID_ARG, "n_blocks < 0");
    if (n_blocks == 0 || elems_per_block == 0) return AIR_KV_OK;
    if (!wire || !codes || !scales) return fail(AIR_KV_E_INVALID_ARG, "NULL wire, codes or scales");
    if (elems_per_block > (size_t)INT64_MAX / 2) return fail(AIR_KV_E_INVALID_ARG, "block too large");
    hipError_t e = airkv::launch_wire_int8((hipStream_t)stream, wire, n_blocks, (int64_t)elems_per_block,
                                           codes, scales);
    return e == hipSuccess ? AIR_KV_OK : hip_fail(e, "air_kv_wire_int8_quantize launch");
}

static int check_ids(const air_kv_pool *p, const int32_t *ids, int32_t n) {
    for (int32_t i = 0; i < n; ++i)
        if (ids[i] < 0 || ids[i] >= p->desc.num_blocks)
            return fail(AIR_KV_E_INVALID_ARG, "block id %d outside the pool", ids[i]);
    return AIR_KV_OK;
}

// Host swap copies.  Whole blocks move through a device staging buffer in
// the host layout (K slab, V slab, K scales, V scales per block), so each
// chunk of up to kStageBytes crosses PCIe as one transfer instead of one
// transfer per slab.  The staging is allocated on the first call and kept;
// if that allocation fails the slabs are copied one by one.
static constexpr size_t kStageBytes = (size_t)64 << 20;

static bool ensure_stage(air_kv_pool *p) {
    if (p->stage) return true;
    size_t nb = kStageBytes / p->block_bytes;
    if (nb < 1) nb = 1;
    void *mem = nullptr;
    if (hipMalloc(&mem, nb * p->block_bytes + nb * sizeof(int32_t)) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    p->stage = mem;
    p->stage_blocks = nb;
    return true;
}

// The slabs of block b, in the host layout.
static void block_slabs(const air_kv_pool *p, size_t b, uint8_t *ptrs[4], size_t sizes[4]) {
    ptrs[0] = (uint8_t *)p->k_pages + b * p->page_slab_bytes;
    ptrs[1] = (uint8_t *)p->v_pages + b * p->page_slab_bytes;
    ptrs[2] = p->k_scales ? (uint8_t *)p->k_scales + b * p->scale_slab_bytes : nullptr;
    ptrs[3] = p->v_scales ? (uint8_t *)p->v_scales + b * p->scale_slab_bytes : nullptr;
    sizes[0] = sizes[1] = p->page_slab_bytes;
    sizes[2] = sizes[3] = p->scale_slab_bytes;
}

static int move_blocks(air_kv_pool *p, hipStream_t s, const int32_t *ids, int32_t n, uint8_t *host,
                       bool to_host) {
    const size_t bb = p->block_bytes;
    if (ensure_stage(p)) {
        int32_t *dids = (int32_t *)((uint8_t *)p->stage + p->stage_blocks * bb);
        for (int32_t c0 = 0; c0 < n; c0 += (int32_t)p->stage_blocks) {
            const int32_t cn = n - c0 < (int32_t)p->stage_blocks ? n - c0 : (int32_t)p->stage_blocks;
            hipError_t e = hipMemcpyAsync(dids, ids + c0, cn * sizeof(int32_t), hipMemcpyHostToDevice, s);
            if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync(ids)");
            if (to_host) {
                if ((e = airkv::launch_stage_blocks(*p, s, dids, cn, p->stage, true)) != hipSuccess)
                    return hip_fail(e, "stage blocks");
                if ((e = hipMemcpyAsync(host + (size_t)c0 * bb, p->stage, cn * bb, hipMemcpyDeviceToHost, s)) !=
                    hipSuccess)
                    return hip_fail(e, "hipMemcpyAsync(D2H)");
            } else {
                if ((e = hipMemcpyAsync(p->stage, host + (size_t)c0 * bb, cn * bb, hipMemcpyHostToDevice, s)) !=
                    hipSuccess)
                    return hip_fail(e, "hipMemcpyAsync(H2D)");
                if ((e = airkv::launch_stage_blocks(*p, s, dids, cn, p->stage, false)) != hipSuccess)
                    return hip_fail(e, "unstage blocks");
            }
        }
    } else {
        for (int32_t i = 0; i < n; ++i) {
            uint8_t *ptrs[4];
            size_t sizes[4];
            block_slabs(p, (size_t)ids[i], ptrs, sizes);
            uint8_t *h = host + (size_t)i * bb;
            for (int j = 0; j < 4; ++j) {
                if (!sizes[j]) continue;
                hipError_t e = to_host ? hipMemcpyAsync(h, ptrs[j], sizes[j], hipMemcpyDeviceToHost, s)
                                       : hipMemcpyAsync(ptrs[j], h, sizes[j], hipMemcpyHostToDevice, s);
                if (e != hipSuccess) return hip_fail(e, to_host ? "hipMemcpyAsync(D2H)" : "hipMemcpyAsync(H2D)");
                h += sizes[j];
            }
        }
    }
    hipError_t e = hipStreamSynchronize(s);
    return e == hipSuccess ? AIR_KV_OK : hip_fail(e, "hipStreamSynchronize");
}

int air_kv_read_blocks(air_kv_pool *p, void *stream, const int32_t *ids, int32_t n, void *host_dst) {
    if (!p) return fail(AIR_KV_E_INVALID_ARG, "pool is NULL");
    if (n < 0 || (n > 0 && (!ids || !host_dst))) return fail(AIR_KV_E_INVALID_ARG, "bad block list");
    if (int rc = check_ids(p, ids, n)) return rc;
    if (n == 0) return AIR_KV_OK;
    return move_blocks(p, (hipStream_t)stream, ids, n, (uint8_t *)host_dst, true);
}

int air_kv_write_blocks(air_kv_pool *p, void *stream, const int32_t *ids, int32_t n, const void *host_src) {
    if (!p) return fail(AIR_KV_E_INVALID_ARG, "pool is NULL");
    if (n < 0 || (n > 0 && (!ids || !host_src))) return fail(AIR_KV_E_INVALID_ARG, "bad block list");
    if (int rc = check_ids(p, ids, n)) return rc;
    if (n == 0) return AIR_KV_OK;
    return move_blocks(p, (hipStream_t)stream, ids, n, (uint8_t *)const_cast<void *>(host_src), false);
}

int air_kv_pool_read_cb(void *ctx, uint32_t block, uint8_t *dst, size_t bytes) {
    air_kv_pool *p = (air_kv_pool *)ctx;
    if (!p) return fail(AIR_KV_E_INVALID_ARG, "read callback: pool is NULL");
    if (bytes != p->block_bytes)
        return fail(AIR_KV_E_INVALID_ARG, "read callback: %zu bytes asked, the pool's blocks hold %zu", bytes,
                    p->block_bytes);
    int32_t id = (int32_t)block;
    return air_kv_read_blocks(p, nullptr, &id, 1, dst);
}

int air_kv_pool_write_cb(void *ctx, uint32_t block, const uint8_t *src, size_t bytes) {
    air_kv_pool *p = (air_kv_pool *)ctx;
    if (!p) return fail(AIR_KV_E_INVALID_ARG, "write callback: pool is NULL");
    if (bytes != p->block_bytes)
        return fail(AIR_KV_E_INVALID_ARG, "write callback: %zu bytes given, the pool's blocks hold %zu", bytes,
                    p->block_bytes);
    int32_t id = (int32_t)block;
    return air_kv_write_blocks(p, nullptr, &id, 1, src);
}

int air_kv_pool_error_count(air_kv_pool *p, void *stream, int64_t *count, int32_t reset) {
    if (!p || !count) return fail(AIR_KV_E_INVALID_ARG, "pool or count is NULL");
    hipStream_t s = (hipStream_t)stream;
    unsigned long long v = 0;
    hipError_t e = hipMemcpyAsync(&v, p->errors, sizeof(v), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e == hipSuccess && reset) {
        e = hipMemsetAsync(p->errors, 0, sizeof(v), s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
    }
    if (e != hipSuccess) return hip_fail(e, "error counter read");
    *count = (int64_t)v;
    return AIR_KV_OK;
}

}  // extern "C"
