// Internal definition of the device pool and the kernel launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "air_kv.h"

struct air_kv_pool {
    air_kv_pool_desc desc;
    int device = 0;
    int cus = 256;               // compute units of that device (launch sizing)
    void *k_pages = nullptr;     // [num_blocks][n_kv_heads][block_size][head_dim]
    void *v_pages = nullptr;
    float *k_scales = nullptr;   // [num_blocks][n_kv_heads][block_size][head_dim/scale_group]
    float *v_scales = nullptr;
    unsigned long long *errors = nullptr;   // device counter of skipped bad slots / entries
    size_t elem_bytes = 0;
    size_t page_slab_bytes = 0;  // one block of K (or of V)
    size_t scale_slab_bytes = 0; // one block of K scales (or of V scales)
    size_t block_bytes = 0;      // K + V + scales of one block
    // Host swap copies: device staging of whole blocks (host layout) plus
    // their ids, allocated on first use and kept until the pool is destroyed.
    void *stage = nullptr;
    size_t stage_blocks = 0;     // blocks the staging holds
};

namespace airkv {

inline size_t dtype_bytes(int dt) { return dt == AIR_KV_F32 ? 4 : dt == AIR_KV_BF16 ? 2 : 1; }
inline bool dtype_quantized(int dt) { return dt == AIR_KV_INT8 || dt == AIR_KV_FP8; }

// Partitioning of one decode launch (shared by the workspace query).
struct DecodePlan {
    int32_t group;        // q heads per kv head
    int32_t dtype;        // page dtype of the pool
    bool mfma;            // matrix-core kernel with balanced slices (else fixed partitions)
    // fixed partitions (vector kernel)
    int32_t part_tokens;  // tokens per split-K partition (multiple of block_size)
    int32_t num_parts;    // partitions per sequence
    // balanced slices (matrix-core kernel)
    int32_t slices;       // slices per kv head (one wave each)
    int32_t slices_qf32;  // the same for f32 queries (their kernel may hold fewer waves per SIMD)
    int32_t slices_append;  // the same for the fused append + decode
    int32_t batch_per_launch;
    int32_t max_splits;   // pieces per sequence at most
    int32_t slots;        // partial rows per (kv head, q head of the group): slices + batch
    size_t ws_bytes;
};
int plan_decode(const air_kv_pool &pool, int32_t n_q_heads, int32_t batch, int32_t max_blocks,
                int32_t max_splits, DecodePlan *plan);

hipError_t launch_append(const air_kv_pool &pool, hipStream_t s, const float *k, const float *v,
                         const int64_t *slots, int32_t n_tokens);
hipError_t launch_gather(const air_kv_pool &pool, hipStream_t s, const int32_t *tables,
                         const int32_t *lens, const int64_t *out_offsets, int32_t batch,
                         int32_t max_blocks, void *out_k, void *out_v, int32_t out_dtype,
                         int32_t out_layout);
hipError_t launch_decode(const air_kv_pool &pool, hipStream_t s, const DecodePlan &plan,
                         const void *q, int32_t q_dtype, int32_t n_q_heads, const int32_t *tables,
                         const int32_t *lens, int32_t batch, int32_t max_blocks, float scale,
                         void *workspace, void *out, int32_t out_dtype,
                         const float *k_new = nullptr, const float *v_new = nullptr);
// Paged prefill on the vector decode kernel, for pools the matrix-core
// prefill does not take (arguments as air_paged_prefill's, validated).
hipError_t launch_prefill_rows(const air_kv_pool &pool, hipStream_t s, const void *q, int32_t q_dtype,
                               int32_t n_q_heads, const int32_t *cu_q, int32_t total_q, int32_t max_q_len,
                               const int32_t *tables, const int32_t *lens, int32_t batch, int32_t max_blocks,
                               float scale, void *out, int32_t out_dtype);
hipError_t launch_copy_blocks(const air_kv_pool &pool, hipStream_t s, const int32_t *src,
                              const int32_t *dst, int32_t n);
hipError_t launch_stage_blocks(const air_kv_pool &pool, hipStream_t s, const int32_t *ids, int32_t n,
                               void *staging, bool to_staging);
size_t wire_block_bytes(const air_kv_pool &pool);
hipError_t launch_pack_blocks(const air_kv_pool &pool, hipStream_t s, const int32_t *ids, int32_t n,
                              void *out);
hipError_t launch_pack_blocks_int8(const air_kv_pool &pool, hipStream_t s, const int32_t *ids,
                                   int32_t n, int8_t *codes, float *scales);
hipError_t launch_unpack_blocks(const air_kv_pool &pool, hipStream_t s, const int32_t *ids, int32_t n,
                                const void *in);
hipError_t launch_wire_int8(hipStream_t s, const void *wire, int32_t n_blocks, int64_t elems,
                            int8_t *codes, float *scales);

}  // namespace airkv
