// Launch parameters of the paged prefill kernel.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace airkv {

struct PrefillArgs {
    const void *q;                 // [total_q][n_q_heads][head_dim], q_dtype
    int32_t q_dtype, n_q_heads;
    const int32_t *cu_q;           // [batch + 1] query row offsets
    const int32_t *tables, *lens;  // [batch][max_blocks], [batch]
    int32_t batch, max_blocks, total_q;
    int64_t max_len;               // max_blocks * block_size (set by launch_prefill)
    float scale_log2;              // softmax scale * log2(e)
    int32_t n_kv_heads, group, scale_group;
    int64_t num_blocks;
    const void *k_pages, *v_pages;
    const float *k_scales, *v_scales;
    void *out;                     // like q, out_dtype
    int32_t out_dtype;
    unsigned long long *errors;
    // launch shape (set by launch_prefill)
    int32_t nz;                    // slots per sequence
    int32_t ns_max;                // pieces a slot's keys may be cut into (1: no key split)
    int32_t slots;                 // resident workgroups of the launch: the balance target
    void *ws;                      // key-split workspace (ns_max > 1)
    int32_t ws_units;              // split slots the workspace holds
};

// Key-split workspace: a 64-byte header (int32 count of split slots), one
// int4 descriptor {sequence, slot, pieces, 0} per split slot, the launch
// plan (one int2 per grid row: item, slot info), padded to 256 bytes, then
// per (split slot, kv head, piece) the piece's partial output: [wave][16][lane]
// f32x4 accumulators, then [wave][lane] running maxima and [wave][lane] sums.
constexpr int64_t kPrefillPieceAccBytes = 4 * 16 * 64 * 16;
constexpr int64_t kPrefillPieceBytes = kPrefillPieceAccBytes + 2 * 256 * 4;
__host__ __device__ inline int64_t prefill_ws_header(int64_t units, int64_t rows) {
    return (64 + 16 * units + 8 * rows + 255) / 256 * 256;
}

struct PrefillPlan {
    int32_t nz, ns_max, units;     // units: split slots a full workspace holds
    int64_t ws_bytes;              // workspace that allows the key split (0: none needed)
};
PrefillPlan prefill_plan(int32_t batch, int32_t n_kv_heads, int32_t group, int32_t max_q_len, int cus);

bool prefill_supported(int dtype, int head_dim, int block_size, int scale_group);
// a.ws / a.ws_units: the workspace, or NULL / 0 for no key split
hipError_t launch_prefill(PrefillArgs a, int dtype, int block_size, int32_t max_q_len, int cus,
                          hipStream_t s);

}  // namespace airkv
