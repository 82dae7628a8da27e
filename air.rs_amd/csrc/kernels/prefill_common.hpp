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
    float scale_log2;              // softmax scale * log2(e)
    int32_t n_kv_heads, group, scale_group;
    int64_t num_blocks;
    const void *k_pages, *v_pages;
    const float *k_scales, *v_scales;
    void *out;                     // like q, out_dtype
    int32_t out_dtype;
    unsigned long long *errors;
};

bool prefill_supported(int dtype, int head_dim, int block_size, int scale_group);
hipError_t launch_prefill(const PrefillArgs &a, int dtype, int block_size, int32_t max_q_len,
                          hipStream_t s);

}  // namespace airkv
