// Shared launch parameters of the paged decode kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace airkv {

// Everything a decode kernel needs; built once per launch on the host.
struct DecodeArgs {
    const void *q;
    int32_t q_dtype, n_q_heads;
    const int32_t *tables, *lens;
    int32_t batch, max_blocks, part_tokens, num_parts;
    float scale_log2;              // softmax scale * log2(e): exp(x*s) == exp2(x*scale_log2)
    int32_t n_kv_heads, block_size, scale_group, group;
    int64_t num_blocks;
    const void *k_pages, *v_pages;
    const float *k_scales, *v_scales;
    float *part_o;                 // [batch][n_q][num_parts][head_dim] unnormalised partial outputs
    float *part_ml;                // [batch][n_q][num_parts][2]: running max (log2 units), sum
    void *out;
    int32_t out_dtype;
    unsigned long long *errors;
};

bool decode_mfma_supported(int dtype, int head_dim, int block_size, int group);
hipError_t launch_decode_mfma(const DecodeArgs &a, hipStream_t s, int dtype, int head_dim);

}  // namespace airkv
