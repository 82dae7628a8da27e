// Shared launch parameters of the paged decode kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

struct air_kv_pool;

namespace airkv {

struct DecodePlan;

// Everything a decode kernel needs; built once per launch on the host.
struct DecodeArgs {
    const void *q;
    int32_t q_dtype, n_q_heads;
    const int32_t *tables, *lens;
    int32_t batch, max_blocks;
    int32_t part_tokens, num_parts;  // fixed partitions (vector kernel)
    int32_t slices, slots;           // balanced slices (matrix-core kernel)
    int32_t max_splits;              // pieces per sequence at most (matrix-core kernel)
    float scale_log2;              // softmax scale * log2(e): exp(x*s) == exp2(x*scale_log2)
    int32_t n_kv_heads, block_size, scale_group, group, head_dim;
    int64_t num_blocks;
    const void *k_pages, *v_pages;
    const float *k_scales, *v_scales;
    // Vector kernel: [batch][n_q][num_parts][head_dim] and [..][2].
    // Matrix-core kernel: [n_kv][slots][group][head_dim] and [..][2].
    float *part_o;                 // unnormalised partial outputs
    float *part_ml;                // running max (log2 units), sum
    int32_t *prefix;               // matrix-core kernel: tiles before each sequence, [batch + 1], then the chunk
    void *out;
    int32_t out_dtype;
    unsigned long long *errors;
    // Matrix-core kernel, bf16 pools: the decode step's new K / V rows,
    // [batch][n_kv_heads][head_dim] f32, written as each sequence's token
    // seq_lens[b] - 1 by the wave that computes that token's tile (NULL: none)
    const float *k_new, *v_new;
    // Vector kernel as a prefill (NULL: decode): sequence b's query rows
    // cu_q[b] .. cu_q[b + 1] - 1 of total_q, each attending causally,
    // num_parts row slots per sequence
    const int32_t *cu_q;
    int32_t total_q;
};

bool decode_mfma_supported(int dtype, int head_dim, int block_size, int group, int scale_group);
int plan_decode_mfma(const air_kv_pool &p, int32_t n_q_heads, int32_t batch, int32_t max_blocks,
                     int32_t max_splits, DecodePlan *plan);
hipError_t launch_decode_mfma(const DecodeArgs &a, const DecodePlan &plan, void *workspace,
                              hipStream_t s);

}  // namespace airkv
