// Launch parameters of the warm-tier KV codec kernels (src/kv_compress.rs).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace airkv {

// Where the rows of a codec launch come from: a dense [n_rows][dim] array
// (ids == nullptr) or the K / V slabs of pool blocks, row r being row
// r % rows_per_block of block ids[r / rows_per_block].
struct RowSource {
    const void *base;
    const float *scales;       // quantized pools: per-group scales, else nullptr
    const int32_t *ids;        // device block ids, or nullptr
    int64_t rows_per_block;    // n_kv_heads * block_size
    int64_t num_blocks;
    int32_t scale_group;       // 0 for unquantized sources
};

enum class CompressKind { Key, Value, Qjl };

struct CompressArgs {
    RowSource src;
    int32_t src_dtype;         // AIR_KV_F32 / BF16 / INT8 / FP8
    int32_t dim;               // 32, 64 or 128
    int64_t n_rows;
    uint64_t *bits;            // key / qjl: [n_rows][ceil(bits / 64)]
    uint8_t *codes;            // value: [n_rows][dim]
    float *f0, *f1;            // key: magnitude, mean; value: scale, min; qjl: magnitude
    const float *proj;         // qjl: [proj_dim][dim]
    int32_t proj_dim;
    unsigned long long *errors;   // pool error counter (block sources) or nullptr
};

struct DecompressArgs {
    const uint64_t *bits;
    const uint8_t *codes;
    const float *f0, *f1;
    int64_t n_rows;
    int32_t dim;
    float *out;
};

constexpr int kMaxQjlProj = 512;

struct QjlScoreArgs {
    const uint64_t *key_bits;
    const float *key_magnitude;
    int64_t n_keys;
    int32_t proj_dim;
    const uint64_t *query_bits;
    float query_magnitude;
    float *cos_out, *dot_out;
    float cos_table[kMaxQjlProj + 1];   // cos(pi * h / proj_dim), h = 0 .. 64 * words
};

bool compress_dim_supported(int dim);
hipError_t launch_compress(CompressKind kind, const CompressArgs &a, int cus, hipStream_t s);
hipError_t launch_decompress(bool key, const DecompressArgs &a, int cus, hipStream_t s);
hipError_t launch_qjl_scores(const QjlScoreArgs &a, int cus, hipStream_t s);

}  // namespace airkv
