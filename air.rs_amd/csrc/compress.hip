// extern "C" entry points of the warm-tier KV codecs (air_kv.h,
// "kv_compress codecs").
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>

#include "host/status.hpp"
#include "kernels/compress_common.hpp"
#include "pool.hpp"

using airkv::fail;

namespace {

int hip_fail(hipError_t e, const char *what) {
    return fail(AIR_KV_E_HIP, "%s: %s", what, hipGetErrorString(e));
}

// Compute units of the current device (grid sizing of the row kernels).
int current_cus() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        return 256;
    return cus;
}

bool aligned(const void *p, size_t a) { return ((uintptr_t)p % a) == 0; }

int check_rows(const void *rows, int32_t dtype, int64_t n_rows, int32_t dim) {
    if (n_rows < 0) return fail(AIR_KV_E_INVALID_ARG, "n_rows < 0");
    if (!airkv::compress_dim_supported(dim))
        return fail(AIR_KV_E_INVALID_ARG, "dim %d not supported (32, 64 or 128)", dim);
    if (dtype != AIR_KV_F32 && dtype != AIR_KV_BF16)
        return fail(AIR_KV_E_INVALID_ARG, "rows_dtype must be F32 or BF16");
    if (n_rows > 0 && !rows) return fail(AIR_KV_E_INVALID_ARG, "rows is NULL");
    if (n_rows > 0 && !aligned(rows, 16)) return fail(AIR_KV_E_INVALID_ARG, "rows must be 16-byte aligned");
    return AIR_KV_OK;
}

airkv::RowSource dense(const void *rows) {
    airkv::RowSource s;
    s.base = rows;
    s.scales = nullptr;
    s.ids = nullptr;
    s.rows_per_block = 1;
    s.num_blocks = 0;
    s.scale_group = 0;
    return s;
}

airkv::RowSource pool_rows(const air_kv_pool &p, const int32_t *ids, bool values) {
    airkv::RowSource s;
    s.base = values ? p.v_pages : p.k_pages;
    s.scales = values ? p.v_scales : p.k_scales;
    s.ids = ids;
    s.rows_per_block = (int64_t)p.desc.n_kv_heads * p.desc.block_size;
    s.num_blocks = p.desc.num_blocks;
    s.scale_group = airkv::dtype_quantized(p.desc.dtype) ? p.desc.scale_group : 0;
    return s;
}

airkv::CompressArgs args(const airkv::RowSource &src, int32_t dtype, int32_t dim, int64_t n_rows) {
    airkv::CompressArgs a;
    std::memset(&a, 0, sizeof(a));
    a.src = src;
    a.src_dtype = dtype;
    a.dim = dim;
    a.n_rows = n_rows;
    return a;
}

int launch(airkv::CompressKind kind, const airkv::CompressArgs &a, int cus, void *stream,
           const char *what) {
    hipError_t e = airkv::launch_compress(kind, a, cus, (hipStream_t)stream);
    return e == hipSuccess ? AIR_KV_OK : hip_fail(e, what);
}

}  // namespace

extern "C" {

int air_kv_key_compress(void *stream, const void *rows, int32_t rows_dtype, int64_t n_rows, int32_t dim,
                        uint64_t *bits, float *magnitude, float *mean) {
    if (int rc = check_rows(rows, rows_dtype, n_rows, dim)) return rc;
    if (n_rows == 0) return AIR_KV_OK;
    if (!bits || !magnitude || !mean) return fail(AIR_KV_E_INVALID_ARG, "NULL output");
    airkv::CompressArgs a = args(dense(rows), rows_dtype, dim, n_rows);
    a.bits = bits;
    a.f0 = magnitude;
    a.f1 = mean;
    return launch(airkv::CompressKind::Key, a, current_cus(), stream, "air_kv_key_compress launch");
}

int air_kv_value_compress(void *stream, const void *rows, int32_t rows_dtype, int64_t n_rows,
                          int32_t dim, uint8_t *codes, float *scale, float *min_val) {
    if (int rc = check_rows(rows, rows_dtype, n_rows, dim)) return rc;
    if (n_rows == 0) return AIR_KV_OK;
    if (!codes || !scale || !min_val) return fail(AIR_KV_E_INVALID_ARG, "NULL output");
    if (!aligned(codes, 16)) return fail(AIR_KV_E_INVALID_ARG, "codes must be 16-byte aligned");
    airkv::CompressArgs a = args(dense(rows), rows_dtype, dim, n_rows);
    a.codes = codes;
    a.f0 = scale;
    a.f1 = min_val;
    return launch(airkv::CompressKind::Value, a, current_cus(), stream, "air_kv_value_compress launch");
}

static int check_proj(const float *proj, int32_t proj_dim) {
    if (proj_dim < 1 || proj_dim > airkv::kMaxQjlProj)
        return fail(AIR_KV_E_INVALID_ARG, "proj_dim %d outside 1..%d", proj_dim, airkv::kMaxQjlProj);
    if (!proj) return fail(AIR_KV_E_INVALID_ARG, "proj is NULL");
    return AIR_KV_OK;
}

int air_kv_qjl_compress(void *stream, const void *rows, int32_t rows_dtype, int64_t n_rows, int32_t dim,
                        const float *proj, int32_t proj_dim, uint64_t *bits, float *magnitude) {
    if (int rc = check_rows(rows, rows_dtype, n_rows, dim)) return rc;
    if (int rc = check_proj(proj, proj_dim)) return rc;
    if (n_rows == 0) return AIR_KV_OK;
    if (!bits || !magnitude) return fail(AIR_KV_E_INVALID_ARG, "NULL output");
    airkv::CompressArgs a = args(dense(rows), rows_dtype, dim, n_rows);
    a.bits = bits;
    a.f0 = magnitude;
    a.proj = proj;
    a.proj_dim = proj_dim;
    return launch(airkv::CompressKind::Qjl, a, current_cus(), stream, "air_kv_qjl_compress launch");
}

int air_kv_key_decompress(void *stream, const uint64_t *bits, const float *magnitude, const float *mean,
                          int64_t n_rows, int32_t dim, float *out) {
    if (n_rows < 0 || dim < 1) return fail(AIR_KV_E_INVALID_ARG, "n_rows < 0 or dim < 1");
    if (n_rows == 0) return AIR_KV_OK;
    if (!bits || !magnitude || !mean || !out) return fail(AIR_KV_E_INVALID_ARG, "NULL buffer");
    airkv::DecompressArgs a{bits, nullptr, magnitude, mean, n_rows, dim, out};
    hipError_t e = airkv::launch_decompress(true, a, current_cus(), (hipStream_t)stream);
    return e == hipSuccess ? AIR_KV_OK : hip_fail(e, "air_kv_key_decompress launch");
}

int air_kv_value_decompress(void *stream, const uint8_t *codes, const float *scale, const float *min_val,
                            int64_t n_rows, int32_t dim, float *out) {
    if (n_rows < 0 || dim < 1) return fail(AIR_KV_E_INVALID_ARG, "n_rows < 0 or dim < 1");
    if (n_rows == 0) return AIR_KV_OK;
    if (!codes || !scale || !min_val || !out) return fail(AIR_KV_E_INVALID_ARG, "NULL buffer");
    airkv::DecompressArgs a{nullptr, codes, scale, min_val, n_rows, dim, out};
    hipError_t e = airkv::launch_decompress(false, a, current_cus(), (hipStream_t)stream);
    return e == hipSuccess ? AIR_KV_OK : hip_fail(e, "air_kv_value_decompress launch");
}

int air_kv_qjl_scores(void *stream, const uint64_t *key_bits, const float *key_magnitude, int64_t n_keys,
                      int32_t proj_dim, const uint64_t *query_bits, float query_magnitude, float *cos_sim,
                      float *dot) {
    if (n_keys < 0) return fail(AIR_KV_E_INVALID_ARG, "n_keys < 0");
    if (proj_dim < 1 || proj_dim > airkv::kMaxQjlProj)
        return fail(AIR_KV_E_INVALID_ARG, "proj_dim %d outside 1..%d", proj_dim, airkv::kMaxQjlProj);
    if (n_keys == 0) return AIR_KV_OK;
    if (!key_bits || !query_bits || (!cos_sim && !dot) || (dot && !key_magnitude))
        return fail(AIR_KV_E_INVALID_ARG, "NULL buffer");
    airkv::QjlScoreArgs a;
    a.key_bits = key_bits;
    a.key_magnitude = key_magnitude;
    a.n_keys = n_keys;
    a.proj_dim = proj_dim;
    a.query_bits = query_bits;
    a.query_magnitude = query_magnitude;
    a.cos_out = cos_sim;
    a.dot_out = dot;
    // approx_cos_sim (src/kv_compress.rs:961-969): cos(PI * hamming / m),
    // the product taken before the division, evaluated here by the host's
    // libm for every distance the packed words can produce.
    const float pi = 3.14159265358979323846f;
    const int max_h = ((proj_dim + 63) / 64) * 64;
    for (int h = 0; h <= max_h; ++h) a.cos_table[h] = cosf(pi * (float)h / (float)proj_dim);
    hipError_t e = airkv::launch_qjl_scores(a, current_cus(), (hipStream_t)stream);
    return e == hipSuccess ? AIR_KV_OK : hip_fail(e, "air_kv_qjl_scores launch");
}

int air_kv_compress_blocks(air_kv_pool *p, void *stream, const int32_t *ids, int32_t n, uint64_t *key_bits,
                           float *key_magnitude, float *key_mean, uint8_t *value_codes, float *value_scale,
                           float *value_min) {
    if (!p) return fail(AIR_KV_E_INVALID_ARG, "pool is NULL");
    const int32_t dim = p->desc.head_dim;
    if (!airkv::compress_dim_supported(dim))
        return fail(AIR_KV_E_INVALID_ARG, "head_dim %d not supported (32, 64 or 128)", dim);
    if (n < 0) return fail(AIR_KV_E_INVALID_ARG, "n < 0");
    if (n == 0) return AIR_KV_OK;
    if (!ids || !key_bits || !key_magnitude || !key_mean || !value_codes || !value_scale || !value_min)
        return fail(AIR_KV_E_INVALID_ARG, "NULL buffer");
    if (!aligned(value_codes, 16)) return fail(AIR_KV_E_INVALID_ARG, "value_codes must be 16-byte aligned");
    const int64_t rows = (int64_t)n * p->desc.n_kv_heads * p->desc.block_size;
    airkv::CompressArgs k = args(pool_rows(*p, ids, false), p->desc.dtype, dim, rows);
    k.bits = key_bits;
    k.f0 = key_magnitude;
    k.f1 = key_mean;
    k.errors = p->errors;              // out-of-pool ids are counted once, by the key launch
    if (int rc = launch(airkv::CompressKind::Key, k, p->cus, stream, "air_kv_compress_blocks launch")) return rc;
    airkv::CompressArgs v = args(pool_rows(*p, ids, true), p->desc.dtype, dim, rows);
    v.codes = value_codes;
    v.f0 = value_scale;
    v.f1 = value_min;
    return launch(airkv::CompressKind::Value, v, p->cus, stream, "air_kv_compress_blocks launch");
}

int air_kv_qjl_compress_blocks(air_kv_pool *p, void *stream, const int32_t *ids, int32_t n, const float *proj,
                               int32_t proj_dim, uint64_t *bits, float *magnitude) {
    if (!p) return fail(AIR_KV_E_INVALID_ARG, "pool is NULL");
    const int32_t dim = p->desc.head_dim;
    if (!airkv::compress_dim_supported(dim))
        return fail(AIR_KV_E_INVALID_ARG, "head_dim %d not supported (32, 64 or 128)", dim);
    if (int rc = check_proj(proj, proj_dim)) return rc;
    if (n < 0) return fail(AIR_KV_E_INVALID_ARG, "n < 0");
    if (n == 0) return AIR_KV_OK;
    if (!ids || !bits || !magnitude) return fail(AIR_KV_E_INVALID_ARG, "NULL buffer");
    const int64_t rows = (int64_t)n * p->desc.n_kv_heads * p->desc.block_size;
    airkv::CompressArgs a = args(pool_rows(*p, ids, false), p->desc.dtype, dim, rows);
    a.bits = bits;
    a.f0 = magnitude;
    a.proj = proj;
    a.proj_dim = proj_dim;
    a.errors = p->errors;
    return launch(airkv::CompressKind::Qjl, a, p->cus, stream, "air_kv_qjl_compress_blocks launch");
}

}  // extern "C"
