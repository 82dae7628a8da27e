/*
 * airkv_oracle.h -- CPU restatement of the reference's paged-KV algorithms.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  The
 * product library (libairkv.so) never links or calls it.
 *
 * Every function cites the reference (SunayHegde2006/Air.rs) file:line it
 * restates.  Layouts of the paged pool follow the build's device layout:
 *   k_pages / v_pages : [num_blocks][n_kv_heads][block_size][head_dim]
 *   k_scales/v_scales : [num_blocks][n_kv_heads][block_size][head_dim/group]
 *   slot = block * block_size + offset   (src/paged_attention.rs:216-234)
 */
#ifndef AIRKV_ORACLE_H
#define AIRKV_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* cache element types; values match include/air_kv.h */
enum { ORC_F32 = 0, ORC_BF16 = 1, ORC_INT8 = 2, ORC_FP8 = 3 };

/* ---- generators (reference test generators) ---------------------------- */
float orc_lcg_next(uint64_t *state);
void orc_lcg_fill(uint64_t seed, float *out, size_t n);
void orc_box_muller_fill(uint64_t seed, float *out, size_t n);

/* ---- scalar codecs ------------------------------------------------------ */
uint16_t orc_bf16_from_f32(float x);
float orc_bf16_to_f32(uint16_t b);
uint8_t orc_fp8_from_f32(float x);
float orc_fp8_to_f32(uint8_t b);
/* element-wise bulk forms of the three codecs above */
void orc_bf16_from_f32_n(const float *x, size_t n, uint16_t *out);
void orc_fp8_from_f32_n(const float *x, size_t n, uint8_t *out);
void orc_fp8_to_f32_n(const uint8_t *b, size_t n, float *out);

/* Q8_0 group quantizer (src/kv_cache.rs:54-75): n <= 32 elements. */
float orc_q8_quantize_group(const float *x, int n, int8_t *q);
/* Whole-buffer Q8Tensor::quantize: blocks of 32, n_blocks = ceil(n/32). */
void orc_q8_quantize(const float *x, size_t n, int8_t *q, float *scales);
void orc_q8_dequantize(const int8_t *q, const float *scales, size_t n, float *out);
/* FP8 per-group quantizer with the Fp8Layer scale rule (src/fp8.rs:228-238). */
float orc_fp8_quantize_group(const float *x, int n, uint8_t *q);
/* KvBlock::int8_quantize over a bf16 buffer (src/pd_disagg.rs:65-83). */
float orc_pd_int8_quantize(const uint16_t *bf16, size_t n, int8_t *q);
size_t orc_kvblock_serialise(uint32_t block_id, uint16_t layer_idx, const uint8_t *data, uint32_t n,
                             uint8_t *out);
int orc_kvblock_deserialise(const uint8_t *buf, size_t len, uint32_t *block_id, uint16_t *layer_idx,
                            uint32_t *data_len);
size_t orc_tcp_int8_payload(uint32_t block_id, uint16_t layer_idx, const uint16_t *bf16, size_t n,
                            uint8_t *out);

/* ---- paged pool operations (definitional) -------------------------------- */
/* Append n_tokens rows src[t][h][d] (f32) into the pool at slot_mapping[t].
 * Slots < 0 are skipped.  Returns the number of out-of-range slots. */
int orc_kv_append(int dtype, int block_size, int n_kv_heads, int head_dim, int group,
                  int64_t num_blocks, const float *k_src, const float *v_src,
                  const int64_t *slot_mapping, int n_tokens, void *k_pages,
                  void *v_pages, float *k_scales, float *v_scales);

/* Gather seq b to out + out_offsets[b] in layout 0 = [head][len][dim] or
 * 1 = [len][head][dim]; out_dtype ORC_F32 or ORC_BF16 (dequantized). */
int orc_kv_gather(int dtype, int block_size, int n_kv_heads, int head_dim, int group,
                  int64_t num_blocks, const void *k_pages, const void *v_pages,
                  const float *k_scales, const float *v_scales,
                  const int32_t *block_tables, const int32_t *seq_lens,
                  const int64_t *out_offsets, int batch, int max_blocks,
                  void *out_k, void *out_v, int out_dtype, int out_layout);

/* ---- flash decode (src/flash_decode.rs) ----------------------------------- */
void orc_chunk_attention(const float *q, const float *k_chunk, const float *v_chunk,
                         int chunk_len, int head_dim, float scale, float *out,
                         float *local_max, float *local_sum);
int orc_reduce_chunks(const float *outs, const float *maxes, const float *sums,
                      int n_chunks, int head_dim, float *out);
int orc_flash_decode(const float *q, const float *k, const float *v, int kv_len,
                     int head_dim, int chunk, float scale, float *out);
void orc_reference_attention(const float *q, const float *k, const float *v,
                             int kv_len, int head_dim, float scale, float *out);
void orc_reference_attention_f64(const float *q, const float *k, const float *v,
                                 int kv_len, int head_dim, double scale, double *out);

/* Paged decode: for every (seq, q head) gather the kv head h / group and
 * run orc_flash_decode over seq_lens[b] tokens.  q [batch][n_q][d] f32,
 * out [batch][n_q][d] f32.  Returns 0, or -1 on a bad table entry. */
int orc_paged_decode(int dtype, int block_size, int n_kv_heads, int head_dim, int group,
                     int64_t num_blocks, const void *k_pages, const void *v_pages,
                     const float *k_scales, const float *v_scales, const float *q,
                     int n_q_heads, const int32_t *block_tables, const int32_t *seq_lens,
                     int batch, int max_blocks, float scale, int chunk, float *out);

/* ---- kv_compress warm-tier codecs (src/kv_compress.rs) -------------------- */
void orc_key_compress(const float *key, size_t dim, uint64_t *bits, float *magnitude, float *mean);
void orc_key_decompress(const uint64_t *bits, float magnitude, float mean, size_t dim, float *out);
void orc_value_compress(const float *v, size_t dim, uint8_t *q, float *scale, float *min_val);
void orc_value_decompress(const uint8_t *q, float scale, float min_val, size_t dim, float *out);
void orc_qjl_projection_matrix(size_t proj_dim, size_t orig_dim, uint64_t seed, float *out);
void orc_qjl_compress(const float *key, size_t dim, const float *proj, size_t proj_dim,
                      uint64_t *bits, float *magnitude);
float orc_qjl_cos_sim(const uint64_t *a, const uint64_t *b, size_t proj_dim);

/* ---- blockwise causal attention (src/chunked_attn.rs) --------------------- */
void orc_blockwise_attention_head(const float *q, const float *k, const float *v, int seq_q,
                                  int seq_kv, int head_dim, float scale, int block_size,
                                  int causal, int q_offset, float *out);
int orc_paged_prefill(int dtype, int block_size, int n_kv_heads, int head_dim, int scale_group,
                      int group, int64_t num_blocks, const void *k_pages, const void *v_pages,
                      const float *k_scales, const float *v_scales, const float *q, int n_q_heads,
                      const int32_t *cu_q, const int32_t *block_tables, const int32_t *seq_lens,
                      int batch, int max_blocks, float scale, int kv_block, float *out);

#ifdef __cplusplus
}
#endif
#endif
