/*
 * airkv_oracle.c -- CPU restatement of the reference's paged-KV algorithms.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product).  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 *
 * Built with gcc -O2 -ffp-contract=off so that every f32 operation rounds
 * exactly once, as Rust's f32 arithmetic does (Rust never contracts a*b+c).
 * Rust scalar facts relied upon (language spec): f32::round rounds half away
 * from zero (C roundf); `x as i8` saturates and maps NaN to 0; f32::max
 * returns the other operand when one is NaN, signalling NaNs included
 * (rust_max below; glibc fmaxf instead returns NaN for a signalling NaN);
 * `u32::MAX as f32` is 4294967296.0f.
 *
 * Parity status of each function is recorded in its header comment; the
 * checks live in tests/test_oracle_*.py.
 */
#include "airkv_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static inline uint32_t f2u(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }

/* Rust f32::max: "If one of the arguments is NaN, then the other argument is
 * returned", for quiet and signalling NaNs alike. */
static inline float rust_max(float a, float b) {
    if (isnan(a)) return b;
    if (isnan(b)) return a;
    return a > b ? a : b;
}
static inline float u2f(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

/* ------------------------------------------------------------------------ */
/* Generators                                                               */
/* ------------------------------------------------------------------------ */

/* Uniform in [-1, 1): src/flash_decode.rs:220-223 (test `lcg`). */
float orc_lcg_next(uint64_t *state) {
    *state = *state * 6364136223846793005ULL + 1442695040888963407ULL;
    float num = (float)(*state >> 33);
    const float den = (float)4294967295u; /* u32::MAX as f32 == 2^32 */
    return num / den * 2.0f - 1.0f;
}

/* src/flash_decode.rs:225-228 (test `randn`, which is uniform despite its name) */
void orc_lcg_fill(uint64_t seed, float *out, size_t n) {
    uint64_t s = seed;
    for (size_t i = 0; i < n; ++i) out[i] = orc_lcg_next(&s);
}

/* Box-Muller normals on the same LCG: src/kv_compress.rs:989-1015 with
 * orig_dim = 1 (scale 1).  libm log/cos/sin may differ across hosts in the
 * last bit; inputs are generated once and handed to both CPU and GPU. */
void orc_box_muller_fill(uint64_t seed, float *out, size_t n) {
    uint64_t state = seed + 1;
    const float two53 = 9007199254740992.0f;
    size_t i = 0;
    while (i < n) {
        state = state * 6364136223846793005ULL + 1442695040888963407ULL;
        float u1 = (float)(state >> 11) / two53;
        state = state * 6364136223846793005ULL + 1442695040888963407ULL;
        float u2 = (float)(state >> 11) / two53;
        u1 = rust_max(u1, 1e-10f);
        float r = sqrtf(-2.0f * logf(u1));
        float theta = 2.0f * 3.14159265358979323846f * u2;
        out[i++] = r * cosf(theta);
        if (i < n) out[i++] = r * sinf(theta);
    }
}

/* ------------------------------------------------------------------------ */
/* Scalar codecs                                                            */
/* ------------------------------------------------------------------------ */

/* half 2.7.1 `bf16::from_f32` (dependency of the reference, Cargo.lock:1651-
 * 1654; called at src/pd_disagg.rs:66-69 and by candle to_dtype at
 * src/kv_cache.rs:275-276): NaN keeps its high half with the quiet bit set;
 * otherwise round to nearest, ties to even. */
uint16_t orc_bf16_from_f32(float x) {
    uint32_t u = f2u(x);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x0040u);
    uint32_t round_bit = 0x8000u;
    if ((u & round_bit) && (u & (3u * round_bit - 1u))) return (uint16_t)((u >> 16) + 1u);
    return (uint16_t)(u >> 16);
}

float orc_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

/* F8E4M3::from_f32, src/fp8.rs:54-91.  Quirks kept: -0.0 -> 0x00 (sign is
 * `x < 0.0`); |x| >= 256 saturates to 0x7E/0xFE because an exponent field of
 * 15 is treated as overflow (:79-82); the mantissa rounds half-up on the
 * magnitude and is capped at 0b111 without carrying into the exponent
 * (:85-86); subnormal results flush to signed zero (:75-78). */
uint8_t orc_fp8_from_f32(float x) {
    if (isnan(x)) return 0x7F;
    uint8_t sign = x < 0.0f ? 1 : 0;
    float a = fabsf(x);
    if (a == 0.0f) return (uint8_t)(sign << 7);
    if (a >= 448.0f) return (uint8_t)((sign << 7) | 0x7E);
    uint32_t bits = f2u(a);
    int exp32 = (int)((bits >> 23) & 0xFF);
    uint32_t mant32 = bits & 0x007FFFFFu;
    int exp8 = exp32 - 127 + 7;
    if (exp8 <= 0) return (uint8_t)(sign << 7);
    if (exp8 >= 15) return (uint8_t)((sign << 7) | 0x7E);
    uint32_t mant3 = (mant32 + (1u << 19)) >> 20;
    if (mant3 > 7u) mant3 = 7u;
    return (uint8_t)((sign << 7) | ((uint32_t)exp8 << 3) | mant3);
}

/* F8E4M3::to_f32, src/fp8.rs:94-112.  0x7F is the only NaN; 0xFF decodes to
 * -480; an exponent field of 0 decodes to +0.0 regardless of sign. */
float orc_fp8_to_f32(uint8_t b) {
    if (b == 0x7F) return NAN;
    float sign = (b >> 7) == 1 ? -1.0f : 1.0f;
    int exp8 = (b >> 3) & 0xF;
    int mant3 = b & 0x7;
    if (exp8 == 0) return 0.0f;
    float mantissa = 1.0f + (float)mant3 / 8.0f;
    return sign * ldexpf(1.0f, exp8 - 7) * mantissa;
}

void orc_bf16_from_f32_n(const float *x, size_t n, uint16_t *out) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_bf16_from_f32(x[i]);
}

void orc_fp8_from_f32_n(const float *x, size_t n, uint8_t *out) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_fp8_from_f32(x[i]);
}

void orc_fp8_to_f32_n(const uint8_t *b, size_t n, float *out) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_fp8_to_f32(b[i]);
}

/* Saturating Rust `as i8` of an already-rounded value; NaN -> 0. */
static inline int8_t rust_as_i8(float r) {
    if (isnan(r)) return 0;
    if (r <= -128.0f) return -128;
    if (r >= 127.0f) return 127;
    return (int8_t)r;
}

/* One Q8_0 block, src/kv_cache.rs:59-72: absmax fold from 0.0 with
 * f32::max; scale = absmax == 0 ? 1 : absmax / 127; inv = 1 / scale;
 * q = clamp(round(x * inv), -127, 127) as i8 (clamp keeps NaN, cast -> 0). */
float orc_q8_quantize_group(const float *x, int n, int8_t *q) {
    float max_abs = 0.0f;
    for (int i = 0; i < n; ++i) max_abs = rust_max(max_abs, fabsf(x[i]));
    float scale = (max_abs == 0.0f) ? 1.0f : max_abs / 127.0f;
    float inv = 1.0f / scale;
    for (int i = 0; i < n; ++i) {
        float r = roundf(x[i] * inv);
        if (!isnan(r)) r = r < -127.0f ? -127.0f : (r > 127.0f ? 127.0f : r);
        q[i] = rust_as_i8(r);
    }
    return scale;
}

/* Q8Tensor::quantize, src/kv_cache.rs:54-75 (chunks of 32, last may be short). */
void orc_q8_quantize(const float *x, size_t n, int8_t *q, float *scales) {
    size_t nb = (n + 31) / 32;
    for (size_t b = 0; b < nb; ++b) {
        size_t s = b * 32, cnt = (n - s) < 32 ? (n - s) : 32;
        scales[b] = orc_q8_quantize_group(x + s, (int)cnt, q + s);
    }
}

/* Q8Tensor::dequantize, src/kv_cache.rs:78-92: quant as f32 * scale. */
void orc_q8_dequantize(const int8_t *q, const float *scales, size_t n, float *out) {
    for (size_t i = 0; i < n; ++i) out[i] = (float)q[i] * scales[i / 32];
}

/* Fp8Layer::from_f32_weight scale rule, src/fp8.rs:228-238, applied to one
 * group: absmax fold from 0.0; scale = absmax < 1e-8 ? 1 : absmax / 448;
 * code = F8E4M3::from_f32(x / scale) (a true division, :237). */
float orc_fp8_quantize_group(const float *x, int n, uint8_t *q) {
    float max_abs = 0.0f;
    for (int i = 0; i < n; ++i) max_abs = rust_max(max_abs, fabsf(x[i]));
    float scale = (max_abs < 1e-8f) ? 1.0f : max_abs / 448.0f;
    for (int i = 0; i < n; ++i) q[i] = orc_fp8_from_f32(x[i] / scale);
    return scale;
}

/* KvBlock::int8_quantize, src/pd_disagg.rs:65-83: one scale over the whole
 * bf16 buffer, no clamp, saturating `as i8`. */
float orc_pd_int8_quantize(const uint16_t *bf16, size_t n, int8_t *q) {
    float max_val = 0.0f;
    for (size_t i = 0; i < n; ++i) max_val = rust_max(max_val, fabsf(orc_bf16_to_f32(bf16[i])));
    float scale = max_val > 0.0f ? max_val / 127.0f : 1.0f;
    float inv = 1.0f / scale;
    for (size_t i = 0; i < n; ++i) q[i] = rust_as_i8(roundf(orc_bf16_to_f32(bf16[i]) * inv));
    return scale;
}

/* KvBlock::serialise, src/pd_disagg.rs:52-62: block_id.to_le_bytes(),
 * layer_idx.to_le_bytes(), (data.len() as u32).to_le_bytes(), data.  The
 * bytes are assembled one at a time from the integers (no host byte-order
 * assumption).  Returns the frame length. */
size_t orc_kvblock_serialise(uint32_t block_id, uint16_t layer_idx, const uint8_t *data, uint32_t n,
                             uint8_t *out) {
    size_t o = 0;
    for (int i = 0; i < 4; ++i) out[o++] = (uint8_t)(block_id >> (8 * i));
    for (int i = 0; i < 2; ++i) out[o++] = (uint8_t)(layer_idx >> (8 * i));
    for (int i = 0; i < 4; ++i) out[o++] = (uint8_t)(n >> (8 * i));
    for (uint32_t i = 0; i < n; ++i) out[o++] = data[i];
    return o;
}

/* KvBlock::deserialise, src/pd_disagg.rs:85-104: None (returns 0) when the
 * buffer is shorter than 10 bytes or than 10 + data_len; else 1, with the
 * fields and the data offset (10). */
int orc_kvblock_deserialise(const uint8_t *buf, size_t len, uint32_t *block_id, uint16_t *layer_idx,
                            uint32_t *data_len) {
    if (len < 10) return 0;
    uint32_t id = 0, n = 0;
    for (int i = 0; i < 4; ++i) id |= (uint32_t)buf[i] << (8 * i);
    const uint16_t layer = (uint16_t)(buf[4] | (buf[5] << 8));
    for (int i = 0; i < 4; ++i) n |= (uint32_t)buf[6 + i] << (8 * i);
    if (len < 10 + (size_t)n) return 0;
    *block_id = id;
    *layer_idx = layer;
    *data_len = n;
    return 1;
}

/* The int8 payload of TcpKvConnector::send_blocks, src/pd_disagg.rs:267-276:
 * KvBlock::int8_quantize of the block's bf16 data, then block_id, layer_idx,
 * scale (f32 bits), (q.len() as u32), the codes as bytes.  Returns the
 * payload length. */
size_t orc_tcp_int8_payload(uint32_t block_id, uint16_t layer_idx, const uint16_t *bf16, size_t n,
                            uint8_t *out) {
    int8_t *q = (int8_t *)(out + 14);
    const float scale = orc_pd_int8_quantize(bf16, n, q);
    uint32_t sbits;
    memcpy(&sbits, &scale, 4);
    size_t o = 0;
    for (int i = 0; i < 4; ++i) out[o++] = (uint8_t)(block_id >> (8 * i));
    for (int i = 0; i < 2; ++i) out[o++] = (uint8_t)(layer_idx >> (8 * i));
    for (int i = 0; i < 4; ++i) out[o++] = (uint8_t)(sbits >> (8 * i));
    for (int i = 0; i < 4; ++i) out[o++] = (uint8_t)((uint32_t)n >> (8 * i));
    return o + n;
}

/* ------------------------------------------------------------------------ */
/* Paged pool: append and gather                                            */
/* ------------------------------------------------------------------------ */

static size_t elem_bytes(int dtype) {
    switch (dtype) {
    case ORC_F32: return 4;
    case ORC_BF16: return 2;
    default: return 1;
    }
}

/* Definitional append (reshape-and-cache).  The reference appends with
 * Tensor::cat (src/model.rs:569) and stores through save_layer
 * (src/kv_cache.rs:286-339); the paged form writes row (t, h) to
 * page[slot / bs][h][slot % bs][:], the slot arithmetic of
 * src/paged_attention.rs:216-234.  int8 rows are Q8_0 blocks of `group`
 * elements (src/kv_cache.rs:54-75); fp8 rows use the Fp8Layer scale rule. */
int orc_kv_append(int dtype, int block_size, int n_kv_heads, int head_dim, int group,
                  int64_t num_blocks, const float *k_src, const float *v_src,
                  const int64_t *slot_mapping, int n_tokens, void *k_pages,
                  void *v_pages, float *k_scales, float *v_scales) {
    int bad = 0;
    size_t eb = elem_bytes(dtype);
    int ng = (dtype == ORC_INT8 || dtype == ORC_FP8) ? head_dim / group : 0;
    for (int t = 0; t < n_tokens; ++t) {
        int64_t slot = slot_mapping[t];
        if (slot < 0) continue;
        if (slot >= num_blocks * (int64_t)block_size) { ++bad; continue; }
        int64_t blk = slot / block_size, off = slot % block_size;
        for (int h = 0; h < n_kv_heads; ++h) {
            size_t row = (size_t)((blk * n_kv_heads + h) * block_size + off);
            for (int kv = 0; kv < 2; ++kv) {
                const float *src = (kv ? v_src : k_src) + ((size_t)t * n_kv_heads + h) * head_dim;
                uint8_t *dst = (uint8_t *)(kv ? v_pages : k_pages) + row * head_dim * eb;
                float *sc = kv ? v_scales : k_scales;
                switch (dtype) {
                case ORC_F32: memcpy(dst, src, head_dim * 4); break;
                case ORC_BF16:
                    for (int d = 0; d < head_dim; ++d) {
                        uint16_t b = orc_bf16_from_f32(src[d]);
                        memcpy(dst + 2 * d, &b, 2);
                    }
                    break;
                case ORC_INT8:
                    for (int g = 0; g < ng; ++g)
                        sc[row * ng + g] = orc_q8_quantize_group(src + g * group, group,
                                                                 (int8_t *)dst + g * group);
                    break;
                case ORC_FP8:
                    for (int g = 0; g < ng; ++g)
                        sc[row * ng + g] = orc_fp8_quantize_group(src + g * group, group,
                                                                  dst + g * group);
                    break;
                }
            }
        }
    }
    return bad;
}

/* Element (row, d) of a pool as f32: dequant q*scale (src/kv_cache.rs:88),
 * to_f32(code)*scale (src/fp8.rs:263-264). */
static float pool_value(int dtype, const void *pages, const float *scales, int head_dim,
                        int group, size_t row, int d) {
    switch (dtype) {
    case ORC_F32: return ((const float *)pages)[row * head_dim + d];
    case ORC_BF16: return orc_bf16_to_f32(((const uint16_t *)pages)[row * head_dim + d]);
    case ORC_INT8:
        return (float)((const int8_t *)pages)[row * head_dim + d] *
               scales[row * (head_dim / group) + d / group];
    default:
        return orc_fp8_to_f32(((const uint8_t *)pages)[row * head_dim + d]) *
               scales[row * (head_dim / group) + d / group];
    }
}

/* Definitional gather: out[h][t][:] = page[table[t / bs]][h][t % bs][:]
 * for t < len (layout 0, the per-head k_cache[kv_len x d] that
 * src/flash_decode.rs:153-163 consumes) or out[t][h][:] (layout 1, the dense
 * [seq, n_kv, d] of src/kv_cache.rs:121-122).  A bf16 cache gathered to bf16
 * copies the raw bits. */
int orc_kv_gather(int dtype, int block_size, int n_kv_heads, int head_dim, int group,
                  int64_t num_blocks, const void *k_pages, const void *v_pages,
                  const float *k_scales, const float *v_scales,
                  const int32_t *block_tables, const int32_t *seq_lens,
                  const int64_t *out_offsets, int batch, int max_blocks,
                  void *out_k, void *out_v, int out_dtype, int out_layout) {
    int bad = 0;
    for (int b = 0; b < batch; ++b) {
        int len = seq_lens[b];
        if (len < 0 || len > max_blocks * block_size) { ++bad; continue; }
        for (int t = 0; t < len; ++t) {
            int32_t blk = block_tables[(size_t)b * max_blocks + t / block_size];
            if (blk < 0 || blk >= num_blocks) { ++bad; continue; }
            for (int h = 0; h < n_kv_heads; ++h) {
                size_t row = ((size_t)blk * n_kv_heads + h) * block_size + t % block_size;
                size_t o = out_layout == 0 ? ((size_t)h * len + t) * head_dim
                                           : ((size_t)t * n_kv_heads + h) * head_dim;
                o += (size_t)out_offsets[b];
                for (int kv = 0; kv < 2; ++kv) {
                    const void *pages = kv ? v_pages : k_pages;
                    const float *sc = kv ? v_scales : k_scales;
                    void *out = kv ? out_v : out_k;
                    for (int d = 0; d < head_dim; ++d) {
                        if (out_dtype == ORC_F32) {
                            ((float *)out)[o + d] = pool_value(dtype, pages, sc, head_dim, group, row, d);
                        } else if (dtype == ORC_BF16) {
                            ((uint16_t *)out)[o + d] = ((const uint16_t *)pages)[row * head_dim + d];
                        } else {
                            ((uint16_t *)out)[o + d] = orc_bf16_from_f32(
                                pool_value(dtype, pages, sc, head_dim, group, row, d));
                        }
                    }
                }
            }
        }
    }
    return bad;
}

/* ------------------------------------------------------------------------ */
/* Flash decode                                                             */
/* ------------------------------------------------------------------------ */

/* chunk_attention, src/flash_decode.rs:70-109 (the scale is a parameter;
 * the reference uses 1/sqrt(d) computed in f32, :81). */
void orc_chunk_attention(const float *q, const float *k_chunk, const float *v_chunk,
                         int chunk_len, int head_dim, float scale, float *out,
                         float *local_max, float *local_sum) {
    float *scores = (float *)malloc(sizeof(float) * (size_t)(chunk_len > 0 ? chunk_len : 1));
    for (int i = 0; i < chunk_len; ++i) {
        float dot = 0.0f;
        for (int j = 0; j < head_dim; ++j) dot += q[j] * k_chunk[(size_t)i * head_dim + j];
        scores[i] = dot * scale;
    }
    float m = -INFINITY;
    for (int i = 0; i < chunk_len; ++i) m = rust_max(m, scores[i]);
    float l = 0.0f;
    for (int i = 0; i < chunk_len; ++i) { scores[i] = expf(scores[i] - m); l += scores[i]; }
    for (int j = 0; j < head_dim; ++j) out[j] = 0.0f;
    for (int i = 0; i < chunk_len; ++i) {
        const float *vr = v_chunk + (size_t)i * head_dim;
        for (int j = 0; j < head_dim; ++j) out[j] += (scores[i] / l) * vr[j];
    }
    *local_max = m;
    *local_sum = l;
    free(scores);
}

/* reduce_chunks, src/flash_decode.rs:114-142.  Returns -1 where the
 * reference asserts (no chunks, or total_sum <= 1e-8). */
int orc_reduce_chunks(const float *outs, const float *maxes, const float *sums,
                      int n_chunks, int head_dim, float *out) {
    if (n_chunks <= 0) return -1;
    float gm = -INFINITY;
    for (int p = 0; p < n_chunks; ++p) gm = rust_max(gm, maxes[p]);
    float *rs = (float *)malloc(sizeof(float) * (size_t)n_chunks);
    float total = 0.0f;
    for (int p = 0; p < n_chunks; ++p) { rs[p] = expf(maxes[p] - gm) * sums[p]; total += rs[p]; }
    if (!(total > 1e-8f)) { free(rs); return -1; }
    for (int j = 0; j < head_dim; ++j) out[j] = 0.0f;
    for (int p = 0; p < n_chunks; ++p) {
        float w = rs[p] / total;
        for (int j = 0; j < head_dim; ++j) out[j] += w * outs[(size_t)p * head_dim + j];
    }
    free(rs);
    return 0;
}

/* flash_decode, src/flash_decode.rs:153-173: chunks of `chunk` tokens (the
 * last may be short), then reduce_chunks. */
int orc_flash_decode(const float *q, const float *k, const float *v, int kv_len,
                     int head_dim, int chunk, float scale, float *out) {
    if (chunk <= 0) return -1;
    int n_chunks = (kv_len + chunk - 1) / chunk;
    if (n_chunks == 0) return -1;
    float *outs = (float *)malloc(sizeof(float) * (size_t)n_chunks * head_dim);
    float *mx = (float *)malloc(sizeof(float) * (size_t)n_chunks);
    float *sm = (float *)malloc(sizeof(float) * (size_t)n_chunks);
    for (int p = 0; p < n_chunks; ++p) {
        int s = p * chunk, n = (kv_len - s) < chunk ? (kv_len - s) : chunk;
        orc_chunk_attention(q, k + (size_t)s * head_dim, v + (size_t)s * head_dim, n, head_dim,
                            scale, outs + (size_t)p * head_dim, &mx[p], &sm[p]);
    }
    int rc = orc_reduce_chunks(outs, mx, sm, n_chunks, head_dim, out);
    free(outs); free(mx); free(sm);
    return rc;
}

/* reference_attention, src/flash_decode.rs:179-207 (naive softmax). */
void orc_reference_attention(const float *q, const float *k, const float *v,
                             int kv_len, int head_dim, float scale, float *out) {
    float *s = (float *)malloc(sizeof(float) * (size_t)(kv_len > 0 ? kv_len : 1));
    for (int i = 0; i < kv_len; ++i) {
        float dot = 0.0f;
        for (int j = 0; j < head_dim; ++j) dot += q[j] * k[(size_t)i * head_dim + j];
        s[i] = dot * scale;
    }
    float m = -INFINITY;
    for (int i = 0; i < kv_len; ++i) m = rust_max(m, s[i]);
    float sum = 0.0f;
    for (int i = 0; i < kv_len; ++i) { s[i] = expf(s[i] - m); sum += s[i]; }
    for (int j = 0; j < head_dim; ++j) out[j] = 0.0f;
    for (int i = 0; i < kv_len; ++i) {
        float w = s[i] / sum;
        for (int j = 0; j < head_dim; ++j) out[j] += w * v[(size_t)i * head_dim + j];
    }
    free(s);
}

/* The same naive softmax in float64: an independent second oracle. */
void orc_reference_attention_f64(const float *q, const float *k, const float *v,
                                 int kv_len, int head_dim, double scale, double *out) {
    double *s = (double *)malloc(sizeof(double) * (size_t)(kv_len > 0 ? kv_len : 1));
    for (int i = 0; i < kv_len; ++i) {
        double dot = 0.0;
        for (int j = 0; j < head_dim; ++j) dot += (double)q[j] * (double)k[(size_t)i * head_dim + j];
        s[i] = dot * scale;
    }
    double m = -INFINITY;
    for (int i = 0; i < kv_len; ++i) m = s[i] > m ? s[i] : m;
    double sum = 0.0;
    for (int i = 0; i < kv_len; ++i) { s[i] = exp(s[i] - m); sum += s[i]; }
    for (int j = 0; j < head_dim; ++j) out[j] = 0.0;
    for (int i = 0; i < kv_len; ++i)
        for (int j = 0; j < head_dim; ++j) out[j] += s[i] / sum * (double)v[(size_t)i * head_dim + j];
    free(s);
}

/* Paged decode = gather of kv head h / group (GQA mapping of
 * src/chunked_attn.rs:240-243 and src/ops.rs:572-584) followed by
 * flash_decode over all seq_lens[b] tokens, for every q head.  The
 * reference has no paged decode; this is the composition of its pieces.
 * A zero-length sequence yields a zero output row (the reference would
 * assert in reduce_chunks). */
int orc_paged_decode(int dtype, int block_size, int n_kv_heads, int head_dim, int group,
                     int64_t num_blocks, const void *k_pages, const void *v_pages,
                     const float *k_scales, const float *v_scales, const float *q,
                     int n_q_heads, const int32_t *block_tables, const int32_t *seq_lens,
                     int batch, int max_blocks, float scale, int chunk, float *out) {
    if (n_q_heads % n_kv_heads) return -1;
    int groups = n_q_heads / n_kv_heads;
    for (int b = 0; b < batch; ++b) {
        int len = seq_lens[b];
        if (len < 0 || len > max_blocks * block_size) return -1;
        float *kc = (float *)malloc(sizeof(float) * (size_t)(len > 0 ? len : 1) * head_dim);
        float *vc = (float *)malloc(sizeof(float) * (size_t)(len > 0 ? len : 1) * head_dim);
        for (int qh = 0; qh < n_q_heads; ++qh) {
            int kvh = qh / groups;
            float *o = out + ((size_t)b * n_q_heads + qh) * head_dim;
            if (len == 0) { for (int j = 0; j < head_dim; ++j) o[j] = 0.0f; continue; }
            for (int t = 0; t < len; ++t) {
                int32_t blk = block_tables[(size_t)b * max_blocks + t / block_size];
                if (blk < 0 || blk >= num_blocks) { free(kc); free(vc); return -1; }
                size_t row = ((size_t)blk * n_kv_heads + kvh) * block_size + t % block_size;
                for (int d = 0; d < head_dim; ++d) {
                    kc[(size_t)t * head_dim + d] = pool_value(dtype, k_pages, k_scales, head_dim, group, row, d);
                    vc[(size_t)t * head_dim + d] = pool_value(dtype, v_pages, v_scales, head_dim, group, row, d);
                }
            }
            if (orc_flash_decode(q + ((size_t)b * n_q_heads + qh) * head_dim, kc, vc, len,
                                 head_dim, chunk, scale, o)) {
                free(kc); free(vc); return -1;
            }
        }
        free(kc); free(vc);
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* kv_compress warm-tier codecs (src/kv_compress.rs)                         */
/* ------------------------------------------------------------------------ */

/* Rust f32::min: NaN-ignoring, like rust_max. */
static inline float rust_min(float a, float b) {
    if (isnan(a)) return b;
    if (isnan(b)) return a;
    return a < b ? a : b;
}

/* `iter.sum::<f32>()`: a left fold in element order.  Current Rust starts the
 * fold at -0.0 (the additive identity that keeps the sign of an all -0.0
 * sum); only empty and all-negative-zero inputs can tell the difference. */
static float rust_sum_sq(const float *x, size_t n) {
    float s = -0.0f;
    for (size_t i = 0; i < n; ++i) s += x[i] * x[i];
    return s;
}

/* CompressedKey::compress (src/kv_compress.rs:79-109): mean and L2 norm by
 * left folds, bit i = key[i] >= mean (a NaN element leaves its bit clear),
 * packed LSB-first into ceil(dim / 64) words. */
void orc_key_compress(const float *key, size_t dim, uint64_t *bits, float *magnitude,
                      float *mean) {
    float s = -0.0f;
    for (size_t i = 0; i < dim; ++i) s += key[i];
    const float m = dim > 0 ? s / (float)dim : 0.0f;
    for (size_t w = 0; w < (dim + 63) / 64; ++w) bits[w] = 0;
    for (size_t i = 0; i < dim; ++i)
        if (key[i] >= m) bits[i / 64] |= 1ull << (i % 64);
    *magnitude = sqrtf(rust_sum_sq(key, dim));
    *mean = m;
}

/* CompressedKey::decompress (:112-127): sign_i * (|k| / sqrt(dim)) + mean,
 * as a product and a sum (no fused multiply-add in Rust). */
void orc_key_decompress(const uint64_t *bits, float magnitude, float mean, size_t dim, float *out) {
    const float scale = dim > 0 ? magnitude / sqrtf((float)dim) : 0.0f;
    for (size_t i = 0; i < dim; ++i) {
        const float sign = ((bits[i / 64] >> (i % 64)) & 1u) ? 1.0f : -1.0f;
        const float p = sign * scale;
        out[i] = p + mean;
    }
}

/* CompressedValue::compress (:187-218): NaN-ignoring min / max folds from
 * +inf / -inf; scale = range / 255 (or 1.0 when range <= 0);
 * q = round_half_away((v - min) / scale) clamped to [0, 255]; Rust's `as u8`
 * sends NaN to 0.  An empty vector has scale 0 and min 0. */
void orc_value_compress(const float *v, size_t dim, uint8_t *q, float *scale, float *min_val) {
    if (dim == 0) {
        *scale = 0.0f;
        *min_val = 0.0f;
        return;
    }
    float lo = INFINITY, hi = -INFINITY;
    for (size_t i = 0; i < dim; ++i) {
        lo = rust_min(lo, v[i]);
        hi = rust_max(hi, v[i]);
    }
    const float range = hi - lo;
    const float s = range > 0.0f ? range / 255.0f : 1.0f;
    for (size_t i = 0; i < dim; ++i) {
        float r = roundf((v[i] - lo) / s);
        if (r < 0.0f) r = 0.0f;
        if (r > 255.0f) r = 255.0f;
        q[i] = isnan(r) ? 0 : (uint8_t)r;
    }
    *scale = s;
    *min_val = lo;
}

/* CompressedValue::decompress (:221-226): q * scale + min (product, then sum). */
void orc_value_decompress(const uint8_t *q, float scale, float min_val, size_t dim, float *out) {
    for (size_t i = 0; i < dim; ++i) {
        const float p = (float)q[i] * scale;
        out[i] = p + min_val;
    }
}

/* qjl_projection_matrix (:994-1015): the Box-Muller pairs of
 * orc_box_muller_fill, each value scaled by 1 / sqrt(orig_dim) after the
 * trigonometric factor: r * cos(theta) * scale, left to right. */
void orc_qjl_projection_matrix(size_t proj_dim, size_t orig_dim, uint64_t seed, float *out) {
    const size_t n = proj_dim * orig_dim;
    uint64_t state = seed + 1;
    const float two53 = 9007199254740992.0f;
    const float scale = 1.0f / sqrtf((float)orig_dim);
    size_t i = 0;
    while (i < n) {
        state = state * 6364136223846793005ULL + 1442695040888963407ULL;
        float u1 = (float)(state >> 11) / two53;
        state = state * 6364136223846793005ULL + 1442695040888963407ULL;
        const float u2 = (float)(state >> 11) / two53;
        u1 = rust_max(u1, 1e-10f);
        const float r = sqrtf(-2.0f * logf(u1));
        const float theta = 2.0f * 3.14159265358979323846f * u2;
        float a = r * cosf(theta);
        out[i++] = a * scale;
        if (i < n) {
            a = r * sinf(theta);
            out[i++] = a * scale;
        }
    }
}

/* QjlKey::compress (:930-951): |k| by a left fold of squares; bit i set when
 * the left-folded dot product of row i of R with k is > 0. */
void orc_qjl_compress(const float *key, size_t dim, const float *proj, size_t proj_dim,
                      uint64_t *bits, float *magnitude) {
    for (size_t w = 0; w < (proj_dim + 63) / 64; ++w) bits[w] = 0;
    for (size_t i = 0; i < proj_dim; ++i) {
        const float *row = proj + i * dim;
        float dot = -0.0f;
        for (size_t j = 0; j < dim; ++j) {
            const float p = row[j] * key[j];
            dot += p;
        }
        if (dot > 0.0f) bits[i / 64] |= 1ull << (i % 64);
    }
    *magnitude = sqrtf(rust_sum_sq(key, dim));
}

/* QjlKey::approx_cos_sim (:959-968): cos(pi * hamming / m), the product
 * taken before the division. */
float orc_qjl_cos_sim(const uint64_t *a, const uint64_t *b, size_t proj_dim) {
    uint32_t ham = 0;
    for (size_t w = 0; w < (proj_dim + 63) / 64; ++w) ham += (uint32_t)__builtin_popcountll(a[w] ^ b[w]);
    const float angle = 3.14159265358979323846f * (float)ham / (float)proj_dim;
    return cosf(angle);
}

/* ------------------------------------------------------------------------ */
/* Blockwise (chunked, causal) attention (src/chunked_attn.rs)               */
/* ------------------------------------------------------------------------ */

/* blockwise_attention_head (src/chunked_attn.rs:114-213) for one head:
 * q [seq_q][d], k / v [seq_kv][d]; query qi sits at absolute position
 * q_offset + qi and, when causal, sees keys 0..=that position.  Per KV block
 * of block_size keys: scores (left-folded dot product, then * scale), block
 * max, running-max update (exp(m_old - m_new) rescale of acc and l), block
 * probabilities exp(s - m_new) summed left to right, acc += p * v row by row;
 * finally acc / max(l, 1e-8).  Each f32 operation rounds once, in the
 * reference's order (the libm expf is glibc's, which Rust's f32::exp calls
 * on Linux). */
void orc_blockwise_attention_head(const float *q, const float *k, const float *v, int seq_q,
                                  int seq_kv, int head_dim, float scale, int block_size,
                                  int causal, int q_offset, float *out) {
    float *l = (float *)malloc(sizeof(float) * (size_t)(seq_q > 0 ? seq_q : 1));
    float *m = (float *)malloc(sizeof(float) * (size_t)(seq_q > 0 ? seq_q : 1));
    int bs = block_size < seq_kv ? block_size : seq_kv;
    if (bs < 1) bs = 1;
    float *s_row = (float *)malloc(sizeof(float) * (size_t)bs);
    float *p_row = (float *)malloc(sizeof(float) * (size_t)bs);
    for (int i = 0; i < seq_q; ++i) {
        l[i] = 0.0f;
        m[i] = -INFINITY;
        for (int j = 0; j < head_dim; ++j) out[(size_t)i * head_dim + j] = 0.0f;
    }
    const int n_blocks = (seq_kv + bs - 1) / bs;
    for (int kb = 0; kb < n_blocks; ++kb) {
        const int ks = kb * bs;
        const int ke = ks + bs < seq_kv ? ks + bs : seq_kv;
        const int blk = ke - ks;
        for (int qi = 0; qi < seq_q; ++qi) {
            const int qpos = q_offset + qi;
            const float *qr = q + (size_t)qi * head_dim;
            for (int kj = 0; kj < blk; ++kj) {
                if (causal && ks + kj > qpos) { s_row[kj] = -INFINITY; continue; }
                const float *kr = k + (size_t)(ks + kj) * head_dim;
                float dot = -0.0f;
                for (int j = 0; j < head_dim; ++j) { const float p = qr[j] * kr[j]; dot += p; }
                s_row[kj] = dot * scale;
            }
            float mb = -INFINITY;
            for (int kj = 0; kj < blk; ++kj) mb = rust_max(mb, s_row[kj]);
            const float m_new = rust_max(m[qi], mb);
            const float e_old = expf(m[qi] - m_new);
            float *o = out + (size_t)qi * head_dim;
            for (int j = 0; j < head_dim; ++j) o[j] *= e_old;
            l[qi] *= e_old;
            float bl = 0.0f;
            for (int kj = 0; kj < blk; ++kj) { p_row[kj] = expf(s_row[kj] - m_new); bl += p_row[kj]; }
            for (int kj = 0; kj < blk; ++kj) {
                const float *vr = v + (size_t)(ks + kj) * head_dim;
                for (int j = 0; j < head_dim; ++j) { const float t = p_row[kj] * vr[j]; o[j] += t; }
            }
            l[qi] += bl;
            m[qi] = m_new;
        }
    }
    for (int qi = 0; qi < seq_q; ++qi) {
        const float den = rust_max(l[qi], 1e-8f);
        for (int j = 0; j < head_dim; ++j) out[(size_t)qi * head_dim + j] /= den;
    }
    free(l); free(m); free(s_row); free(p_row);
}

/* Paged prefill over a pool (device layout): for each sequence b, its
 * q_len = cu_q[b+1] - cu_q[b] newest tokens (already in the cache, whose
 * length is seq_lens[b]) attend causally over all seq_lens[b] tokens, i.e.
 * blockwise_attention_head with q_offset = seq_lens[b] - q_len, per query
 * head h on kv head h / group (the mask of src/ops.rs:762-790).  q / out:
 * [total_q][n_q_heads][head_dim] f32.  Returns 0, or -1 on a bad table entry
 * or a q_len above seq_len. */
int orc_paged_prefill(int dtype, int block_size, int n_kv_heads, int head_dim, int scale_group,
                      int group, int64_t num_blocks, const void *k_pages, const void *v_pages,
                      const float *k_scales, const float *v_scales, const float *q, int n_q_heads,
                      const int32_t *cu_q, const int32_t *block_tables, const int32_t *seq_lens,
                      int batch, int max_blocks, float scale, int kv_block, float *out) {
    for (int b = 0; b < batch; ++b) {
        const int len = seq_lens[b], nq = cu_q[b + 1] - cu_q[b];
        if (len < 0 || len > max_blocks * block_size || nq < 0 || nq > len) return -1;
        if (nq == 0) continue;
        for (int t = 0; t < len; ++t) {
            const int32_t blk = block_tables[(size_t)b * max_blocks + t / block_size];
            if (blk < 0 || blk >= num_blocks) return -1;
        }
        float *kc = (float *)malloc(sizeof(float) * (size_t)len * head_dim);
        float *vc = (float *)malloc(sizeof(float) * (size_t)len * head_dim);
        float *qh = (float *)malloc(sizeof(float) * (size_t)nq * head_dim);
        float *oh = (float *)malloc(sizeof(float) * (size_t)nq * head_dim);
        for (int h = 0; h < n_q_heads; ++h) {
            const int kvh = h / group;
            for (int t = 0; t < len; ++t) {
                const int32_t blk = block_tables[(size_t)b * max_blocks + t / block_size];
                const size_t row = ((size_t)blk * n_kv_heads + kvh) * block_size + t % block_size;
                for (int j = 0; j < head_dim; ++j) {
                    kc[(size_t)t * head_dim + j] = pool_value(dtype, k_pages, k_scales, head_dim, scale_group, row, j);
                    vc[(size_t)t * head_dim + j] = pool_value(dtype, v_pages, v_scales, head_dim, scale_group, row, j);
                }
            }
            for (int r = 0; r < nq; ++r)
                memcpy(qh + (size_t)r * head_dim, q + ((size_t)(cu_q[b] + r) * n_q_heads + h) * head_dim,
                       sizeof(float) * head_dim);
            orc_blockwise_attention_head(qh, kc, vc, nq, len, head_dim, scale, kv_block, 1, len - nq, oh);
            for (int r = 0; r < nq; ++r)
                memcpy(out + ((size_t)(cu_q[b] + r) * n_q_heads + h) * head_dim, oh + (size_t)r * head_dim,
                       sizeof(float) * head_dim);
        }
        free(kc); free(vc); free(qh); free(oh);
    }
    return 0;
}
