// Host-side framing of KvBlocks for prefill/decode disaggregation: the byte
// layouts of src/pd_disagg.rs around the wire data that air_kv_pack_blocks /
// air_kv_pack_blocks_int8 produce on the device.  Every integer is
// little-endian, as the reference's to_le_bytes writes it; the functions do
// not depend on the host's byte order.
#include <cstring>

#include "air_kv.h"
#include "status.hpp"

using airkv::fail;

namespace {

constexpr size_t kFrameHeader = 10;    // [block_id:4][layer_idx:2][data_len:4]
constexpr size_t kInt8Header = 14;     // [block_id:4][layer_idx:2][scale:4][len:4]

void put_u16(uint8_t *p, uint16_t v) {
    p[0] = (uint8_t)v;
    p[1] = (uint8_t)(v >> 8);
}
void put_u32(uint8_t *p, uint32_t v) {
    for (int i = 0; i < 4; ++i) p[i] = (uint8_t)(v >> (8 * i));
}
uint16_t get_u16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
uint32_t get_u32(const uint8_t *p) {
    uint32_t v = 0;
    for (int i = 0; i < 4; ++i) v |= (uint32_t)p[i] << (8 * i);
    return v;
}

void frame(uint8_t *out, uint32_t block_id, uint16_t layer_idx, const void *data, uint32_t data_len) {
    put_u32(out, block_id);
    put_u16(out + 4, layer_idx);
    put_u32(out + 6, data_len);
    if (data_len) std::memcpy(out + kFrameHeader, data, data_len);
}

void int8_payload(uint8_t *out, uint32_t block_id, uint16_t layer_idx, float scale, const int8_t *codes,
                  uint32_t n) {
    uint32_t sbits;
    std::memcpy(&sbits, &scale, 4);
    put_u32(out, block_id);
    put_u16(out + 4, layer_idx);
    put_u32(out + 6, sbits);
    put_u32(out + 10, n);
    if (n) std::memcpy(out + kInt8Header, codes, n);
}

}  // namespace

extern "C" {

size_t air_kv_block_frame_bytes(size_t data_len) { return kFrameHeader + data_len; }

int air_kv_block_serialise(uint32_t block_id, uint16_t layer_idx, const void *data, size_t data_len, void *out,
                           size_t cap, size_t *written) {
    if (!out || (data_len && !data)) return fail(AIR_KV_E_INVALID_ARG, "serialise: NULL buffer");
    if (data_len > UINT32_MAX) return fail(AIR_KV_E_INVALID_ARG, "serialise: data_len above u32");
    if (cap < kFrameHeader + data_len)
        return fail(AIR_KV_E_INVALID_ARG, "serialise: %zu bytes of room for a %zu-byte frame", cap,
                    kFrameHeader + data_len);
    frame((uint8_t *)out, block_id, layer_idx, data, (uint32_t)data_len);
    if (written) *written = kFrameHeader + data_len;
    return AIR_KV_OK;
}

int air_kv_block_deserialise(const void *buf, size_t len, uint32_t *block_id, uint16_t *layer_idx,
                             const void **data, size_t *data_len) {
    if (!buf && len) return fail(AIR_KV_E_INVALID_ARG, "deserialise: NULL buffer");
    if (len < kFrameHeader) return fail(AIR_KV_E_INVALID_ARG, "deserialise: %zu bytes, shorter than the header", len);
    const uint8_t *p = (const uint8_t *)buf;
    const size_t n = get_u32(p + 6);
    if (len < kFrameHeader + n)
        return fail(AIR_KV_E_INVALID_ARG, "deserialise: frame announces %zu data bytes, %zu present", n,
                    len - kFrameHeader);
    if (block_id) *block_id = get_u32(p);
    if (layer_idx) *layer_idx = get_u16(p + 4);
    if (data) *data = p + kFrameHeader;
    if (data_len) *data_len = n;
    return AIR_KV_OK;
}

int air_kv_block_serialise_n(const uint32_t *block_ids, uint16_t layer_idx, const void *data, size_t block_bytes,
                             int32_t n, void *out) {
    if (n < 0) return fail(AIR_KV_E_INVALID_ARG, "serialise_n: n < 0");
    if (n == 0) return AIR_KV_OK;
    if (!block_ids || !out || (block_bytes && !data)) return fail(AIR_KV_E_INVALID_ARG, "serialise_n: NULL buffer");
    if (block_bytes > UINT32_MAX) return fail(AIR_KV_E_INVALID_ARG, "serialise_n: block_bytes above u32");
    uint8_t *o = (uint8_t *)out;
    const uint8_t *d = (const uint8_t *)data;
    for (int32_t i = 0; i < n; ++i)
        frame(o + (size_t)i * (kFrameHeader + block_bytes), block_ids[i], layer_idx, d + (size_t)i * block_bytes,
              (uint32_t)block_bytes);
    return AIR_KV_OK;
}

size_t air_kv_int8_payload_bytes(size_t n_codes) { return kInt8Header + n_codes; }

int air_kv_int8_payload_serialise(uint32_t block_id, uint16_t layer_idx, float scale, const int8_t *codes,
                                  size_t n_codes, void *out, size_t cap, size_t *written) {
    if (!out || (n_codes && !codes)) return fail(AIR_KV_E_INVALID_ARG, "int8 payload: NULL buffer");
    if (n_codes > UINT32_MAX) return fail(AIR_KV_E_INVALID_ARG, "int8 payload: more than u32 codes");
    if (cap < kInt8Header + n_codes)
        return fail(AIR_KV_E_INVALID_ARG, "int8 payload: %zu bytes of room for %zu", cap, kInt8Header + n_codes);
    int8_payload((uint8_t *)out, block_id, layer_idx, scale, codes, (uint32_t)n_codes);
    if (written) *written = kInt8Header + n_codes;
    return AIR_KV_OK;
}

int air_kv_int8_payload_deserialise(const void *buf, size_t len, uint32_t *block_id, uint16_t *layer_idx,
                                    float *scale, const int8_t **codes, size_t *n_codes) {
    if (!buf && len) return fail(AIR_KV_E_INVALID_ARG, "int8 payload: NULL buffer");
    if (len < kInt8Header) return fail(AIR_KV_E_INVALID_ARG, "int8 payload: %zu bytes, shorter than the header", len);
    const uint8_t *p = (const uint8_t *)buf;
    const size_t n = get_u32(p + 10);
    if (len < kInt8Header + n)
        return fail(AIR_KV_E_INVALID_ARG, "int8 payload: %zu codes announced, %zu present", n, len - kInt8Header);
    if (block_id) *block_id = get_u32(p);
    if (layer_idx) *layer_idx = get_u16(p + 4);
    if (scale) {
        const uint32_t sbits = get_u32(p + 6);
        std::memcpy(scale, &sbits, 4);
    }
    if (codes) *codes = (const int8_t *)(p + kInt8Header);
    if (n_codes) *n_codes = n;
    return AIR_KV_OK;
}

int air_kv_int8_payload_serialise_n(const uint32_t *block_ids, uint16_t layer_idx, const float *scales,
                                    const int8_t *codes, size_t codes_per_block, int32_t n, void *out) {
    if (n < 0) return fail(AIR_KV_E_INVALID_ARG, "int8 payload_n: n < 0");
    if (n == 0) return AIR_KV_OK;
    if (!block_ids || !scales || !out || (codes_per_block && !codes))
        return fail(AIR_KV_E_INVALID_ARG, "int8 payload_n: NULL buffer");
    if (codes_per_block > UINT32_MAX) return fail(AIR_KV_E_INVALID_ARG, "int8 payload_n: more than u32 codes");
    uint8_t *o = (uint8_t *)out;
    for (int32_t i = 0; i < n; ++i)
        int8_payload(o + (size_t)i * (kInt8Header + codes_per_block), block_ids[i], layer_idx, scales[i],
                     codes + (size_t)i * codes_per_block, (uint32_t)codes_per_block);
    return AIR_KV_OK;
}

}  // extern "C"
