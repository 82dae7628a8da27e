// Moving 8 consecutive head_dim elements of one (token, kv head) row between
// registers (as f32) and a page of any pool dtype: the shared building block
// of append, gather and the KvBlock wire kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "air_kv.h"
#include "codecs.hpp"

namespace airkv {

// Page rows are written with plain stores: the c2 append of 32768 tokens ran
// in 70.4 us against 74.7 with non-temporal ones (same box, two runs each),
// and wire unpacking was unchanged.  (Gather's contiguous outputs and the
// block copies measured the other way and keep non-temporal stores.)
template <typename T>
__device__ __forceinline__ void pio_store(T v, T *p) {
    *p = v;
}

typedef float pio_f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t pio_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t pio_u32x2 __attribute__((ext_vector_type(2)));

// Page -> 8 f32 (INT8/FP8 dequantized as q * scale, src/kv_cache.rs:88 and
// src/fp8.rs:263-264).  For BF16 pages `raw` receives the 16 source bytes so
// a bf16 destination can copy them without re-rounding.
template <int DT>
__device__ __forceinline__ void load8(const void *pages, const float *scales, int64_t elem,
                                      int64_t scale_idx, float (&x)[8], pio_u32x4 *raw) {
    if constexpr (DT == AIR_KV_F32) {
        const pio_f32x4 *p = reinterpret_cast<const pio_f32x4 *>((const float *)pages + elem);
        const pio_f32x4 a = __builtin_nontemporal_load(p), b = __builtin_nontemporal_load(p + 1);
        x[0] = a[0]; x[1] = a[1]; x[2] = a[2]; x[3] = a[3]; x[4] = b[0]; x[5] = b[1]; x[6] = b[2]; x[7] = b[3];
    } else if constexpr (DT == AIR_KV_BF16) {
        const pio_u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const pio_u32x4 *>((const uint16_t *)pages + elem));
        *raw = w;
        uint32_t u[4] = {w[0], w[1], w[2], w[3]};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            x[2 * j] = __uint_as_float(u[j] << 16);
            x[2 * j + 1] = __uint_as_float(u[j] & 0xFFFF0000u);
        }
    } else {
        const pio_u32x2 w = __builtin_nontemporal_load(reinterpret_cast<const pio_u32x2 *>((const uint8_t *)pages + elem));
        const float s = scales[scale_idx];
        uint32_t u[2] = {w[0], w[1]};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint32_t byte = (u[j >> 2] >> (8 * (j & 3))) & 0xFFu;
            float val;
            if constexpr (DT == AIR_KV_INT8) val = (float)(int32_t)(int8_t)byte;
            else val = fp8_decode(byte);
            {
#pragma clang fp contract(off)
                x[j] = val * s;   // q as f32 * scale (src/kv_cache.rs:88, src/fp8.rs:263-264)
            }
        }
    }
}


// A lane's value from lane (l & ~3) | perm[l & 3] of its quad, or from the
// mirror image of its 8- or 16-lane row (DPP: no LDS round trip).  The
// source lanes must be active.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int kQuadXor1 = 0xB1;        // quad_perm [1, 0, 3, 2]: lane l ^ 1
constexpr int kQuadXor2 = 0x4E;        // quad_perm [2, 3, 0, 1]: lane l ^ 2
constexpr int kRowHalfMirror = 0x141;  // lane 7 - l within each 8 lanes
constexpr int kRowMirror = 0x140;      // lane 15 - l within each 16 lanes

// The absmax of m over each aligned run of lanes_per_group (a power of two,
// at most 64) lanes, in every lane of the run: after the two quad steps a
// lane holds its quad's maximum, the half-row mirror joins the other quad of
// its 8 lanes, the row mirror the other half of its 16, and shuffles the
// rest.  Every lane of a run must be active.
__device__ __forceinline__ float group_absmax(float m, int lanes_per_group) {
    if (lanes_per_group > 1) m = absmax_step(m, dpp_f32<kQuadXor1>(m));
    if (lanes_per_group > 2) m = absmax_step(m, dpp_f32<kQuadXor2>(m));
    if (lanes_per_group > 4) m = absmax_step(m, dpp_f32<kRowHalfMirror>(m));
    if (lanes_per_group > 8) m = absmax_step(m, dpp_f32<kRowMirror>(m));
    for (int mask = 16; mask < lanes_per_group; mask <<= 1) m = absmax_step(m, __shfl_xor(m, mask));
    return m;
}

// The INT8 / FP8 codes (element 4i + j in byte j of w[i]) and the group
// scale of a lane's N f32 of one scale group: the lanes_per_group
// consecutive lanes holding the group reduce its absmax with butterfly
// shuffles (every lane of the group must call this).  The absmax folds from 0.0 with a
// NaN-ignoring max (src/kv_cache.rs:60, src/fp8.rs:228-232); max is order
// independent, so the lane-parallel reduction equals the reference's
// sequential fold.  Shared by the append kernel and the fused append of the
// decode kernel, so both write the same bytes.
template <int DT, int N>
__device__ __forceinline__ void quantize_elems(const float (&x)[N], int lanes_per_group, uint32_t (&w)[N / 4],
                                               float &scale) {
    static_assert(DT == AIR_KV_INT8 || DT == AIR_KV_FP8, "1-byte pages only");
    static_assert(N % 4 == 0, "whole code words");
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < N; ++j) m = absmax_step(m, x[j]);
    m = group_absmax(m, lanes_per_group);
    if constexpr (DT == AIR_KV_INT8) {
        scale = q8_scale(m);
        float inv;
        {
#pragma clang fp contract(off)
            inv = 1.0f / scale;
        }
#pragma unroll
        for (int i = 0; i < N / 4; ++i) w[i] = 0;
#pragma unroll
        for (int j = 0; j < N; ++j) w[j / 4] |= (uint32_t)(uint8_t)q8_code(x[j], inv) << (8 * (j % 4));
    } else {
        scale = fp8_scale(m);
        float y;
        {
#pragma clang fp contract(off)
            y = 1.0f / scale;
        }
        const bool mark = __builtin_isnormal(scale) && __builtin_isnormal(y);
        fp8_codes<N>(x, scale, y, mark, w);
    }
}

// quantize_elems of a lane's 8 elements: codes of elements 0..3 in lo, 4..7 in hi.
template <int DT>
__device__ __forceinline__ void quantize_chunk(const float (&x)[8], int lanes_per_group, uint32_t &lo,
                                               uint32_t &hi, float &scale) {
    uint32_t w[2];
    quantize_elems<DT, 8>(x, lanes_per_group, w, scale);
    lo = w[0];
    hi = w[1];
}

// 8 f32 -> page: F32 stored as is, BF16 rounded to nearest even, INT8 / FP8
// quantized with one scale per scale_group elements; the lanes_per_group
// consecutive lanes holding one group reduce its absmax with butterfly
// shuffles (every lane of the group must call this), and the `lead` lane
// stores the scale.  Nothing is stored when `valid` is false.
template <int DT>
__device__ __forceinline__ void store_row_chunk(const float (&x)[8], void *pages, float *scales,
                                                int64_t elem, int64_t scale_idx, bool lead,
                                                int lanes_per_group, bool valid) {
    if constexpr (DT == AIR_KV_F32) {
        if (valid) {
            pio_f32x4 *o = reinterpret_cast<pio_f32x4 *>((float *)pages + elem);
            pio_store(pio_f32x4{x[0], x[1], x[2], x[3]}, o);
            pio_store(pio_f32x4{x[4], x[5], x[6], x[7]}, o + 1);
        }
    } else if constexpr (DT == AIR_KV_BF16) {
        if (valid) {
            pio_u32x4 w;
            w[0] = (uint32_t)bf16_rne(x[0]) | ((uint32_t)bf16_rne(x[1]) << 16);
            w[1] = (uint32_t)bf16_rne(x[2]) | ((uint32_t)bf16_rne(x[3]) << 16);
            w[2] = (uint32_t)bf16_rne(x[4]) | ((uint32_t)bf16_rne(x[5]) << 16);
            w[3] = (uint32_t)bf16_rne(x[6]) | ((uint32_t)bf16_rne(x[7]) << 16);
            pio_store(w, reinterpret_cast<pio_u32x4 *>((uint16_t *)pages + elem));
        }
    } else {
        uint32_t lo, hi;
        float scale;
        quantize_chunk<DT>(x, lanes_per_group, lo, hi, scale);
        if (valid) {
            pio_store(pio_u32x2{lo, hi}, reinterpret_cast<pio_u32x2 *>((uint8_t *)pages + elem));
            if (lead) scales[scale_idx] = scale;
        }
    }
}

}  // namespace airkv
