// decode.h -- bit-exact per-format decoders for one 32-weight part of a block.
//
// decode_part<T>(blk, p, out) writes weights 32p .. 32p+31 of the block at
// `blk` into out[0..31], rounding exactly like the reference CPU decoder
// (src/quants.c:85-248): every product and difference rounds on its own
// (the code object is compiled with -ffp-contract=off) and operands combine
// in the reference's order. Q2_K, Q3_K and IQ2_XXS are not in the
// reference; they follow the public ggml layout. These are the decoders of
// the standalone dequant kernel and of the generic matvec, so both share
// one definition of every format.
#pragma once
#include "common.h"
#include "../iq_tables.h"

__constant__ uint64_t c_iq2xs_grid[512] = SEPIA_IQ2XS_GRID_INIT;
__constant__ uint32_t c_iq3xxs_grid[256] = SEPIA_IQ3XXS_GRID_INIT;
__constant__ int8_t c_iq4nl[16] = SEPIA_IQ4NL_VALUES_INIT;
// IQ2_XXS codebook: not available offline; installed at run time by
// sepia_hip_set_iq2xxs_grid (the type is rejected until then).
__device__ uint64_t g_iq2xxs_grid[256];

template <int T> struct Fmt;
template <> struct Fmt<ST_Q8_0>    { static constexpr int elems = 32,  bytes = 34,  parts = 1; };
template <> struct Fmt<ST_Q2_K>    { static constexpr int elems = 256, bytes = 84,  parts = 8; };
template <> struct Fmt<ST_Q3_K>    { static constexpr int elems = 256, bytes = 110, parts = 8; };
template <> struct Fmt<ST_Q4_K>    { static constexpr int elems = 256, bytes = 144, parts = 8; };
template <> struct Fmt<ST_Q5_K>    { static constexpr int elems = 256, bytes = 176, parts = 8; };
template <> struct Fmt<ST_Q6_K>    { static constexpr int elems = 256, bytes = 210, parts = 8; };
template <> struct Fmt<ST_IQ2_XXS> { static constexpr int elems = 256, bytes = 66,  parts = 8; };
template <> struct Fmt<ST_IQ2_XS>  { static constexpr int elems = 256, bytes = 74,  parts = 8; };
template <> struct Fmt<ST_IQ3_XXS> { static constexpr int elems = 256, bytes = 98,  parts = 8; };
template <> struct Fmt<ST_IQ4_XS>  { static constexpr int elems = 256, bytes = 136, parts = 8; };

__device__ __forceinline__ float h2f(const uint8_t *p) { return f16_bits_to_f32(ld_u16(p)); }

// Even-parity sign byte of a 7-bit sign index: bit j negates weight j.
__device__ __forceinline__ uint32_t iq_signs(uint32_t idx7) {
    return idx7 | ((__builtin_popcount(idx7) & 1u) << 7);
}

// 6-bit (scale, min) pair j of the packed K-quant scale bytes
// (src/quants.c:96-102).
__device__ __forceinline__ void k4_scale_min(const uint8_t *s, int j, int &sc, int &mn) {
    if (j < 4) {
        sc = ld_u8(s + j) & 63;
        mn = ld_u8(s + j + 4) & 63;
    } else {
        sc = (ld_u8(s + j + 4) & 15) | ((ld_u8(s + j - 4) >> 6) << 4);
        mn = (ld_u8(s + j + 4) >> 4) | ((ld_u8(s + j) >> 6) << 4);
    }
}

template <int T> __device__ void decode_part(const uint8_t *b, int p, float *out);

// src/quants.c:85-94
template <> __device__ void decode_part<ST_Q8_0>(const uint8_t *b, int, float *out) {
    const float d = h2f(b);
#pragma unroll
    for (int i = 0; i < 32; i++) out[i] = d * (float)(int8_t)ld_u8(b + 2 + i);
}

// src/quants.c:104-125: part p = sub-block p; nibble (p & 1) of qs[32*(p/2) + l].
template <> __device__ void decode_part<ST_Q4_K>(const uint8_t *b, int p, float *out) {
    const float d = h2f(b), dmin = h2f(b + 2);
    int sc, mn;
    k4_scale_min(b + 4, p, sc, mn);
    const float ds = d * (float)sc, dm = dmin * (float)mn;
    const uint8_t *qs = b + 16 + 32 * (p >> 1);
    const int sh = 4 * (p & 1);
#pragma unroll
    for (int l = 0; l < 32; l++) out[l] = ds * (float)((ld_u8(qs + l) >> sh) & 15) - dm;
}

// src/quants.c:127-151: as Q4_K plus bit p of qh[l] worth 16.
template <> __device__ void decode_part<ST_Q5_K>(const uint8_t *b, int p, float *out) {
    const float d = h2f(b), dmin = h2f(b + 2);
    int sc, mn;
    k4_scale_min(b + 4, p, sc, mn);
    const float ds = d * (float)sc, dm = dmin * (float)mn;
    const uint8_t *qh = b + 16, *ql = b + 48 + 32 * (p >> 1);
    const int sh = 4 * (p & 1);
#pragma unroll
    for (int l = 0; l < 32; l++) {
        int q = (ld_u8(ql + l) >> sh) & 15;
        if ((ld_u8(qh + l) >> p) & 1) q += 16;
        out[l] = ds * (float)q - dm;
    }
}

// src/quants.c:153-177: part p = 32r + l rows of half h = p/4, r = p%4.
template <> __device__ void decode_part<ST_Q6_K>(const uint8_t *b, int p, float *out) {
    const float d = h2f(b + 208);
    const int h = p >> 2, r = p & 3;
    const uint8_t *ql = b + 64 * h + 32 * (r & 1), *qh = b + 128 + 32 * h;
    const int8_t *sc = (const int8_t *)(b + 192 + 8 * h + 2 * r);
    const int sh = 4 * (r >> 1);
#pragma unroll
    for (int l = 0; l < 32; l++) {
        int q = (((ld_u8(ql + l) >> sh) & 15) | (((ld_u8(qh + l) >> (2 * r)) & 3) << 4)) - 32;
        out[l] = d * (float)sc[l >> 4] * (float)q;
    }
}

// ggml Q2_K: part p = half h (p/4), shift s (p%4); weights 16g + l use scale
// byte 8h + 2s + g and bits (qs[32h + 16g + l] >> 2s) & 3.
template <> __device__ void decode_part<ST_Q2_K>(const uint8_t *b, int p, float *out) {
    const float d = h2f(b + 80), dmin = h2f(b + 82);
    const int h = p >> 2, s = p & 3;
    const uint8_t *qs = b + 16 + 32 * h;
#pragma unroll
    for (int g = 0; g < 2; g++) {
        const uint32_t scb = ld_u8(b + 8 * h + 2 * s + g);
        const float dl = d * (float)(scb & 15), ml = dmin * (float)(scb >> 4);
#pragma unroll
        for (int l = 0; l < 16; l++) out[16 * g + l] = dl * (float)((ld_u8(qs + 16 * g + l) >> (2 * s)) & 3) - ml;
    }
}

// Q3_K 6-bit scale j, stored +32 (ggml's 12-byte packing).
__device__ __forceinline__ int q3_scale(const uint8_t *s, int j) {
    int lo = (j < 8) ? (ld_u8(s + j) & 15) : (ld_u8(s + j - 8) >> 4);
    int hi = (ld_u8(s + 8 + (j & 3)) >> (2 * (j >> 2))) & 3;
    return (lo | (hi << 4)) - 32;
}

// ggml Q3_K: as Q2_K's indexing; q = bits - 4 unless hmask[16g + l] bit (4h + s).
template <> __device__ void decode_part<ST_Q3_K>(const uint8_t *b, int p, float *out) {
    const float d = h2f(b + 108);
    const int h = p >> 2, s = p & 3;
    const uint8_t *qs = b + 32 + 32 * h;
#pragma unroll
    for (int g = 0; g < 2; g++) {
        const float dl = d * (float)q3_scale(b + 96, 8 * h + 2 * s + g);
#pragma unroll
        for (int l = 0; l < 16; l++) {
            int q = (ld_u8(qs + 16 * g + l) >> (2 * s)) & 3;
            if (!((ld_u8(b + 16 * g + l) >> (4 * h + s)) & 1)) q -= 4;
            out[16 * g + l] = dl * (float)q;
        }
    }
}

// src/quants.c:179-201
template <> __device__ void decode_part<ST_IQ2_XS>(const uint8_t *b, int p, float *out) {
    const float d = h2f(b);
    const uint32_t sb = ld_u8(b + 66 + p);
#pragma unroll
    for (int l = 0; l < 4; l++) {
        const float db = d * (0.5f + (float)((l < 2) ? (sb & 15) : (sb >> 4))) * 0.25f;
        const uint32_t v = ld_u16(b + 2 + 2 * (4 * p + l));
        const uint64_t g = c_iq2xs_grid[v & 511];
        const uint32_t sg = iq_signs(v >> 9);
#pragma unroll
        for (int j = 0; j < 8; j++)
            out[8 * l + j] = db * (float)((g >> (8 * j)) & 0xFF) * (((sg >> j) & 1) ? -1.0f : 1.0f);
    }
}

// ggml IQ2_XXS: 4 grid bytes, then u32 of 4 x 7-bit sign indices + 4-bit scale.
template <> __device__ void decode_part<ST_IQ2_XXS>(const uint8_t *b, int p, float *out) {
    const float d = h2f(b);
    const uint8_t *q = b + 2 + 8 * p;
    const uint32_t s = ld_u32(q + 4);
    const float db = d * (0.5f + (float)(s >> 28)) * 0.25f;
#pragma unroll
    for (int l = 0; l < 4; l++) {
        const uint64_t g = g_iq2xxs_grid[ld_u8(q + l)];
        const uint32_t sg = iq_signs((s >> (7 * l)) & 127);
#pragma unroll
        for (int j = 0; j < 8; j++)
            out[8 * l + j] = db * (float)((g >> (8 * j)) & 0xFF) * (((sg >> j) & 1) ? -1.0f : 1.0f);
    }
}

// src/quants.c:203-226
template <> __device__ void decode_part<ST_IQ3_XXS>(const uint8_t *b, int p, float *out) {
    const float d = h2f(b);
    const uint32_t a = ld_u32(b + 66 + 4 * p);
    const float db = d * (0.5f + (float)(a >> 28)) * 0.5f;
#pragma unroll
    for (int l = 0; l < 4; l++) {
        const uint32_t sg = iq_signs((a >> (7 * l)) & 127);
#pragma unroll
        for (int half = 0; half < 2; half++) {
            const uint32_t g = c_iq3xxs_grid[ld_u8(b + 2 + 8 * p + 2 * l + half)];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int bit = 4 * half + j;
                out[8 * l + bit] = db * (float)((g >> (8 * j)) & 0xFF) * (((sg >> bit) & 1) ? -1.0f : 1.0f);
            }
        }
    }
}

// src/quants.c:228-248
template <> __device__ void decode_part<ST_IQ4_XS>(const uint8_t *b, int p, float *out) {
    const float d = h2f(b);
    const uint32_t sh = ld_u16(b + 2);
    const int ls = ((ld_u8(b + 4 + p / 2) >> (4 * (p & 1))) & 15) | (((sh >> (2 * p)) & 3) << 4);
    const float dl = d * (float)(ls - 32);
    const uint8_t *qs = b + 8 + 16 * p;
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const uint32_t v = ld_u8(qs + j);
        out[j] = dl * (float)c_iq4nl[v & 15];
        out[16 + j] = dl * (float)c_iq4nl[v >> 4];
    }
}
