// matvec.h -- wave-level row dot products.
//
// row_dot_generic<T>: one 64-lane wave computes dot(deq(row), x) for one
// quantized row of n_blocks blocks. Lanes take the row's 32-weight parts in
// turn (lane, lane+64, ...), decode each with the bit-exact decoder into
// registers and fold it into an f32 FMA chain; wave_sum adds the 64 partials.
// Every lane returns the row total.
#pragma once
#include "common.h"
#include "decode.h"

template <int T>
__device__ __forceinline__ float row_dot_generic(const uint8_t *__restrict__ row, int64_t n_blocks,
                                                 const float *__restrict__ x) {
    const int lane = threadIdx.x & 63;
    const int64_t n_parts = n_blocks * Fmt<T>::parts;
    float acc = 0.0f;
    for (int64_t u = lane; u < n_parts; u += SEPIA_WAVE) {
        const int64_t b = u / Fmt<T>::parts;
        const int p = (int)(u % Fmt<T>::parts);
        float w[32];
        decode_part<T>(row + b * Fmt<T>::bytes, p, w);
        const float4 *xv = (const float4 *)(x + b * Fmt<T>::elems + 32 * p);
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float4 xx = xv[k];
            acc = __builtin_fmaf(w[4 * k + 0], xx.x, acc);
            acc = __builtin_fmaf(w[4 * k + 1], xx.y, acc);
            acc = __builtin_fmaf(w[4 * k + 2], xx.z, acc);
            acc = __builtin_fmaf(w[4 * k + 3], xx.w, acc);
        }
    }
    return wave_sum(acc);
}

// Runtime type dispatch (the switch value is uniform across the wave).
__device__ __forceinline__ float row_dot_any(int t, const uint8_t *row, int64_t n_blocks, const float *x) {
    switch (t) {
    case ST_Q8_0: return row_dot_generic<ST_Q8_0>(row, n_blocks, x);
    case ST_Q2_K: return row_dot_generic<ST_Q2_K>(row, n_blocks, x);
    case ST_Q3_K: return row_dot_generic<ST_Q3_K>(row, n_blocks, x);
    case ST_Q4_K: return row_dot_generic<ST_Q4_K>(row, n_blocks, x);
    case ST_Q5_K: return row_dot_generic<ST_Q5_K>(row, n_blocks, x);
    case ST_Q6_K: return row_dot_generic<ST_Q6_K>(row, n_blocks, x);
    case ST_IQ2_XXS: return row_dot_generic<ST_IQ2_XXS>(row, n_blocks, x);
    case ST_IQ2_XS: return row_dot_generic<ST_IQ2_XS>(row, n_blocks, x);
    case ST_IQ3_XXS: return row_dot_generic<ST_IQ3_XXS>(row, n_blocks, x);
    case ST_IQ4_XS: return row_dot_generic<ST_IQ4_XS>(row, n_blocks, x);
    default: return 0.0f;
    }
}

// f32 row: float4 loads when the row and x are 16-byte aligned, scalars otherwise.
__device__ __forceinline__ float row_dot_f32(const float *__restrict__ w, const float *__restrict__ x, int64_t n) {
    const int lane = threadIdx.x & 63;
    float acc = 0.0f;
    if ((((uintptr_t)w | (uintptr_t)x) & 15) == 0) {
        const int64_t n4 = n >> 2;
        const float4 *w4 = (const float4 *)w, *x4 = (const float4 *)x;
        for (int64_t i = lane; i < n4; i += SEPIA_WAVE) {
            const float4 a = w4[i], b = x4[i];
            acc = __builtin_fmaf(a.x, b.x, acc);
            acc = __builtin_fmaf(a.y, b.y, acc);
            acc = __builtin_fmaf(a.z, b.z, acc);
            acc = __builtin_fmaf(a.w, b.w, acc);
        }
        for (int64_t i = (n4 << 2) + lane; i < n; i += SEPIA_WAVE) acc = __builtin_fmaf(w[i], x[i], acc);
    } else {
        for (int64_t i = lane; i < n; i += SEPIA_WAVE) acc = __builtin_fmaf(w[i], x[i], acc);
    }
    return wave_sum(acc);
}
