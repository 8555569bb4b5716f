// common.h -- device helpers shared by every sepia kernel (gfx950, wave64).
//
// The whole code object is compiled with -ffp-contract=off: products and
// sums round separately unless a kernel asks for a fused multiply-add
// explicitly with __builtin_fmaf. The dequantizers rely on that for bit
// exactness; the accumulating kernels use explicit FMAs.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define SEPIA_WAVE 64

// Type ids: the GGUF ggml_type enum (reference src/quants.h:6-10 plus Q2_K,
// Q3_K, IQ2_XXS from tools/gguf_inspect.py:62-84).
enum {
    ST_F32 = 0, ST_F16 = 1, ST_Q8_0 = 8, ST_Q2_K = 10, ST_Q3_K = 11, ST_Q4_K = 12,
    ST_Q5_K = 13, ST_Q6_K = 14, ST_IQ2_XXS = 16, ST_IQ2_XS = 17, ST_IQ3_XXS = 18, ST_IQ4_XS = 23,
};

__device__ __forceinline__ uint32_t ld_u8(const uint8_t *p) { return *p; }
__device__ __forceinline__ uint32_t ld_u16(const uint8_t *p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }
__device__ __forceinline__ uint32_t ld_u32(const uint8_t *p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

// binary16 -> binary32 through the hardware conversion: exact for every
// finite value and infinity (f16 subnormals become f32 normals).
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)h);
    return (float)v;
}

// binary16 -> binary32 with the integer recipe that also keeps NaN payloads
// unquieted (reference src/quants.c:58-77); used where the raw f16 value is
// the output (the F16 dequant), not for block scales.
__device__ __forceinline__ float f16_bits_to_f32_exact(uint32_t h) {
    uint32_t sign = (h >> 15) << 31;
    int32_t e = (h >> 10) & 31;
    uint32_t m = h & 0x3FFu, out;
    if (e == 31) {
        out = sign | 0x7F800000u | (m << 13);
    } else if (e != 0) {
        out = sign | ((uint32_t)(e + 112) << 23) | (m << 13);
    } else if (m == 0) {
        out = sign;
    } else {
        int32_t lz = __builtin_clz(m) - 21;      // shifts that bring bit 10 up
        out = sign | ((uint32_t)(113 - lz) << 23) | (((m << lz) & 0x3FFu) << 13);
    }
    return __builtin_bit_cast(float, out);
}

// Kernel entry: one scalar load from each 64-byte line of the first BYTES
// of the kernarg segment, all waited for at once. A kernel that reads its
// arguments lazily (inside branches, a few at a time) otherwise waits one
// memory round trip per dependent group of them, since the segment is not
// in the scalar cache when the kernel starts; afterwards those loads hit.
// BYTES must not exceed the kernel's kernarg segment.
template <int BYTES>
__device__ __forceinline__ void sepia_kernarg_warm() {
    const __attribute__((address_space(4))) uint32_t *ka =
        (const __attribute__((address_space(4))) uint32_t *)__builtin_amdgcn_kernarg_segment_ptr();
    uint32_t acc = 0;
#pragma unroll
    for (int o = 0; o < BYTES; o += 64) acc ^= ka[o / 4];
    asm volatile("" : : "s"(acc));
}

// Device error word and wait bound, set by the host when it loads the code
// object (sepia_hip.c): sepia_err_word points at a host-visible word that
// the host reads after each batch, sepia_wait_ticks bounds every spin wait
// of a kernel in s_memrealtime ticks (100 MHz). The whole library is one
// code object, so these are its only definitions.
// Both are constant memory: the kernels read them through the scalar cache.
// (As plain device globals the bound was a vector load in every spin of a
// wait, and under a launch's weight stream each such load took a loaded
// memory round trip, so a wave saw its counter reached that much later.)
extern "C" __constant__ uint32_t *sepia_err_word;
extern "C" __constant__ uint64_t sepia_wait_ticks;
// Record error `code` (first one wins) in *err, or in the device error word
// when err is NULL; lane 0 of the calling wave writes.
__device__ __forceinline__ void sepia_report_error(uint32_t *err, uint32_t code, int lane) {
    if (lane != 0) return;
    if (err) {
        __hip_atomic_store(err, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    uint32_t *w = sepia_err_word;
    if (w) {
        uint32_t zero = 0u;
        __hip_atomic_compare_exchange_strong(w, &zero, code, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

// Sum over the 64 lanes of a wave; every lane gets the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, SEPIA_WAVE);
    return v;
}

__device__ __forceinline__ float sigmoid_f32(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ __forceinline__ float silu_f32(float x) { return x * sigmoid_f32(x); }
