// synth.h -- seeded synthetic weights generated in place in HBM, so the
// benchmark's multi-GB expert sets never cross PCIe.
//
// sepia_synth_fill writes counter-based random bytes (splitmix64 of the
// seed and the word index). sepia_synth_patch_f16 then overwrites one f16
// field per block with a value uniform in [lo, hi], rounded to f16.
#pragma once
#include "common.h"

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

extern "C" __global__ __launch_bounds__(256) void sepia_synth_fill(
    uint8_t *__restrict__ base, uint64_t n_bytes, uint64_t seed) {
    const uint64_t n_words = n_bytes >> 2;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    uint32_t *w = (uint32_t *)base;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_words; i += stride)
        w[i] = (uint32_t)mix64(seed * 0x100000001B3ull + i);
    if (blockIdx.x == 0 && threadIdx.x < (n_bytes & 3))
        base[(n_words << 2) + threadIdx.x] = (uint8_t)mix64(seed * 0x100000001B3ull + n_words + threadIdx.x);
}

extern "C" __global__ __launch_bounds__(256) void sepia_synth_patch_f16(
    uint8_t *__restrict__ base, uint64_t n_blocks, uint32_t block_bytes, uint32_t field_off, uint64_t seed,
    float lo, float hi) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t b = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; b < n_blocks; b += stride) {
        const uint64_t r = mix64((seed ^ 0x5EEDull) * 0x9E3779B97F4A7C15ull + b);
        const float u = (float)(r >> 40) * (1.0f / 16777216.0f);
        const _Float16 v = (_Float16)(lo + u * (hi - lo));
        const uint16_t bits = __builtin_bit_cast(uint16_t, v);
        uint8_t *p = base + b * block_bytes + field_off;
        p[0] = (uint8_t)(bits & 0xFF);
        p[1] = (uint8_t)(bits >> 8);
    }
}
