// qdot.h -- integer dot products of quantized 64-weight units with x.
//
// x is staged per workgroup as three signed int8 digit planes: within each
// 256-column block, x[c] ~= xs * (p0 * 65536 + p1 * 256 + p2), with
// xs = max|x| / 8355000 so that the digits stay within int8. The rounding
// error is below 6e-8 of the block's largest |x| -- far inside
// the 1e-4 * ||y||_inf bar (16-bit planes are not: up to 7e-5 measured on
// these formats) -- and the weight side is exact integers, so each unit's dot
// is formed exactly with v_dot4_i32_i8 (4 weights x 1 plane per instruction)
// and scaled once. The K-quant "min" terms use the exact f32 sums of x over
// 16-column groups, also staged per block.
//
// A unit is 64 weights of one block that the format stores together; its
// columns are four 16-column segments (seg_col). Each decoder loads a unit's
// bytes for one row (load) and returns its contribution to the row's dot
// (dot), given the unit's x planes XU.
#pragma once
#include "common.h"

struct XU {
    int32_t p[3][16];  // plane k, word 4*seg + w = columns seg_col(seg) + 4w .. + 3 (byte j = column +j)
    float gsum[4];     // f32 sum of x over each segment
    float xs;          // block scale
};

__device__ __forceinline__ int32_t sdot4(int32_t a, int32_t b, int32_t c) {
    return __builtin_amdgcn_sdot4(a, b, c, false);
}

__device__ __forceinline__ uint32_t ld32(const uint8_t *p) { return *(const uint32_t *)p; }
__device__ __forceinline__ uint2 ld64(const uint8_t *p) { return *(const uint2 *)p; }
__device__ __forceinline__ uint4 ld128(const uint8_t *p) { return *(const uint4 *)p; }

// 16 bytes at a 2-byte-aligned address, from naturally aligned dword loads
// (the address's low bits select the byte shift of v_alignbyte_b32).
__device__ __forceinline__ uint4 ld128_a2(const uint8_t *p) {
    const uint8_t *b = (const uint8_t *)((uintptr_t)p & ~(uintptr_t)3);
    const uint32_t sh = (uint32_t)((uintptr_t)p & 3);
    const uint4 a = *(const uint4 *)b;
    const uint32_t e = *(const uint32_t *)(b + 16);
    return make_uint4(__builtin_amdgcn_alignbyte(a.y, a.x, sh), __builtin_amdgcn_alignbyte(a.z, a.y, sh),
                      __builtin_amdgcn_alignbyte(a.w, a.z, sh), __builtin_amdgcn_alignbyte(e, a.w, sh));
}
__device__ __forceinline__ uint32_t ld32_a2(const uint8_t *p) {
    const uint8_t *b = (const uint8_t *)((uintptr_t)p & ~(uintptr_t)3);
    const uint32_t sh = (uint32_t)((uintptr_t)p & 3);
    return __builtin_amdgcn_alignbyte(*(const uint32_t *)(b + 4), *(const uint32_t *)b, sh);
}

__device__ __forceinline__ float half_lo(uint32_t v) { return f16_bits_to_f32(v & 0xFFFFu); }
__device__ __forceinline__ float half_hi(uint32_t v) { return f16_bits_to_f32(v >> 16); }

// Combine the three plane sums into f32: T0 * 65536 + T1 * 256 + T2.
__device__ __forceinline__ float planes_f(int32_t t0, int32_t t1, int32_t t2) {
    return __builtin_fmaf((float)t0, 65536.0f, __builtin_fmaf((float)t1, 256.0f, (float)t2));
}

template <int T> struct QU;

// ---------------------------------------------------------------- Q2_K
// Block {scales[16]@0, qs[64]@16, d@80, dmin@82}. Unit k = (h = k>>1, g = k&1):
// qs bytes 32h + 16g .. +15; bit pair s of qs byte (32h + 16g + i) is weight
// 128h + 32s + 16g + i, in group 8h + 2s + g whose scale byte holds
// (min << 4 | scale). Segment s = those 16 weights.
template <> struct QU<ST_Q2_K> {
    static constexpr int bytes = 84;
    struct Data { uint4 q; uint2 sc; uint32_t dd; };
    __device__ static int seg_col(int k, int s) { return 128 * (k >> 1) + 32 * s + 16 * (k & 1); }
    __device__ static Data load(const uint8_t *blk, int k) {
        Data r;
        r.q = ld128(blk + 16 + 16 * k);
        r.sc = ld64(blk + 8 * (k >> 1));
        r.dd = ld32(blk + 80);
        return r;
    }
    __device__ static float dot(const Data &r, int k, const XU &x) {
        const int g = k & 1;
        const uint32_t qw[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
        int32_t t0 = 0, t1 = 0, t2 = 0;
        float mn = 0.0f;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            int32_t a0 = 0, a1 = 0, a2 = 0;
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const int32_t m = (int32_t)((qw[w] >> (2 * s)) & 0x03030303u);
                a0 = sdot4(m, x.p[0][4 * s + w], a0);
                a1 = sdot4(m, x.p[1][4 * s + w], a1);
                a2 = sdot4(m, x.p[2][4 * s + w], a2);
            }
            const int bi = 2 * s + g;                                  // byte in r.sc
            const uint32_t scb = ((bi < 4 ? r.sc.x : r.sc.y) >> (8 * (bi & 3))) & 0xFFu;
            const int32_t sc = (int32_t)(scb & 15u);
            t0 += __mul24(sc, a0);
            t1 += __mul24(sc, a1);
            t2 += __mul24(sc, a2);
            mn = __builtin_fmaf((float)(scb >> 4), x.gsum[s], mn);
        }
        const float d = half_lo(r.dd), dmin = half_hi(r.dd);
        return __builtin_fmaf(d * x.xs, planes_f(t0, t1, t2), -(dmin * mn));
    }
};

// ---------------------------------------------------------------- Q3_K
// Block {hmask[32]@0, qs[64]@32, scales[12]@96, d@108}; blocks are only
// 2-byte aligned (110 bytes). Unit k = (h, g) as Q2_K; weight
// 128h + 32s + 16g + i has low bits (qs[32h + 16g + i] >> 2s) & 3 and is
// lowered by 4 unless bit 4h + s of hmask[16g + i] is set. Scale j (6 bits,
// stored +32) of group 8h + 2s + g: low nibble of byte j % 8 (j < 8) or its
// high nibble, top two bits from byte 8 + j % 4 at shift 2 * (j / 4).
template <> struct QU<ST_Q3_K> {
    static constexpr int bytes = 110;
    struct Data { uint4 q, hm; uint32_t s0, s1, s2, d; };
    __device__ static int seg_col(int k, int s) { return 128 * (k >> 1) + 32 * s + 16 * (k & 1); }
    __device__ static Data load(const uint8_t *blk, int k) {
        Data r;
        r.q = ld128_a2(blk + 32 + 16 * k);
        r.hm = ld128_a2(blk + 16 * (k & 1));
        const uint4 s = ld128_a2(blk + 96);   // scales[12] then d
        r.s0 = s.x;
        r.s1 = s.y;
        r.s2 = s.z;
        r.d = s.w;
        return r;
    }
    __device__ static float dot(const Data &r, int k, const XU &x) {
        const int h = k >> 1, g = k & 1;
        const uint32_t qw[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
        const uint32_t hw[4] = {r.hm.x, r.hm.y, r.hm.z, r.hm.w};
        int32_t t0 = 0, t1 = 0, t2 = 0;
        float sx = 0.0f;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            int32_t a0 = 0, a1 = 0, a2 = 0;
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const uint32_t lo = (qw[w] >> (2 * s)) & 0x03030303u;
                const uint32_t hb = (hw[w] >> (4 * h + s)) & 0x01010101u;
                const int32_t v = (int32_t)(lo | (hb << 2));            // q + 4, in 0..7
                a0 = sdot4(v, x.p[0][4 * s + w], a0);
                a1 = sdot4(v, x.p[1][4 * s + w], a1);
                a2 = sdot4(v, x.p[2][4 * s + w], a2);
            }
            const int j = 8 * h + 2 * s + g;
            const int jb = j & 7;
            const uint32_t lob = ((jb < 4 ? r.s0 : r.s1) >> (8 * (jb & 3))) & 0xFFu;
            const uint32_t nib = (j < 8) ? (lob & 15u) : (lob >> 4);
            const uint32_t top = (r.s2 >> (8 * (j & 3) + 2 * (j >> 2))) & 3u;
            const int32_t sc = (int32_t)(nib | (top << 4)) - 32;
            t0 += __mul24(sc, a0);
            t1 += __mul24(sc, a1);
            t2 += __mul24(sc, a2);
            sx = __builtin_fmaf((float)sc, x.gsum[s], sx);
        }
        const float d = half_lo(r.d);
        // sum (q + 4) x - 4 sum x, per group scale
        return d * __builtin_fmaf(x.xs, planes_f(t0, t1, t2), -4.0f * sx);
    }
};

// ---------------------------------------------------------------- Q4_K
// Block {d@0, dmin@2, scales[12]@4, qs[128]@16}. Unit k = 64-weight chunk:
// low nibbles of qs[32k .. 32k+31] are sub-block 2k (columns 64k..64k+31),
// high nibbles sub-block 2k+1 (64k+32..64k+63); y = d*sc*q - dmin*m.
template <> struct QU<ST_Q4_K> {
    static constexpr int bytes = 144;
    struct Data { uint4 qa, qb; uint32_t s0, s1, s2, dd; };
    __device__ static int seg_col(int k, int s) { return 64 * k + 16 * s; }
    __device__ static Data load(const uint8_t *blk, int k) {
        Data r;
        r.qa = ld128(blk + 16 + 32 * k);
        r.qb = ld128(blk + 32 + 32 * k);
        const uint4 h = ld128(blk);
        r.dd = h.x;
        r.s0 = h.y;
        r.s1 = h.z;
        r.s2 = h.w;
        return r;
    }
    // 6-bit (scale, min) of sub-block j from the packed bytes s[0..11].
    __device__ static void scale_min(const Data &r, int j, int32_t &sc, int32_t &mn) {
        const uint32_t b[3] = {r.s0, r.s1, r.s2};
        auto byte = [&](int i) -> uint32_t { return (b[i >> 2] >> (8 * (i & 3))) & 0xFFu; };
        if (j < 4) {
            sc = (int32_t)(byte(j) & 63u);
            mn = (int32_t)(byte(j + 4) & 63u);
        } else {
            sc = (int32_t)((byte(j + 4) & 15u) | ((byte(j - 4) >> 6) << 4));
            mn = (int32_t)((byte(j + 4) >> 4) | ((byte(j) >> 6) << 4));
        }
    }
    __device__ static float dot(const Data &r, int k, const XU &x) {
        const uint32_t qw[8] = {r.qa.x, r.qa.y, r.qa.z, r.qa.w, r.qb.x, r.qb.y, r.qb.z, r.qb.w};
        int32_t t0 = 0, t1 = 0, t2 = 0;
        float mn_acc = 0.0f;
#pragma unroll
        for (int half = 0; half < 2; half++) {
            int32_t a0 = 0, a1 = 0, a2 = 0;
#pragma unroll
            for (int w = 0; w < 8; w++) {
                const int32_t v = (int32_t)((qw[w] >> (4 * half)) & 0x0F0F0F0Fu);
                // sub-block half covers segments 2*half, 2*half+1: word w -> segment 2*half + w/4
                a0 = sdot4(v, x.p[0][8 * half + w], a0);
                a1 = sdot4(v, x.p[1][8 * half + w], a1);
                a2 = sdot4(v, x.p[2][8 * half + w], a2);
            }
            int32_t sc, mn;
            scale_min(r, 2 * k + half, sc, mn);
            t0 += __mul24(sc, a0);
            t1 += __mul24(sc, a1);
            t2 += __mul24(sc, a2);
            mn_acc = __builtin_fmaf((float)mn, x.gsum[2 * half] + x.gsum[2 * half + 1], mn_acc);
        }
        const float d = half_lo(r.dd), dmin = half_hi(r.dd);
        return __builtin_fmaf(d * x.xs, planes_f(t0, t1, t2), -(dmin * mn_acc));
    }
};
