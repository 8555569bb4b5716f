// qdot.h -- integer dot products of quantized 64-weight units with x.
//
// x is carried as "x planes" (XP): per 16-column segment, a scale xs and three
// signed int8 digit planes with x[c] ~= xs * (p0 * 65536 + p1 * 256 + p2),
// xs = max|x over the segment| / 8355000 so the digits stay within int8. The
// rounding error is below 6e-8 of the segment's largest |x|, far inside the
// 1e-4 * ||y||_inf bar (16-bit planes are not: up to 7e-5 measured on these
// formats). Each segment also carries its exact f32 sum, used by the
// K-quant "min" and "-4" terms. The weight side is exact integers, so a
// segment's dot is formed exactly with v_dot4_i32_i8 (4 weights x 1 plane per
// instruction) and scaled once.
//
// XP memory layout for a vector of n columns (n a multiple of 16), in global
// memory or LDS: int8 planes[3][n] (plane-major), float scale[n / 16],
// float sum[n / 16].
//
// A unit is 64 weights of one block that the format stores together; its
// columns are four 16-column segments (seg_col). Each decoder loads a unit's
// bytes for one row (load) and returns its contribution to the row's dot
// (dot), given the unit's x planes XU.
#pragma once
#include "common.h"

struct XU {
    int32_t p[3][16];  // plane k, word 4*seg + w = columns seg_col(seg) + 4w .. + 3 (byte j = column +j)
    float xs[4];       // segment scales
    float gsum[4];     // f32 sum of x over each segment
};

struct XPView {
    const int8_t *planes;  // [3][n]
    const float *scale;    // [n / 16]
    const float *sum;      // [n / 16]
    int64_t n;
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

__device__ __forceinline__ float half_lo(uint32_t v) { return f16_bits_to_f32(v & 0xFFFFu); }
__device__ __forceinline__ float half_hi(uint32_t v) { return f16_bits_to_f32(v >> 16); }

// xs * (a0 * 65536 + a1 * 256 + a2): one segment's dot in f32.
__device__ __forceinline__ float seg_f(int32_t a0, int32_t a1, int32_t a2, float xs) {
    return xs * __builtin_fmaf((float)a0, 65536.0f, __builtin_fmaf((float)a1, 256.0f, (float)a2));
}

template <int T> struct QU;

// ---------------------------------------------------------------- Q2_K
// Block {scales[16]@0, qs[64]@16, d@80, dmin@82}. Unit k = (h = k>>1, g = k&1):
// qs bytes 32h + 16g .. +15; bit pair s of qs byte (32h + 16g + i) is weight
// 128h + 32s + 16g + i, in group 8h + 2s + g whose scale byte holds
// (min << 4 | scale). Segment s = those 16 weights.
template <> struct QU<ST_Q2_K> {
    static constexpr int bytes = 84;
    static constexpr int align = 4;
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
        float acc = 0.0f, mn = 0.0f;
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
            acc = __builtin_fmaf((float)(scb & 15u), seg_f(a0, a1, a2, x.xs[s]), acc);
            mn = __builtin_fmaf((float)(scb >> 4), x.gsum[s], mn);
        }
        return __builtin_fmaf(half_lo(r.dd), acc, -(half_hi(r.dd) * mn));
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
    static constexpr int align = 2;
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
        float acc = 0.0f;
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
            const float sc = (float)((int32_t)(nib | (top << 4)) - 32);
            // sum over the group of (q + 4) x - 4 x
            acc = __builtin_fmaf(sc, __builtin_fmaf(-4.0f, x.gsum[s], seg_f(a0, a1, a2, x.xs[s])), acc);
        }
        return half_lo(r.d) * acc;
    }
};

// ---------------------------------------------------------------- Q4_K
// Block {d@0, dmin@2, scales[12]@4, qs[128]@16}. Unit k = 64-weight chunk:
// low nibbles of qs[32k .. 32k+31] are sub-block 2k (columns 64k..64k+31),
// high nibbles sub-block 2k+1 (64k+32..64k+63); y = d*sc*q - dmin*m.
template <> struct QU<ST_Q4_K> {
    static constexpr int bytes = 144;
    static constexpr int align = 4;
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
    // 6-bit (scale, min) of sub-block j from the packed bytes s[0..11]
    // (reference src/quants.c:115-121).
    __device__ static void scale_min(const Data &r, int j, uint32_t &sc, uint32_t &mn) {
        const uint32_t b[3] = {r.s0, r.s1, r.s2};
        auto byte = [&](int i) -> uint32_t { return (b[i >> 2] >> (8 * (i & 3))) & 0xFFu; };
        if (j < 4) {
            sc = byte(j) & 63u;
            mn = byte(j + 4) & 63u;
        } else {
            sc = (byte(j + 4) & 15u) | ((byte(j - 4) >> 6) << 4);
            mn = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
        }
    }
    __device__ static float dot(const Data &r, int k, const XU &x) {
        const uint32_t qw[8] = {r.qa.x, r.qa.y, r.qa.z, r.qa.w, r.qb.x, r.qb.y, r.qb.z, r.qb.w};
        float acc = 0.0f, mn_acc = 0.0f;
#pragma unroll
        for (int half = 0; half < 2; half++) {
            float sub = 0.0f;
#pragma unroll
            for (int sg = 0; sg < 2; sg++) {       // the two segments of the sub-block
                int32_t a0 = 0, a1 = 0, a2 = 0;
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    const int32_t v = (int32_t)((qw[4 * sg + w] >> (4 * half)) & 0x0F0F0F0Fu);
                    const int xi = 8 * half + 4 * sg + w;
                    a0 = sdot4(v, x.p[0][xi], a0);
                    a1 = sdot4(v, x.p[1][xi], a1);
                    a2 = sdot4(v, x.p[2][xi], a2);
                }
                sub += seg_f(a0, a1, a2, x.xs[2 * half + sg]);
            }
            uint32_t sc, mn;
            scale_min(r, 2 * k + half, sc, mn);
            acc = __builtin_fmaf((float)sc, sub, acc);
            mn_acc = __builtin_fmaf((float)mn, x.gsum[2 * half] + x.gsum[2 * half + 1], mn_acc);
        }
        return __builtin_fmaf(half_lo(r.dd), acc, -(half_hi(r.dd) * mn_acc));
    }
};

// Load a unit's x planes (its four segments) from an XP array.
template <int T>
__device__ __forceinline__ void load_xu(const XPView &xp, int64_t block, int k, XU &X) {
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const int64_t col = 256 * block + QU<T>::seg_col(k, s);
#pragma unroll
        for (int p = 0; p < 3; p++) {
            const int4 v = *(const int4 *)(xp.planes + p * xp.n + col);
            X.p[p][4 * s + 0] = v.x;
            X.p[p][4 * s + 1] = v.y;
            X.p[p][4 * s + 2] = v.z;
            X.p[p][4 * s + 3] = v.w;
        }
        X.xs[s] = xp.scale[col >> 4];
        X.gsum[s] = xp.sum[col >> 4];
    }
}

// Convert 4 consecutive values (one quad; 4 quads = one segment, held by 4
// consecutive lanes) to XP form: the lanes of a segment agree on its scale
// through two shuffles. Writes plane bytes at columns 4q .. 4q+3 and, from
// the segment's first lane, its scale and sum.
__device__ __forceinline__ void xp_quad(float4 v, int64_t q, int8_t *planes, float *scale, float *sum, int64_t n) {
    float m = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    m = fmaxf(m, __shfl_xor(m, 1, SEPIA_WAVE));
    m = fmaxf(m, __shfl_xor(m, 2, SEPIA_WAVE));
    // |x| * inv <= 8355000 (1 + 2^-22) < 127 * (65536 + 256 + 1): three balanced
    // int8 digits. inv * scale = rcp(m) * m is 1 within 2^-22, so x ~= scale * q.
    const float inv = (m > 0.0f) ? 8355000.0f * __builtin_amdgcn_rcpf(m) : 0.0f;
    const float vals[4] = {v.x, v.y, v.z, v.w};
    uint32_t w0 = 0, w1 = 0, w2 = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int32_t qv = (int32_t)__builtin_rintf(vals[i] * inv);
        const int32_t lo = (int32_t)(int8_t)qv;      // balanced base-256 digits
        const int32_t r1 = (qv - lo) >> 8;
        const int32_t mid = (int32_t)(int8_t)r1;
        const int32_t hi = (r1 - mid) >> 8;
        w0 |= ((uint32_t)hi & 0xFFu) << (8 * i);
        w1 |= ((uint32_t)mid & 0xFFu) << (8 * i);
        w2 |= ((uint32_t)lo & 0xFFu) << (8 * i);
    }
    *(uint32_t *)(planes + 4 * q) = w0;
    *(uint32_t *)(planes + n + 4 * q) = w1;
    *(uint32_t *)(planes + 2 * n + 4 * q) = w2;
    float s = (v.x + v.y) + (v.z + v.w);
    s += __shfl_xor(s, 1, SEPIA_WAVE);
    s += __shfl_xor(s, 2, SEPIA_WAVE);
    if ((q & 3) == 0) {
        scale[q >> 2] = m * (1.0f / 8355000.0f);
        sum[q >> 2] = s;
    }
}
