// qdot.h -- integer dot products of quantized 64-weight units with x.
//
// x is carried as "x planes" (XP): per 16-column segment a scale
// xs = max|x over the segment| / 8355000 and, per column, the integer
// q = rint(x / xs), |q| <= 8355000 < 2^23, so x ~= xs * q. q is stored as its
// three low two's-complement bytes: plane 0 = byte 2 (read signed: q >> 16),
// plane 1 = byte 1 and plane 2 = byte 0 (read unsigned), so
// q = 65536 * p0 + 256 * p1 + p2 exactly. The rounding error of q is below
// 6e-8 of the segment's largest |x|, far inside the 1e-4 * ||y||_inf bar and
// inside the reference's per-element GPU gate (a 2^-16 representation,
// two planes, measured up to 7e-5 * ||y||_inf on these formats and is not).
// Each segment also carries the f32 sum of its 16 values (gs), used by the
// K-quant "min" and "-4" terms.
//
// Weights are small unsigned integers per 16-column segment (<= 15), so one
// segment's sum of w * q is exact in int32 (16 * 15 * 8355000 < 2^31): three
// v_dot4 chains over the planes (signed for p0, unsigned for p1, p2), shifted
// together in integers, converted to f32 once and scaled.
//
// XP layout for a vector of n columns (n a multiple of 16), in global memory
// or LDS: int8 planes[3][n] (plane-major), f32 xs[n / 16], f32 gs[n / 16].
//
// A unit is 64 weights of one block that the format stores together; its
// columns are four 16-column segments (seg_col). QU<T>::load fetches a unit's
// bytes for one row, QU<T>::dot returns its contribution to the row's dot
// product given the unit's planes XU.
#pragma once
#include "common.h"

#define XP_QMAX 8355000.0f

struct XU {
    uint32_t p[3][16];  // plane k, word 4*s + w = columns seg_col(s) + 4w .. + 3 (byte j = column + j)
    float xs[4];        // segment scales
    float gs[4];        // f32 sums of the segments
};

__device__ __forceinline__ int32_t dot_s8(uint32_t w, uint32_t x, int32_t acc) {
    return __builtin_amdgcn_sdot4((int32_t)w, (int32_t)x, acc, false);
}
__device__ __forceinline__ uint32_t dot_u8(uint32_t w, uint32_t x, uint32_t acc) {
    return __builtin_amdgcn_udot4(w, x, acc, false);
}

// sum over one segment (4 words of 4 weights, each byte 0..15) of w * q.
__device__ __forceinline__ int32_t seg_q(const uint32_t (&m)[4], const XU &x, int s) {
    int32_t a0 = 0;
    uint32_t a1 = 0, a2 = 0;
#pragma unroll
    for (int w = 0; w < 4; w++) {
        a0 = dot_s8(m[w], x.p[0][4 * s + w], a0);
        a1 = dot_u8(m[w], x.p[1][4 * s + w], a1);
        a2 = dot_u8(m[w], x.p[2][4 * s + w], a2);
    }
    return (int32_t)(((uint32_t)a0 << 16) + (a1 << 8) + a2);
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

template <int T> struct QU;

// ---------------------------------------------------------------- Q2_K
// Block {scales[16]@0, qs[64]@16, d@80, dmin@82}. Unit k = (h = k>>1, g = k&1):
// qs bytes 32h + 16g .. +15; bit pair s of qs byte (32h + 16g + i) is weight
// 128h + 32s + 16g + i, in group 8h + 2s + g whose scale byte holds
// (min << 4 | scale). Segment s = those 16 weights.
// y = d * sum_s scale_s * (q . x)_s - dmin * sum_s min_s * (sum x)_s.
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
        const uint32_t qw[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
        // scale byte of segment s is byte 2s + g of r.sc: bits 16*(s&1) of
        // (s < 2 ? r.sc.x : r.sc.y) >> 8g
        const uint32_t sh = 8u * (uint32_t)(k & 1);
        const uint32_t sa = r.sc.x >> sh, sb = r.sc.y >> sh;
        const uint32_t lo[2] = {sa & 0x000F000Fu, sb & 0x000F000Fu};
        const uint32_t hi[2] = {(sa >> 4) & 0x000F000Fu, (sb >> 4) & 0x000F000Fu};
        float acc = 0.0f, mn = 0.0f;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            uint32_t m[4];
#pragma unroll
            for (int w = 0; w < 4; w++) m[w] = (qw[w] >> (2 * s)) & 0x03030303u;
            const float t = (float)seg_q(m, x, s);
            const float scf = (float)((lo[s >> 1] >> (16 * (s & 1))) & 0xFFu);
            const float mnf = (float)((hi[s >> 1] >> (16 * (s & 1))) & 0xFFu);
            acc = __builtin_fmaf(t * x.xs[s], scf, acc);
            mn = __builtin_fmaf(mnf, x.gs[s], mn);
        }
        return __builtin_fmaf(half_lo(r.dd), acc, -(half_hi(r.dd) * mn));
    }
};

// ---------------------------------------------------------------- Q3_K
// Block {hmask[32]@0, qs[64]@32, scales[12]@96, d@108}; blocks are only
// 2-byte aligned (110 bytes). Unit k = (h, g) as Q2_K; weight
// 128h + 32s + 16g + i has low bits (qs[32h + 16g + i] >> 2s) & 3 and is
// lowered by 4 unless bit 4h + s of hmask[16g + i] is set. Scale j (6 bits,
// stored +32) of group 8h + 2s + g: bits 4h.. of byte (2s + g) give its low
// nibble, bits 2(2h + s/2).. of byte 8 + (2s + g) % 4 its top two bits.
// Each weight enters the integer dot as (q + 4) in 0..7; the -4 comes back
// through the segment sum: y = d * sum_s (sc_s - 32) * ((q+4) . x - 4 sum x)_s.
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
        const uint32_t h = (uint32_t)(k >> 1);
        const uint32_t base = 8u * (uint32_t)(k & 1) + 4u * h;
        const uint32_t qw[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
        // hmask bits 4h.. moved to bit 2 of each byte: << 2 for h = 0 (bits
        // 0..3 are needed, the top two that fall off are not), >> 2 for h = 1
        uint32_t hf[4];
        const uint32_t hmw[4] = {r.hm.x, r.hm.y, r.hm.z, r.hm.w};
#pragma unroll
        for (int w = 0; w < 4; w++) hf[w] = h ? (hmw[w] >> 2) : (hmw[w] << 2);
        float acc = 0.0f;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            uint32_t m[4];
#pragma unroll
            for (int w = 0; w < 4; w++)
                m[w] = ((qw[w] >> (2 * s)) & 0x03030303u) | ((hf[w] >> s) & 0x04040404u);
            const float t = (float)seg_q(m, x, s);
            const uint32_t lw = (s < 2) ? r.s0 : r.s1;
            const uint32_t low4 = __builtin_amdgcn_ubfe(lw, 16u * (s & 1) + base, 4u);
            const uint32_t top2 = __builtin_amdgcn_ubfe(r.s2, 16u * (s & 1) + 2u * (s >> 1) + base, 2u);
            const float scf = (float)((int32_t)(low4 | (top2 << 4)) - 32);
            acc = __builtin_fmaf(scf, __builtin_fmaf(-4.0f, x.gs[s], t * x.xs[s]), acc);
        }
        return half_lo(r.d) * acc;
    }
};

// ---------------------------------------------------------------- Q4_K
// Block {d@0, dmin@2, scales[12]@4, qs[128]@16}. Unit k = 64-weight chunk:
// low nibbles of qs[32k .. 32k+31] are sub-block 2k (columns 64k..64k+31),
// high nibbles sub-block 2k+1 (64k+32..64k+63); y = d*sc*q - dmin*m, with
// the 6-bit (sc, m) of sub-block j unpacked as reference src/quants.c:96-102.
template <> struct QU<ST_Q4_K> {
    static constexpr int bytes = 144;
    static constexpr int align = 4;
    struct Data { uint4 qa, qb; uint32_t dd, s0, s1, s2; };
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
    // (scale, min) of sub-block j = 2k + half. For j < 4 both are the low 6
    // bits of bytes j and j + 4; for j >= 4 (jj = j - 4) the low nibbles come
    // from byte 8 + jj and the top two bits from the top of bytes jj and jj + 4.
    __device__ static void scale_min(const Data &r, int k, int half, float &sc, float &mn) {
        const uint32_t hi = (uint32_t)(k >> 1);
        const uint32_t jj = (uint32_t)(2 * (k & 1) + half);
        const uint32_t wid = hi ? 4u : 6u, top = hi ? 2u : 0u;
        const uint32_t sl = __builtin_amdgcn_ubfe(hi ? r.s2 : r.s0, 8u * jj, wid);
        const uint32_t st = __builtin_amdgcn_ubfe(r.s0, 8u * jj + 6u, top);
        const uint32_t ml = __builtin_amdgcn_ubfe(hi ? r.s2 : r.s1, 8u * jj + 4u * hi, wid);
        const uint32_t mt = __builtin_amdgcn_ubfe(r.s1, 8u * jj + 6u, top);
        sc = (float)(sl | (st << 4));
        mn = (float)(ml | (mt << 4));
    }
    __device__ static float dot(const Data &r, int k, const XU &x) {
        const uint32_t qw[8] = {r.qa.x, r.qa.y, r.qa.z, r.qa.w, r.qb.x, r.qb.y, r.qb.z, r.qb.w};
        float acc = 0.0f, mn_acc = 0.0f;
#pragma unroll
        for (int half = 0; half < 2; half++) {
            float sub = 0.0f;
#pragma unroll
            for (int sg = 0; sg < 2; sg++) {   // the two segments of the sub-block
                const int s = 2 * half + sg;
                uint32_t m[4];
#pragma unroll
                for (int w = 0; w < 4; w++) m[w] = (qw[4 * sg + w] >> (4 * half)) & 0x0F0F0F0Fu;
                sub = __builtin_fmaf((float)seg_q(m, x, s), x.xs[s], sub);
            }
            float sc, mn;
            scale_min(r, k, half, sc, mn);
            acc = __builtin_fmaf(sc, sub, acc);
            mn_acc = __builtin_fmaf(mn, x.gs[2 * half] + x.gs[2 * half + 1], mn_acc);
        }
        return __builtin_fmaf(half_lo(r.dd), acc, -(half_hi(r.dd) * mn_acc));
    }
};

// Load a unit's planes (its four segments) from an XP array of n columns
// (global memory or LDS).
template <int T>
__device__ __forceinline__ void load_xu(const int8_t *planes, const float *xs, const float *gs, int64_t n,
                                        int64_t block, int k, XU &X) {
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const int64_t col = 256 * block + QU<T>::seg_col(k, s);
#pragma unroll
        for (int p = 0; p < 3; p++) {
            const uint4 v = *(const uint4 *)(planes + p * n + col);
            X.p[p][4 * s + 0] = v.x;
            X.p[p][4 * s + 1] = v.y;
            X.p[p][4 * s + 2] = v.z;
            X.p[p][4 * s + 3] = v.w;
        }
        X.xs[s] = xs[col >> 4];
        X.gs[s] = gs[col >> 4];
    }
}

// One segment (16 consecutive values) to XP form: the planes' 12 words, the
// scale and the f32 sum. v_perm gathers byte k of four q values into one word.
struct XSeg {
    uint4 p0, p1, p2;
    float xs, gs;
};
__device__ __forceinline__ XSeg xp_segment(const float4 (&v)[4]) {
    const float a[16] = {v[0].x, v[0].y, v[0].z, v[0].w, v[1].x, v[1].y, v[1].z, v[1].w,
                         v[2].x, v[2].y, v[2].z, v[2].w, v[3].x, v[3].y, v[3].z, v[3].w};
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) m = fmaxf(m, fabsf(a[i]));
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
    // a NaN or an infinity makes the scale infinite, so every dot that uses
    // the segment comes out non-finite, as the reference's double sum does
    if (!(s == s)) m = INFINITY;
    // |x| * inv <= 8355000 (1 + 2^-22) < 2^23: q fits 24 signed bits.
    // inv * xs = rcp(m) * m is 1 within 2^-22, so x ~= xs * q.
    const float inv = (m > 0.0f) ? XP_QMAX * __builtin_amdgcn_rcpf(m) : 0.0f;
    uint32_t q[16];
#pragma unroll
    for (int i = 0; i < 16; i++) q[i] = (uint32_t)(int32_t)__builtin_rintf(a[i] * inv);
    uint32_t w0[4], w1[4], w2[4];
#pragma unroll
    for (int w = 0; w < 4; w++) {
        // t01 = [q0.b0, q1.b0, q0.b1, q1.b1], t23 likewise; u = byte 2 of each
        const uint32_t t01 = __builtin_amdgcn_perm(q[4 * w + 1], q[4 * w], 0x05010400u);
        const uint32_t t23 = __builtin_amdgcn_perm(q[4 * w + 3], q[4 * w + 2], 0x05010400u);
        const uint32_t u01 = __builtin_amdgcn_perm(q[4 * w + 1], q[4 * w], 0x06020602u);
        const uint32_t u23 = __builtin_amdgcn_perm(q[4 * w + 3], q[4 * w + 2], 0x06020602u);
        w2[w] = __builtin_amdgcn_perm(t23, t01, 0x05040100u);   // byte 0 of q0..q3
        w1[w] = __builtin_amdgcn_perm(t23, t01, 0x07060302u);   // byte 1
        w0[w] = __builtin_amdgcn_perm(u23, u01, 0x05040100u);   // byte 2
    }
    XSeg r;
    r.p0 = make_uint4(w0[0], w0[1], w0[2], w0[3]);
    r.p1 = make_uint4(w1[0], w1[1], w1[2], w1[3]);
    r.p2 = make_uint4(w2[0], w2[1], w2[2], w2[3]);
    r.xs = m * (1.0f / XP_QMAX);
    r.gs = s;
    return r;
}

__device__ __forceinline__ void xp_store(const XSeg &r, int8_t *planes, float *xs, float *gs, int64_t n,
                                         int64_t seg) {
    *(uint4 *)(planes + 16 * seg) = r.p0;
    *(uint4 *)(planes + n + 16 * seg) = r.p1;
    *(uint4 *)(planes + 2 * n + 16 * seg) = r.p2;
    xs[seg] = r.xs;
    gs[seg] = r.gs;
}
