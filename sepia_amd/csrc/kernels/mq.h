// mq.h -- quantized matvecs at decode batch 1 on the matrix cores.
//
// The dot products of quantized rows with x run as exact integer products
// on v_mfma_i32_16x16x64_i8; only the unpacking of the packed weights into
// int8 bytes and the per-segment scale arithmetic stay on the VALU, about
// one VALU instruction per weight instead of the three to five a v_dot4
// formulation needs for the same precision.
//
// x (or h) travels as "XQ" digit planes: per 16-column segment a scale
// xs = max|x| / MQ_QMAX, per column the integer q = round(x / xs) with
// |q| <= MQ_QMAX + 1 < 2^23 - 0x8080, written as three signed base-256
// digits q = 65536 * p0 + 256 * p1 + p2 (p0, p1, p2 in [-128, 127]), so
// x^ = xs * q is within xs / 2 + 2^-22 |x| of x: a 23-bit representation
// relative to the segment's largest |x|. Per segment two sums feed the
// formats' offset terms: gs = sum(x) (exact f32) and gq = xs * sum(q) (the
// sum of x^). A format whose weights are w = a * q - b (K-quant "min")
// uses gs, so the error is sum(a * q * (x^ - x)); one whose offset is part
// of the weight itself (Q3_K's -4) uses gq, so the error is
// sum(w * (x^ - x)) with the true weights.
// XQ layout for n columns: int8 planes[3][n] | f32 xs, gs, gq [n / 16 each].
//
// MFMA mapping. Lane l of a wave is (row j = l & 15, unit g = l >> 4): it
// holds the 64 weights that unit g of the current block stores together
// (format-specific, see MQ<T>::seg_col) for row r0 + j. A unit is four
// 16-weight segments s. For segment s the lane's 16 int8 weights form its
// B operand (B[k = 16g + t][j]); the A operand holds, on lane 20g + p
// (p < 3), digit plane p of the x columns of unit g's segment s and zero on
// every other lane, so D[4g + p][j] = sum_t w_t * p_p(x_t): the three plane
// dots of (row j, unit g, segment s) land in VGPRs 0..2 of lane l itself.
// Four MFMAs cover a block of 16 rows; no data crosses lanes until the final
// row sums.
#pragma once
#include "common.h"

typedef int32_t mq_v4i __attribute__((ext_vector_type(4)));

// |q| + 0x8080 < 2^23, so q + 0x8080 splits into signed byte 2 and
// offset bytes 1 and 0 (below); and 16 * 15 * (QMAX + 1) < 2^31, so one
// segment's integer dot cannot overflow.
#define MQ_QMAX 8355000.0f

// Bytes of an XQ vector of n columns, rounded up to 16 so that it copies in
// 16-byte pieces (the xs/gs/gq tail is 3n / 4 bytes).
__device__ __forceinline__ size_t mq_xq_bytes(int64_t n) { return ((size_t)(3 * n + 3 * (n / 16) * 4) + 15) & ~(size_t)15; }

// ------------------------------------------------------------ x -> XQ ----
// q + 0x8080 = 65536 * p0 + 256 * (p1 + 128) + (p2 + 128): byte 2 of it is
// p0 (two's complement), bytes 1 and 0 are p1 + 128 and p2 + 128, so
// p1, p2 = byte ^ 0x80. round(): v_rndne_f32 + v_cvt_i32_f32.
__device__ __forceinline__ int32_t mq_round(float v) { return (int32_t)__builtin_rintf(v); }

struct XqSeg {
    uint4 p0, p1, p2;
    float xs, gs, gq;
};
__device__ __forceinline__ XqSeg xq_segment(const float (&a)[16]) {
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) m = fmaxf(m, fabsf(a[i]));
    // |a * inv| <= QMAX (1 + 2^-22): rcp is within 1 ulp
    const float inv = (m > 0.0f) ? MQ_QMAX * __builtin_amdgcn_rcpf(m) : 0.0f;
    const float xs = m * (1.0f / MQ_QMAX);
    uint32_t q[16];
    int32_t qs = 0;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int32_t v = mq_round(a[i] * inv);
        qs += v;
        q[i] = (uint32_t)v + 0x8080u;
    }
    uint32_t w0[4], w1[4], w2[4];
#pragma unroll
    for (int w = 0; w < 4; w++) {
        // t01 = [q0.b0, q1.b0, q0.b1, q1.b1], t23 likewise; u = byte 2 of each
        const uint32_t t01 = __builtin_amdgcn_perm(q[4 * w + 1], q[4 * w], 0x05010400u);
        const uint32_t t23 = __builtin_amdgcn_perm(q[4 * w + 3], q[4 * w + 2], 0x05010400u);
        const uint32_t u01 = __builtin_amdgcn_perm(q[4 * w + 1], q[4 * w], 0x06020602u);
        const uint32_t u23 = __builtin_amdgcn_perm(q[4 * w + 3], q[4 * w + 2], 0x06020602u);
        w2[w] = __builtin_amdgcn_perm(t23, t01, 0x05040100u) ^ 0x80808080u;   // byte 0: p2 + 128
        w1[w] = __builtin_amdgcn_perm(t23, t01, 0x07060302u) ^ 0x80808080u;   // byte 1: p1 + 128
        w0[w] = __builtin_amdgcn_perm(u23, u01, 0x05040100u);                 // byte 2: p0
    }
    XqSeg r;
    r.p0 = make_uint4(w0[0], w0[1], w0[2], w0[3]);
    r.p1 = make_uint4(w1[0], w1[1], w1[2], w1[3]);
    r.p2 = make_uint4(w2[0], w2[1], w2[2], w2[3]);
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) sum += a[i];
    r.xs = xs;
    r.gs = sum;
    r.gq = xs * (float)qs;
    return r;
}

__device__ __forceinline__ void xq_store(const XqSeg &r, uint8_t *xq, int64_t n, int64_t seg) {
    *(uint4 *)(xq + 16 * seg) = r.p0;
    *(uint4 *)(xq + n + 16 * seg) = r.p1;
    *(uint4 *)(xq + 2 * n + 16 * seg) = r.p2;
    float *xs = (float *)(xq + 3 * n);
    xs[seg] = r.xs;
    xs[n / 16 + seg] = r.gs;
    xs[n / 8 + seg] = r.gq;
}

// ------------------------------------------------------- weight units ----
__device__ __forceinline__ uint32_t mq_ld32(const uint8_t *p) { return *(const uint32_t *)p; }
__device__ __forceinline__ uint2 mq_ld64(const uint8_t *p) { return *(const uint2 *)p; }
__device__ __forceinline__ uint4 mq_ld128(const uint8_t *p) { return *(const uint4 *)p; }
// 16 bytes at a 2-byte-aligned address from naturally aligned loads (the
// address's low bits give the v_alignbyte shift); reads up to 4 bytes past
// the 16, which the library's allocation padding covers.
__device__ __forceinline__ uint4 mq_ld128_a2(const uint8_t *p) {
    const uint32_t sh = (uint32_t)((uintptr_t)p & 3);
    const uint8_t *b = p - sh;
    const uint4 a = *(const uint4 *)b;
    const uint32_t e = *(const uint32_t *)(b + 16);
    return make_uint4(__builtin_amdgcn_alignbyte(a.y, a.x, sh), __builtin_amdgcn_alignbyte(a.z, a.y, sh),
                      __builtin_amdgcn_alignbyte(a.w, a.z, sh), __builtin_amdgcn_alignbyte(e, a.w, sh));
}
__device__ __forceinline__ float mq_half_lo(uint32_t v) { return f16_bits_to_f32(v & 0xFFFFu); }
__device__ __forceinline__ float mq_half_hi(uint32_t v) { return f16_bits_to_f32(v >> 16); }
// Byte b of v as a float: one v_cvt_f32_ubyte<b> (the compiler otherwise
// folds a preceding mask into a v_bfe and converts byte 0). The operand is
// an ordinary VALU result, never an MFMA result (inline asm is invisible to
// the compiler's MFMA hazard recognizer).
template <int B>
__device__ __forceinline__ float mq_ubyte(uint32_t v) {
    float r;
    if constexpr (B == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(v));
    else if constexpr (B == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(v));
    else if constexpr (B == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(v));
    else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(v));
    return r;
}
// (p0 << 16) + (p1 << 8) + p2 of one segment's three plane dots: the exact
// integer sum of w * q (|.| < 2^31 for 16 weights <= 15 and |q| <= QMAX + 1).
// Plain C on purpose: the operands are MFMA results, and only the compiler's
// hazard recognizer inserts the wait states a VALU read of them needs.
__device__ __forceinline__ float mq_combine(const mq_v4i &d) {
    const uint32_t t = ((uint32_t)d[0] << 8) + (uint32_t)d[1];
    return (float)(int32_t)((t << 8) + (uint32_t)d[2]);
}

// One lane's raw bytes of one block (its unit g): three 16-byte words, used
// as each format needs. One container for all formats, so a pipeline can
// switch formats between iterations.
struct MqRaw {
    uint4 a, b, c;
};

template <int T> struct MQ;

// ---------------------------------------------------------------- Q2_K
// Block {scales[16]@0, qs[64]@16, d@80, dmin@82} (ggml block_q2_K). Unit
// g = (h = g >> 1, g' = g & 1): qs bytes 32h + 16g' + i, i < 16; bit pair s
// of that byte is the weight of column 128h + 32s + 16g' + i, in group
// 8h + 2s + g' whose scale byte holds (min << 4 | scale).
// Row contribution: d * sum_s sc_s (q . x)_s - dmin * sum_s m_s (sum x)_s.
// Raw: a = qs bytes of the unit, b.xy = scale bytes 8h .. 8h+7, b.z = d|dmin.
template <> struct MQ<ST_Q2_K> {
    static constexpr int bytes = 84;
    static constexpr int seg_step = 2;   // segment index step between s and s + 1
    static constexpr int sum_sel = 1;    // offset terms use gs (exact sums)
    __device__ static int seg_col(int g, int s) { return 128 * (g >> 1) + 32 * s + 16 * (g & 1); }
    __device__ static void load(const uint8_t *blk, int g, MqRaw &r) {
        r.a = mq_ld128(blk + 16 + 16 * g);
        const uint2 sc = mq_ld64(blk + 8 * (g >> 1));
        r.b.x = sc.x;
        r.b.y = sc.y;
        r.b.z = mq_ld32(blk + 80);
    }
    // Segment s: s = 0 mask 0x03, s = 1 mask 0x0C (4 q), s = 2 and 3 the same
    // on q >> 4 -- so segments 1 and 3 enter the MFMA scaled by 4.
    __device__ static mq_v4i bop(const MqRaw &r, int, int s) {
        const uint32_t m = (s & 1) ? 0x0C0C0C0Cu : 0x03030303u;
        const uint32_t sh = (s & 2) ? 4u : 0u;
        return mq_v4i{(int32_t)((r.a.x >> sh) & m), (int32_t)((r.a.y >> sh) & m), (int32_t)((r.a.z >> sh) & m),
                      (int32_t)((r.a.w >> sh) & m)};
    }
    __device__ static float finish(const MqRaw &r, int g, const mq_v4i (&D)[4], const float (&xs)[4],
                                   const float (&gv)[4]) {
        // scale bytes 2s + g' of the half's 8 bytes, gathered in s order
        const uint32_t sb = __builtin_amdgcn_perm(r.b.y, r.b.x, (g & 1) ? 0x07050301u : 0x06040200u);
        const uint32_t scw = sb & 0x0F0F0F0Fu, mw = (sb >> 4) & 0x0F0F0F0Fu;
        const float a1 = __builtin_fmaf(mq_combine(D[0]), mq_ubyte<0>(scw) * xs[0],
                                        mq_combine(D[2]) * (mq_ubyte<2>(scw) * xs[2]));
        const float a4 = __builtin_fmaf(mq_combine(D[1]), mq_ubyte<1>(scw) * xs[1],
                                        mq_combine(D[3]) * (mq_ubyte<3>(scw) * xs[3]));
        const float acc = __builtin_fmaf(0.25f, a4, a1);
        float mn = mq_ubyte<0>(mw) * gv[0];
        mn = __builtin_fmaf(mq_ubyte<1>(mw), gv[1], mn);
        mn = __builtin_fmaf(mq_ubyte<2>(mw), gv[2], mn);
        mn = __builtin_fmaf(mq_ubyte<3>(mw), gv[3], mn);
        return __builtin_fmaf(mq_half_lo(r.b.z), acc, -(mq_half_hi(r.b.z) * mn));
    }
};

// ---------------------------------------------------------------- Q3_K
// Block {hmask[32]@0, qs[64]@32, scales[12]@96, d@108}; only 2-byte
// aligned. Unit g = (h, g') as Q2_K: weight 128h + 32s + 16g' + i has low
// bits (qs[32h + 16g' + i] >> 2s) & 3 and is lowered by 4 unless bit 4h + s
// of hmask[16g' + i] is set; its group 8h + 2s + g' has a 6-bit scale stored
// +32 (low nibble in bytes 0..7, top two bits in bytes 8..11, ggml's
// kmask1/kmask2 packing). The B operand holds q + 4 * hbit in 0..7; the -4
// returns through the segment sum:
// contribution = d * sum_s (sc_s - 32) * ((q + 4 hbit) . x^ - 4 sum x^)_s.
// Raw: a = qs bytes, b = hmask bytes, c = scales[12] then d.
template <> struct MQ<ST_Q3_K> {
    static constexpr int bytes = 110;
    static constexpr int seg_step = 2;
    static constexpr int sum_sel = 2;    // the -4 is part of the weight: gq
    __device__ static int seg_col(int g, int s) { return 128 * (g >> 1) + 32 * s + 16 * (g & 1); }
    __device__ static void load(const uint8_t *blk, int g, MqRaw &r) {
        r.a = mq_ld128_a2(blk + 32 + 16 * g);
        r.b = mq_ld128_a2(blk + 16 * (g & 1));
        r.c = mq_ld128_a2(blk + 96);
    }
    __device__ static mq_v4i bop(const MqRaw &r, int g, int s) {
        // hmask bits 4h.. moved to bit 2: << 2 for h = 0, >> 2 for h = 1
        const bool h = (g >> 1) != 0;
        const uint32_t qw[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
        const uint32_t hw[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
        mq_v4i b;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const uint32_t hf = h ? (hw[w] >> 2) : (hw[w] << 2);
            b[w] = (int32_t)(((qw[w] >> (2 * s)) & 0x03030303u) | ((hf >> s) & 0x04040404u));
        }
        return b;
    }
    __device__ static float finish(const MqRaw &r, int g, const mq_v4i (&D)[4], const float (&xs)[4],
                                   const float (&gv)[4]) {
        const uint32_t base = 8u * (uint32_t)(g & 1) + 4u * (uint32_t)(g >> 1);
        float acc = 0.0f;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const uint32_t lw = (s < 2) ? r.c.x : r.c.y;
            const uint32_t low4 = __builtin_amdgcn_ubfe(lw, 16u * (s & 1) + base, 4u);
            const uint32_t top2 = __builtin_amdgcn_ubfe(r.c.z, 16u * (s & 1) + 2u * (s >> 1) + base, 2u);
            const float scf = (float)((int32_t)(low4 | (top2 << 4)) - 32);
            acc = __builtin_fmaf(scf, __builtin_fmaf(-4.0f, gv[s], mq_combine(D[s]) * xs[s]), acc);
        }
        return mq_half_lo(r.c.w) * acc;
    }
};

// ---------------------------------------------------------------- Q4_K
// Block {d@0, dmin@2, scales[12]@4, qs[128]@16}. Unit g = 64-weight chunk:
// low nibbles of qs[32g .. 32g+31] are sub-block 2g (columns 64g .. 64g+31),
// high nibbles sub-block 2g+1 (64g+32 .. 64g+63). Segment s: s = 0 low
// nibbles of bytes 0..15, s = 1 low of 16..31, s = 2 high of 0..15, s = 3
// high of 16..31. y = d*sc*q - dmin*m with the 6-bit (sc, m) of sub-block j
// unpacked as reference src/quants.c:96-102.
// Raw: a, b = qs bytes 32g .. +15, +16 .. +31; c = d|dmin, scales[12].
template <> struct MQ<ST_Q4_K> {
    static constexpr int bytes = 144;
    static constexpr int seg_step = 1;
    static constexpr int sum_sel = 1;
    __device__ static int seg_col(int g, int s) { return 64 * g + 16 * s; }
    __device__ static void load(const uint8_t *blk, int g, MqRaw &r) {
        r.a = mq_ld128(blk + 16 + 32 * g);
        r.b = mq_ld128(blk + 32 + 32 * g);
        r.c = mq_ld128(blk);
    }
    __device__ static mq_v4i bop(const MqRaw &r, int, int s) {
        const uint4 q = (s & 1) ? r.b : r.a;
        const uint32_t sh = (s & 2) ? 4u : 0u, m = 0x0F0F0F0Fu;
        return mq_v4i{(int32_t)((q.x >> sh) & m), (int32_t)((q.y >> sh) & m), (int32_t)((q.z >> sh) & m),
                      (int32_t)((q.w >> sh) & m)};
    }
    // (scale, min) of sub-block j = 2g + half. For j < 4 both are the low 6
    // bits of bytes j and j + 4; for j >= 4 (jj = j - 4) the low nibbles come
    // from byte 8 + jj and the top two bits from the top of bytes jj, jj + 4.
    __device__ static void scale_min(const MqRaw &r, int g, int half, float &sc, float &mn) {
        const uint32_t hi = (uint32_t)(g >> 1);
        const uint32_t jj = (uint32_t)(2 * (g & 1) + half);
        const uint32_t wid = hi ? 4u : 6u, top = hi ? 2u : 0u;
        const uint32_t s0 = r.c.y, s1 = r.c.z, s2 = r.c.w;
        const uint32_t sl = __builtin_amdgcn_ubfe(hi ? s2 : s0, 8u * jj, wid);
        const uint32_t st = __builtin_amdgcn_ubfe(s0, 8u * jj + 6u, top);
        const uint32_t ml = __builtin_amdgcn_ubfe(hi ? s2 : s1, 8u * jj + 4u * hi, wid);
        const uint32_t mt = __builtin_amdgcn_ubfe(s1, 8u * jj + 6u, top);
        sc = (float)(sl | (st << 4));
        mn = (float)(ml | (mt << 4));
    }
    __device__ static float finish(const MqRaw &r, int g, const mq_v4i (&D)[4], const float (&xs)[4],
                                   const float (&gv)[4]) {
        float sc0, mn0, sc1, mn1;
        scale_min(r, g, 0, sc0, mn0);
        scale_min(r, g, 1, sc1, mn1);
        const float sub0 = __builtin_fmaf(mq_combine(D[0]), xs[0], mq_combine(D[1]) * xs[1]);
        const float sub1 = __builtin_fmaf(mq_combine(D[2]), xs[2], mq_combine(D[3]) * xs[3]);
        const float acc = __builtin_fmaf(sc0, sub0, sc1 * sub1);
        const float mn = __builtin_fmaf(mn0, gv[0] + gv[1], mn1 * (gv[2] + gv[3]));
        return __builtin_fmaf(mq_half_lo(r.c.x), acc, -(mq_half_hi(r.c.x) * mn));
    }
};

// Format dispatch for loads (the type is uniform across the workgroup).
__device__ __forceinline__ void mq_load_any(int type, const uint8_t *blk, int g, MqRaw &r) {
    if (type == ST_Q2_K) MQ<ST_Q2_K>::load(blk, g, r);
    else if (type == ST_Q3_K) MQ<ST_Q3_K>::load(blk, g, r);
    else MQ<ST_Q4_K>::load(blk, g, r);
}
__device__ __forceinline__ int mq_bytes_any(int type) {
    return type == ST_Q2_K ? 84 : (type == ST_Q3_K ? 110 : 144);
}

// ---------------------------------------------------- one block, 16 rows ---
// Lane roles: g = unit, a_lane carries A-operand data (lane 20g + p, p < 3).
struct MqLane {
    int lane, g, p;
    bool a_lane;
};
__device__ __forceinline__ MqLane mq_lane() {
    MqLane r;
    r.lane = threadIdx.x & 63;
    r.g = r.lane >> 4;
    r.p = r.lane & 3;
    r.a_lane = ((r.lane & 15) >> 2) == r.g && r.p < 3;
    return r;
}
__device__ __forceinline__ int mq_wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// Contribution of block b of the lane's row (unit g) against an XQ vector
// of n columns in LDS at xq. A operands: every lane reads 16 bytes per
// segment -- lanes 20g + p digit plane p of unit g's segment, all other
// lanes a 128-byte zero area (zoff, a byte offset from xq's LDS base lds0),
// so no lane needs masking and no register needs re-zeroing.
template <int T>
__device__ __forceinline__ float mq_block(const MqRaw &raw, int g, int b, const uint8_t *lds0, uint32_t xoff, int n,
                                          bool a_lane, int p, uint32_t zoff) {
    const uint32_t col0 = 256u * (uint32_t)b + (uint32_t)MQ<T>::seg_col(g, 0);
    const uint32_t abase = a_lane ? xoff + (uint32_t)(p * n) + col0 : zoff;
    const float *xs = (const float *)(lds0 + xoff + 3u * (uint32_t)n) + (col0 >> 4);
    const float *gv = xs + MQ<T>::sum_sel * (n / 16);
    float xsv[4], gvv[4];
#pragma unroll
    for (int s = 0; s < 4; s++) {
        xsv[s] = xs[MQ<T>::seg_step * s];
        gvv[s] = gv[MQ<T>::seg_step * s];
    }
    // two segments at a time: half the A and D registers live at once
    mq_v4i D[4];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        mq_v4i A[2];
#pragma unroll
        for (int s = 0; s < 2; s++)
            A[s] = *(const mq_v4i *)(lds0 + abase +
                                     (uint32_t)(MQ<T>::seg_col(g, 2 * h + s) - MQ<T>::seg_col(g, 0)));
#pragma unroll
        for (int s = 0; s < 2; s++)
            D[2 * h + s] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[s], MQ<T>::bop(raw, g, 2 * h + s),
                                                                 mq_v4i{0, 0, 0, 0}, 0, 0, 0);
    }
    return MQ<T>::finish(raw, g, D, xsv, gvv);
}
__device__ __forceinline__ float mq_block_any(int type, const MqRaw &raw, int g, int b, const uint8_t *lds0,
                                              uint32_t xoff, int n, bool a_lane, int p, uint32_t zoff) {
    if (type == ST_Q2_K) return mq_block<ST_Q2_K>(raw, g, b, lds0, xoff, n, a_lane, p, zoff);
    if (type == ST_Q3_K) return mq_block<ST_Q3_K>(raw, g, b, lds0, xoff, n, a_lane, p, zoff);
    return mq_block<ST_Q4_K>(raw, g, b, lds0, xoff, n, a_lane, p, zoff);
}

// Row sum over the four unit lanes (l, l + 16, l + 32, l + 48) of a wave.
__device__ __forceinline__ float mq_sum_units(float v) {
    v += __shfl_xor(v, 16, SEPIA_WAVE);
    v += __shfl_xor(v, 32, SEPIA_WAVE);
    return v;
}

// ---- f32 vectors -> XQ in LDS, by the whole workgroup: `count` vectors of
// n columns (vector k at src + k * ld floats) to LDS offsets xoff + k * xqb.
// Each thread converts whole 16-column segments. Also writes the 128-byte
// zero area for the A operands; ends with a barrier.
__device__ __forceinline__ void mq_stage_xq(const float *__restrict__ src, int64_t ld, int count, int n,
                                            uint8_t *lds0, uint32_t xoff, uint32_t xqb) {
    const int segs = n >> 4, total = segs * count;
    for (int i = threadIdx.x; i < total; i += blockDim.x) {
        const int k = i / segs, seg = i - k * segs;
        const float4 *x4 = (const float4 *)(src + (int64_t)k * ld) + 4 * seg;
        const float4 v0 = x4[0], v1 = x4[1], v2 = x4[2], v3 = x4[3];
        const float a[16] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w,
                             v2.x, v2.y, v2.z, v2.w, v3.x, v3.y, v3.z, v3.w};
        xq_store(xq_segment(a), lds0 + xoff + (uint32_t)k * xqb, n, seg);
    }
    if (threadIdx.x < 8) ((uint4 *)(lds0))[threadIdx.x] = make_uint4(0, 0, 0, 0);
    __syncthreads();
}

// Pipelines. Every step issues exactly the same loads (tail blocks of a
// wave's chunk load a valid block again and are not computed), and the
// step that prefetches never shares a code path with the last step: the
// compiler's wait-count insertion can then wait for the current step's
// loads only, leaving the next step's in flight.

// ------------------------------------------------------------ matvec ------
// y = W x for one matrix. A workgroup of nw waves covers a row's nb blocks,
// CH per wave (wave w: blocks [w * CH, w * CH + CH)), and walks row groups
// of 16 rows rg = blockIdx.x, + gridDim.x, ...: the loads of the next row
// group are issued before the current one is computed (two register
// stages), so every wave keeps one row group of weights in flight. The
// results collect in LDS and are stored after the last row group: a
// global store inside the loop would hold the issuing wave's next waits
// (vmcnt retires stores and loads in issue order) and, through the
// barrier, every wave.
// LDS: [128-byte zero area][XQ of x][2 x nw x 16 f32 row partials]
//      [nk x 16 f32 results].
template <int T, int CH>
struct MqMv {
    const uint8_t *W;
    uint64_t row_bytes;
    int64_t rows;
    int32_t nb, n, tiles;
    float *y;
    uint8_t *lds0;
    float *red, *res;
    MqLane L;
    int wave, nw, b0, nblk;

    __device__ __forceinline__ void load(int64_t rg, MqRaw (&raw)[CH]) const {
        int64_t row = rg * 16 + (L.lane & 15);
        row = row < rows ? row : rows - 1;
        const uint8_t *p = W + (uint64_t)row * row_bytes;
#pragma unroll
        for (int c = 0; c < CH; c++) {
            const int b = b0 + (c < nblk ? c : nblk - 1);
            MQ<T>::load(p + (uint64_t)b * MQ<T>::bytes, L.g, raw[c]);
        }
    }
    __device__ __forceinline__ void step(int64_t rg, int par, const MqRaw (&cur)[CH]) const {
        float acc = 0.0f;
#pragma unroll
        for (int c = 0; c < CH; c++)
            if (c < nblk) acc += mq_block<T>(cur[c], L.g, b0 + c, lds0, 128u, n, L.a_lane, L.p, 0u);
        acc = mq_sum_units(acc);
        float *rb = red + par * nw * 16;
        if (L.lane < 16) rb[wave * 16 + L.lane] = acc;
        __syncthreads();
        if (threadIdx.x < 16) {
            float s = 0.0f;
            for (int w = 0; w < nw; w++) s += rb[w * 16 + threadIdx.x];
            res[(rg - blockIdx.x) / gridDim.x * 16 + threadIdx.x] = s;
        }
    }
};

template <int T, int CH>
__device__ __forceinline__ void mq_mv(const uint8_t *__restrict__ W, uint64_t row_bytes, int64_t rows, int32_t nb,
                                      const float *__restrict__ x, float *__restrict__ y) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    MqMv<T, CH> m;
    m.W = W;
    m.row_bytes = row_bytes;
    m.rows = rows;
    m.nb = nb;
    m.n = 256 * nb;
    m.tiles = (int32_t)((rows + 15) >> 4);
    m.y = y;
    m.lds0 = smem;
    m.red = (float *)(smem + 128 + mq_xq_bytes(m.n));
    m.L = mq_lane();
    m.wave = mq_wave_id();
    m.nw = blockDim.x >> 6;
    m.res = m.red + 2 * m.nw * 16;
    m.b0 = m.wave * CH;
    m.nblk = nb - m.b0 < CH ? nb - m.b0 : CH;
    MqRaw r0[CH], r1[CH];
    int64_t rg = blockIdx.x;
    const int64_t G = gridDim.x;
    if (rg < m.tiles) m.load(rg, r0);
    mq_stage_xq(x, 0, 1, m.n, smem, 128u, 0u);
    while (rg < m.tiles) {
        if (rg + G < m.tiles) {
            m.load(rg + G, r1);
            m.step(rg, 0, r0);
        } else {
            m.step(rg, 0, r0);
            break;
        }
        rg += G;
        if (rg + G < m.tiles) {
            m.load(rg + G, r0);
            m.step(rg, 1, r1);
        } else {
            m.step(rg, 1, r1);
            break;
        }
        rg += G;
    }
    __syncthreads();
    for (int i = threadIdx.x; (int64_t)blockIdx.x + (int64_t)(i >> 4) * G < m.tiles; i += blockDim.x) {
        const int64_t r = ((int64_t)blockIdx.x + (int64_t)(i >> 4) * G) * 16 + (i & 15);
        if (r < rows) y[r] = m.res[i];
    }
}

#define SEPIA_MQ_MV(name, T, CH)                                                                     \
    extern "C" __global__ __launch_bounds__(1024) void sepia_mq_mv_##name##_c##CH(                  \
        const uint8_t *__restrict__ W, uint64_t row_bytes, int64_t rows, int32_t nb,                 \
        const float *__restrict__ x, float *__restrict__ y) {                                        \
        mq_mv<T, CH>(W, row_bytes, rows, nb, x, y);                                                  \
    }

// --------------------------------------------------------- expert FFN ------
// One projection family of a stack of experts: expert e's quant rows start
// at base + e * stride, row r at + r * row_bytes.
struct MqProj {
    const uint8_t *base;
    uint64_t stride;
    uint64_t row_bytes;
    int64_t n_blocks;
    int32_t type;
    int32_t pad;
};

__device__ __forceinline__ int64_t mq_slot_expert(const int32_t *sel_idx, int32_t fixed, int32_t slot, int32_t topk) {
    return slot < topk ? (sel_idx ? (int64_t)sel_idx[slot] : (int64_t)fixed + slot) : (int64_t)(slot - topk);
}

// Gate/up of one slot, persistent over its row groups (rg = j0, j0 + jstep,
// ...): the pipeline walks iterations (row group, matrix) -- gate, then up of
// the same rows -- each wave taking blocks [w * CH, w * CH + CH), with the
// next iteration's loads in flight while the current one is computed.
// After the up iteration h[r] = silu(gate_r . x) * (up_r . x) goes to LDS;
// the workgroup stores its h values (f32) after the last iteration (see
// the matvec on stores inside the loop).
// LDS: [zero 128][XQ of x][2 x nw x 16 f32][nk x 16 f32 h values].
template <int T, int CH>
struct MqGu {
    const uint8_t *W[2];       // gate, up
    uint64_t row_bytes;
    int32_t nb, n, inter, tiles, jstep, j0;
    float *h;
    uint8_t *lds0;
    float *red, *hb;
    MqLane L;
    int wave, nw, b0, nblk;

    __device__ __forceinline__ int64_t rg_of(int it) const { return (int64_t)j0 + (int64_t)(it >> 1) * jstep; }
    __device__ __forceinline__ void load(int it, MqRaw (&raw)[CH]) const {
        int64_t row = rg_of(it) * 16 + (L.lane & 15);
        row = row < inter ? row : inter - 1;
        const uint8_t *p = W[it & 1] + (uint64_t)row * row_bytes;
#pragma unroll
        for (int c = 0; c < CH; c++)
            MQ<T>::load(p + (uint64_t)(b0 + (c < nblk ? c : nblk - 1)) * MQ<T>::bytes, L.g, raw[c]);
    }
    // gsum: threads < 16 keep the gate sums of the current row group
    __device__ __forceinline__ void step(int it, int par, const MqRaw (&cur)[CH], float &gsum) const {
        float a = 0.0f;
#pragma unroll
        for (int c = 0; c < CH; c++)
            if (c < nblk) a += mq_block<T>(cur[c], L.g, b0 + c, lds0, 128u, n, L.a_lane, L.p, 0u);
        a = mq_sum_units(a);
        float *rb = red + par * nw * 16;
        if (L.lane < 16) rb[wave * 16 + L.lane] = a;
        __syncthreads();
        if (threadIdx.x < 16) {
            float s = 0.0f;
            for (int w = 0; w < nw; w++) s += rb[w * 16 + threadIdx.x];
            if (!(it & 1))
                gsum = s;
            else
                hb[(it >> 1) * 16 + threadIdx.x] = silu_f32(gsum) * s;
        }
    }
};

template <int T, int CH>
__device__ __forceinline__ void mq_gateup_slot(const uint8_t *Wg, const uint8_t *Wu, uint64_t row_bytes, int32_t nb,
                                               int32_t inter, int32_t j0, int32_t jstep, const float *__restrict__ x,
                                               float *__restrict__ h) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    MqGu<T, CH> m;
    m.W[0] = Wg;
    m.W[1] = Wu;
    m.row_bytes = row_bytes;
    m.nb = nb;
    m.n = 256 * nb;
    m.inter = inter;
    m.tiles = (inter + 15) >> 4;
    m.jstep = jstep;
    m.j0 = j0;
    m.h = h;
    m.lds0 = smem;
    m.red = (float *)(smem + 128 + mq_xq_bytes(m.n));
    m.L = mq_lane();
    m.wave = mq_wave_id();
    m.nw = blockDim.x >> 6;
    m.hb = m.red + 2 * m.nw * 16;
    m.b0 = m.wave * CH;
    m.nblk = nb - m.b0 < CH ? nb - m.b0 : CH;
    const int N = j0 < m.tiles ? 2 * ((m.tiles - j0 + jstep - 1) / jstep) : 0;
    MqRaw r0[CH], r1[CH];
    if (N > 0) m.load(0, r0);
    mq_stage_xq(x, 0, 1, m.n, smem, 128u, 0u);
    float gsum = 0.0f;
    for (int it = 0; it < N;) {
        if (it + 1 < N) {
            m.load(it + 1, r1);
            m.step(it, 0, r0, gsum);
        } else {
            m.step(it, 0, r0, gsum);
            break;
        }
        ++it;
        if (it + 1 < N) {
            m.load(it + 1, r0);
            m.step(it, 1, r1, gsum);
        } else {
            m.step(it, 1, r1, gsum);
            break;
        }
        ++it;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < (N >> 1) * 16; i += blockDim.x) {
        const int64_t r = ((int64_t)j0 + (int64_t)(i >> 4) * jstep) * 16 + (i & 15);
        if (r < inter) h[r] = m.hb[i];
    }
}

// grid = n_slots * wps: workgroup k serves slot k / wps and its row groups
// k % wps, + wps, ... Routed slots (< topk) take their expert from sel_idx
// (or fixed + slot); the later slots are the shared experts. h is
// [n_slots][inter] f32.
template <int CH>
__device__ __forceinline__ void mq_gateup(const MqProj &gate, const MqProj &up, const MqProj &s_gate,
                                          const MqProj &s_up, const int32_t *__restrict__ sel_idx, int32_t fixed,
                                          int32_t topk, int32_t inter, int32_t wps, const float *__restrict__ x,
                                          float *__restrict__ h) {
    const int32_t slot = (int32_t)blockIdx.x / wps, j0 = (int32_t)blockIdx.x - slot * wps;
    const int64_t e = mq_slot_expert(sel_idx, fixed, slot, topk);
    const MqProj &G = slot < topk ? gate : s_gate;
    const MqProj &U = slot < topk ? up : s_up;
    const uint8_t *wg = G.base + e * G.stride, *wu = U.base + e * U.stride;
    float *hs = h + (int64_t)slot * inter;
    const int32_t nb = (int32_t)G.n_blocks;
    switch (G.type) {
    case ST_Q2_K: mq_gateup_slot<ST_Q2_K, CH>(wg, wu, G.row_bytes, nb, inter, j0, wps, x, hs); break;
    case ST_Q3_K: mq_gateup_slot<ST_Q3_K, CH>(wg, wu, G.row_bytes, nb, inter, j0, wps, x, hs); break;
    default: mq_gateup_slot<ST_Q4_K, CH>(wg, wu, G.row_bytes, nb, inter, j0, wps, x, hs); break;
    }
}

#define SEPIA_MQ_GATEUP(CH)                                                                              \
    extern "C" __global__ __launch_bounds__(1024) void sepia_mq_gateup_c##CH(                           \
        MqProj gate, MqProj up, MqProj s_gate, MqProj s_up, const int32_t *__restrict__ sel_idx,         \
        int32_t fixed, int32_t topk, int32_t inter, int32_t wps, const float *__restrict__ x,            \
        float *__restrict__ h) {                                                                         \
        mq_gateup<CH>(gate, up, s_gate, s_up, sel_idx, fixed, topk, inter, wps, x, h);                   \
    }

// Down of every slot for the workgroup's row groups of y (rg_k =
// blockIdx.x + k * gridDim.x, k < nk). The slots run in two phases, the
// routed ones (format of `down`) then the shared ones (format of `s_down`);
// within a phase a pipeline walks iterations (slot, k), slot-major, with the
// next iteration's loads in flight while the current one is computed (a
// phase has one format, so every step issues the same loads). Each row's
// slot sums are added in slot order, weighted by sel_w (routed weights, then
// the shared gammas; the shared gamma scales the down output as
// src/sepia.c:3953-3957 does), into an LDS accumulator; y is stored once at
// the end -- deterministic, no atomics. h [n_slots][inter] f32 is staged as
// XQ once per workgroup.
// LDS: [zero 128][n_slots x XQ of h][2 x nw x 16 f32][nk x 16 f32 accumulators]
//      [n_slots f32 weights][n_slots i32 experts].
template <int CH>
struct MqDnCtx {
    const int32_t *e_lds;      // the slots' experts, copied to LDS
    const float *w_lds;        // the slots' weights, copied to LDS
    int32_t fixed, topk, nk, n;
    int64_t hidden;
    uint32_t xqb;
    uint8_t *lds0;
    float *red, *acc;
    MqLane L;
    int wave, nw, b0, nblk;
};

template <int T, int CH>
struct MqDnPhase {
    const MqDnCtx<CH> &c;
    const MqProj &P;
    int slot0;

    __device__ __forceinline__ void load(int it, MqRaw (&raw)[CH]) const {
        const int slot = slot0 + it / c.nk, k = it - (it / c.nk) * c.nk;
        // the slot's expert from LDS: a global load here would make the next
        // iteration's addresses wait for every load in flight
        const int64_t e = (int64_t)c.e_lds[slot];
        const int64_t rg = (int64_t)blockIdx.x + (int64_t)k * gridDim.x;
        int64_t row = rg * 16 + (c.L.lane & 15);
        row = row < c.hidden ? row : c.hidden - 1;
        const uint8_t *p = P.base + e * P.stride + (uint64_t)row * P.row_bytes;
#pragma unroll
        for (int i = 0; i < CH; i++)
            MQ<T>::load(p + (uint64_t)(c.b0 + (i < c.nblk ? i : c.nblk - 1)) * MQ<T>::bytes, c.L.g, raw[i]);
    }
    __device__ __forceinline__ void step(int it, int par, const MqRaw (&cur)[CH]) const {
        const int slot = slot0 + it / c.nk, k = it - (it / c.nk) * c.nk;
        const uint32_t xoff = 128u + (uint32_t)slot * c.xqb;
        float a = 0.0f;
#pragma unroll
        for (int i = 0; i < CH; i++)
            if (i < c.nblk) a += mq_block<T>(cur[i], c.L.g, c.b0 + i, c.lds0, xoff, c.n, c.L.a_lane, c.L.p, 0u);
        a = mq_sum_units(a);
        float *rb = c.red + par * c.nw * 16;
        if (c.L.lane < 16) rb[c.wave * 16 + c.L.lane] = a;
        __syncthreads();
        if (threadIdx.x < 16) {
            float s = 0.0f;
            for (int w = 0; w < c.nw; w++) s += rb[w * 16 + threadIdx.x];
            c.acc[k * 16 + threadIdx.x] = __builtin_fmaf(c.w_lds[slot], s, c.acc[k * 16 + threadIdx.x]);
        }
    }
    __device__ __forceinline__ void run(int nsl) const {
        const int N = nsl * c.nk;
        if (N <= 0) return;
        MqRaw r0[CH], r1[CH];
        load(0, r0);
        for (int it = 0;;) {
            if (it + 1 < N) {
                load(it + 1, r1);
                step(it, 0, r0);
            } else {
                step(it, 0, r0);
                break;
            }
            ++it;
            if (it + 1 < N) {
                load(it + 1, r0);
                step(it, 1, r1);
            } else {
                step(it, 1, r1);
                break;
            }
            ++it;
        }
    }
};

template <int CH>
__device__ __forceinline__ void mq_dn_phase(const MqDnCtx<CH> &c, const MqProj &P, int slot0, int nsl) {
    switch (P.type) {
    case ST_Q2_K: MqDnPhase<ST_Q2_K, CH>{c, P, slot0}.run(nsl); break;
    case ST_Q3_K: MqDnPhase<ST_Q3_K, CH>{c, P, slot0}.run(nsl); break;
    default: MqDnPhase<ST_Q4_K, CH>{c, P, slot0}.run(nsl); break;
    }
}

template <int CH>
__device__ __forceinline__ void mq_down(const MqProj &down, const MqProj &s_down, const int32_t *__restrict__ sel_idx,
                                        const float *__restrict__ sel_w, int32_t fixed, int32_t topk,
                                        int32_t n_shared, int32_t inter, int64_t hidden, const float *__restrict__ h,
                                        float *__restrict__ y) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    MqDnCtx<CH> c;
    c.fixed = fixed;
    c.topk = topk;
    const int n_slots = topk + n_shared;
    const int64_t tiles = (hidden + 15) >> 4;
    c.nk = (int32_t)((tiles - blockIdx.x + gridDim.x - 1) / gridDim.x);
    c.n = inter;
    c.hidden = hidden;
    c.xqb = (uint32_t)mq_xq_bytes(inter);
    c.lds0 = smem;
    c.L = mq_lane();
    c.wave = mq_wave_id();
    c.nw = blockDim.x >> 6;
    c.red = (float *)(smem + 128 + (size_t)n_slots * c.xqb);
    c.acc = c.red + 2 * c.nw * 16;
    float *wl = c.acc + c.nk * 16;
    int32_t *el = (int32_t *)(wl + n_slots);
    c.w_lds = wl;
    c.e_lds = el;
    const int nb = (int32_t)down.n_blocks;
    c.b0 = c.wave * CH;
    c.nblk = nb - c.b0 < CH ? nb - c.b0 : CH;
    for (int i = threadIdx.x; i < c.nk * 16; i += blockDim.x) c.acc[i] = 0.0f;
    if (threadIdx.x < n_slots) {
        wl[threadIdx.x] = sel_w ? sel_w[threadIdx.x] : 1.0f;
        el[threadIdx.x] = (int32_t)mq_slot_expert(sel_idx, fixed, threadIdx.x, topk);
    }
    mq_stage_xq(h, inter, n_slots, inter, smem, 128u, c.xqb);
    mq_dn_phase<CH>(c, down, 0, topk);
    mq_dn_phase<CH>(c, s_down, topk, n_shared);
    if (threadIdx.x < 16) {
        for (int k = 0; k < c.nk; k++) {
            const int64_t r = ((int64_t)blockIdx.x + (int64_t)k * gridDim.x) * 16 + threadIdx.x;
            if (r < hidden) y[r] = c.acc[k * 16 + threadIdx.x];
        }
    }
}

#define SEPIA_MQ_DOWN(CH)                                                                                \
    extern "C" __global__ __launch_bounds__(1024) void sepia_mq_down_c##CH(                             \
        MqProj down, MqProj s_down, const int32_t *__restrict__ sel_idx, const float *__restrict__ sel_w, \
        int32_t fixed, int32_t topk, int32_t n_shared, int32_t inter, int64_t hidden,                    \
        const float *__restrict__ h, float *__restrict__ y) {                                            \
        mq_down<CH>(down, s_down, sel_idx, sel_w, fixed, topk, n_shared, inter, hidden, h, y);           \
    }
