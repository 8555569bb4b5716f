// mq.h -- quantized matvecs at decode batch 1 on the matrix cores.
//
// The dot products of quantized rows with x run as exact integer products
// on v_mfma_i32_16x16x64_i8; only the unpacking of the packed weights into
// int8 bytes and the per-segment scale arithmetic stay on the VALU, about
// one VALU instruction per weight.
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
// XQ layout for n columns: per 256-column block an 832-byte record of 16
// segments x {p0, p1, p2} (16 bytes each, 48 per segment) and 64 bytes of
// padding, then f32 xs, gs, gq [n / 16 each]. The padding spreads the A
// operand reads of one MFMA (three planes of four blocks, 12 lanes) over
// the LDS banks: 832 bytes is 16 banks mod 64 (at most two lanes per bank
// with 32 banks).
//
// Weights reach the waves by LDS DMA (global_load_lds_dwordx4): every wave
// owns a ring of S stages in LDS and fetches its own data, so the bytes in
// flight do not occupy VGPRs and the waves never wait for one another until
// the workgroup's final combine. A step of a wave covers 16 rows x 4 blocks
// of one matrix (a "quad" of blocks); lane l = (row j = l & 15, block
// g = l >> 4) computes with its block, which it reads back as W 16-byte
// words from stage + 16 Wp l (Wp = W rounded up to odd, so that eight
// consecutive lanes hit eight different 16-byte bank groups). The DMA that
// fills a stage takes its 16-byte pieces in that same order, so consecutive
// DMA lanes fetch consecutive words of one block (64 to 144 contiguous
// bytes) instead of one word of 64 different blocks.
//
// MFMA mapping. A block is four 64-weight units u of four 16-weight
// segments s (format-specific column order, MQ<T>::seg_col). For (u, s)
// the lane's 16 int8 weights form its B operand (B[k = 16g + t][j]); the A
// operand holds, on lane 20g + p (p < 3), digit plane p of the x columns of
// block g's (u, s) segment and zero on every other lane, so
// D[4g + p][j] = sum_t w_t * p_p(x_t): the three plane dots of (row j,
// block g) land in VGPRs 0..2 of lane l itself. No data crosses lanes until
// the row sums at the end of an item.
#pragma once
#include "common.h"
#include "route.h"

typedef int32_t mq_v4i __attribute__((ext_vector_type(4)));

// |q| + 0x8080 < 2^23, so q + 0x8080 splits into signed byte 2 and
// offset bytes 1 and 0 (below); and 16 * 15 * (QMAX + 1) < 2^31, so one
// segment's integer dot cannot overflow.
#define MQ_QMAX 8355000.0f
// Bytes of the zero area in front of the XQ vectors: the A operands of the
// lanes that carry no x data read it at the segment offsets of a block
// record (below 720 + 16).
#define MQ_ZERO 768
#define MQ_BREC 832     // bytes of a 256-column block record

// Bytes of the planes part and of a whole XQ vector of n columns (n a
// multiple of 256): 4 bytes per column.
__device__ __forceinline__ uint32_t mq_xq_planes(int64_t n) { return (uint32_t)(n >> 8) * MQ_BREC; }
__device__ __forceinline__ size_t mq_xq_bytes(int64_t n) { return (size_t)mq_xq_planes(n) + 3 * (size_t)(n / 16) * 4; }

// ------------------------------------------------------------ x -> XQ ----
// q + 0x8080 = 65536 * p0 + 256 * (p1 + 128) + (p2 + 128): byte 2 of it is
// p0 (two's complement), bytes 1 and 0 are p1 + 128 and p2 + 128, so
// p1, p2 = byte ^ 0x80. round(): v_rndne_f32 + v_cvt_i32_f32.
__device__ __forceinline__ int32_t mq_round(float v) { return (int32_t)__builtin_rintf(v); }

struct XqSeg {
    uint4 p0, p1, p2;
    float xs, gs, gq;
};
// A segment holding a NaN or an infinity gets m = +inf: every q is 0 and
// xs, gq are inf and NaN, so each dot that uses the segment comes out NaN,
// as the reference's double accumulation makes it non-finite
// (src/sepia.c:731-735). fmaxf drops a NaN operand; the plain sum keeps it.
__device__ __forceinline__ float mq_nonfinite_max(float m, float sum) { return (sum == sum) ? m : INFINITY; }
__device__ __forceinline__ XqSeg xq_segment(const float (&a)[16]) {
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) m = fmaxf(m, fabsf(a[i]));
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) sum += a[i];
    m = mq_nonfinite_max(m, sum);
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
    r.xs = xs;
    r.gs = sum;
    r.gq = xs * (float)qs;
    return r;
}

__device__ __forceinline__ void xq_store(const XqSeg &r, uint8_t *xq, int64_t n, int64_t seg) {
    uint8_t *pl = xq + (seg >> 4) * MQ_BREC + (seg & 15) * 48;
    *(uint4 *)(pl) = r.p0;
    *(uint4 *)(pl + 16) = r.p1;
    *(uint4 *)(pl + 32) = r.p2;
    float *xs = (float *)(xq + mq_xq_planes(n));
    xs[seg] = r.xs;
    xs[n / 16 + seg] = r.gs;
    xs[n / 8 + seg] = r.gq;
}

// Quad (4-lane) exchanges by DPP: lane l reads lane l ^ 1, l ^ 2.
__device__ __forceinline__ float mq_quad_x1(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ float mq_quad_x2(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
}
__device__ __forceinline__ int mq_quad_x1i(int v) { return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false); }
__device__ __forceinline__ int mq_quad_x2i(int v) { return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false); }

// XQ of one 16-column segment by a quad: lane j holds columns 4j .. 4j + 3
// (a), gets word j of each digit plane (p0, p1 + 128, p2 + 128 bytes) and
// the segment's xs, gs and gq. The same values as xq_segment but for the
// order of the gs sum.
struct XqQuad {
    uint32_t p0, p1, p2;
    float xs, gs, gq;
};
__device__ __forceinline__ XqQuad mq_xq_quad(const float (&a)[4]) {
    float m = fmaxf(fmaxf(fabsf(a[0]), fabsf(a[1])), fmaxf(fabsf(a[2]), fabsf(a[3])));
    m = fmaxf(m, mq_quad_x1(m));
    m = fmaxf(m, mq_quad_x2(m));
    float sum = (a[0] + a[1]) + (a[2] + a[3]);
    sum += mq_quad_x1(sum);
    sum += mq_quad_x2(sum);
    m = mq_nonfinite_max(m, sum);
    const float inv = (m > 0.0f) ? MQ_QMAX * __builtin_amdgcn_rcpf(m) : 0.0f;
    XqQuad r;
    r.xs = m * (1.0f / MQ_QMAX);
    uint32_t q[4];
    int32_t qs = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int32_t v = mq_round(a[i] * inv);
        qs += v;
        q[i] = (uint32_t)v + 0x8080u;
    }
    qs += mq_quad_x1i(qs);
    qs += mq_quad_x2i(qs);
    const uint32_t t01 = __builtin_amdgcn_perm(q[1], q[0], 0x05010400u);
    const uint32_t t23 = __builtin_amdgcn_perm(q[3], q[2], 0x05010400u);
    const uint32_t u01 = __builtin_amdgcn_perm(q[1], q[0], 0x06020602u);
    const uint32_t u23 = __builtin_amdgcn_perm(q[3], q[2], 0x06020602u);
    r.p0 = __builtin_amdgcn_perm(u23, u01, 0x05040100u);
    r.p1 = __builtin_amdgcn_perm(t23, t01, 0x07060302u) ^ 0x80808080u;
    r.p2 = __builtin_amdgcn_perm(t23, t01, 0x05040100u) ^ 0x80808080u;
    r.gs = sum;
    r.gq = r.xs * (float)qs;
    return r;
}

// ---- f32 vectors -> XQ in LDS, by the whole workgroup: `count` vectors of
// n columns (vector k at src + k * ld floats) to LDS offsets xoff + k * xqb.
// Each thread converts whole 16-column segments. Also clears the zero area
// at lds0; ends with a barrier.
// The n-float vector src (n a multiple of 256, src 4-byte aligned) into LDS
// at raw by LDS DMA, 1 KB per wave instruction, chunk c by wave c % waves.
// The caller waits for it (these DMAs are older than anything it issues
// next) before mq_stage_xq_lds.
__device__ __forceinline__ void mq_dma16(const uint8_t *base, uint32_t voff, uint32_t lds);
__device__ __forceinline__ void mq_dma_vec(const float *src, int n, uint32_t raw) {
    const int nw = (int)(blockDim.x >> 6), w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const uint32_t lane = threadIdx.x & 63;
    for (int c = w; c < (n >> 8); c += nw) mq_dma16((const uint8_t *)src, (uint32_t)c * 1024u + 16u * lane, raw + (uint32_t)c * 1024u);
}
// XQ of an n-float vector already in LDS (raw, 16-byte aligned), one
// thread per 16-column segment (fewer wave instructions than four lanes
// per segment, which measured slower here). Ends with a barrier.
__device__ __forceinline__ void mq_stage_xq_lds(const float *raw, int n, uint8_t *lds0, uint32_t xoff) {
    const int segs = n >> 4;
    for (int seg = threadIdx.x; seg < segs; seg += blockDim.x) {
        const float4 *x4 = (const float4 *)raw + 4 * seg;
        const float4 v0 = x4[0], v1 = x4[1], v2 = x4[2], v3 = x4[3];
        const float a[16] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w,
                             v2.x, v2.y, v2.z, v2.w, v3.x, v3.y, v3.z, v3.w};
        xq_store(xq_segment(a), lds0 + xoff, n, seg);
    }
    if (threadIdx.x < MQ_ZERO / 16) ((uint4 *)(lds0))[threadIdx.x] = make_uint4(0, 0, 0, 0);
    __syncthreads();
}

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
    if (threadIdx.x < MQ_ZERO / 16) ((uint4 *)(lds0))[threadIdx.x] = make_uint4(0, 0, 0, 0);
    __syncthreads();
}

// ------------------------------------------------------------- LDS DMA ----
__device__ __forceinline__ uint32_t mq_lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)p;
}
// One wave-wide DMA: lane l's 16 bytes at base + voff land at LDS address
// lds + 16 l. Issued as inline asm so that the compiler does not order every
// later LDS read of the workgroup behind it (it cannot tell the rings
// apart); the waits are explicit instead (mq_wait_stages), and the compiler's
// own vmcnt waits stay correct because vector memory operations retire in
// issue order.
// M0 holds the LDS address: the "{m0}" operand lets the compiler write it.
// The base is uniform by construction; readfirstlane states it, so that the
// "s" operand never depends on the compiler's uniformity analysis.
// Wait states: the compiler's hazard recognizer does not look into an asm
// statement, so the asm carries its own. On gfx9 a VMEM instruction that
// reads an SGPR a VALU instruction wrote (v_readfirstlane, when the base
// was in VGPRs) needs 5 wait states, and one that reads M0 after an SALU
// write of it needs 1: s_nop 4 gives the 5 whatever precedes the asm.
#define SEPIA_DMA_WAIT "s_nop 4\n\t"
__device__ __forceinline__ void mq_dma16(const uint8_t *base, uint32_t voff, uint32_t lds) {
    const uint64_t b = (uint64_t)(uintptr_t)base;
    const uint64_t bs = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32)) << 32) |
                        (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
    asm volatile(SEPIA_DMA_WAIT "global_load_lds_dwordx4 %0, %1" : : "v"(voff), "s"((const uint8_t *)(uintptr_t)bs), "{m0}"(lds) : "memory");
}
// s_waitcnt immediates (gfx9 encoding): vmcnt(n) alone, and lgkmcnt(0) alone.
__device__ __forceinline__ constexpr int mq_wc_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
#define MQ_WC_LGKM0 (15 | (3 << 14) | (7 << 4))
// Wait until at most n stages of W DMAs each are still in flight (n <= 3).
// W: DMAs per stage.
template <int W>
__device__ __forceinline__ void mq_wait_stages(int n) {
    if (n <= 0) __builtin_amdgcn_s_waitcnt(mq_wc_vm(0));
    else if (n == 1) __builtin_amdgcn_s_waitcnt(mq_wc_vm(W));
    else if (n == 2) __builtin_amdgcn_s_waitcnt(mq_wc_vm(2 * W));
    else if (n == 3) __builtin_amdgcn_s_waitcnt(mq_wc_vm(3 * W));
    else __builtin_amdgcn_s_waitcnt(mq_wc_vm(4 * W));
}

// ------------------------------------------------------- weight blocks ----
__device__ __forceinline__ float mq_half_lo(uint32_t v) { return f16_bits_to_f32(v & 0xFFFFu); }
__device__ __forceinline__ float mq_half_hi(uint32_t v) { return f16_bits_to_f32(v >> 16); }
// Byte B of v as a float, in plain C (one v_cvt_f32_ubyte<B>, or a bit-field
// extract and a convert when the compiler folds a mask into it). Never
// inline asm here: the compiler's hazard recognizer cannot see what an asm
// statement writes, and it placed such converts onto the operand and result
// registers of MFMAs still in flight.
template <int B>
__device__ __forceinline__ float mq_ubyte(uint32_t v) {
    return (float)((v >> (8 * B)) & 0xFFu);
}
// (p0 << 16) + (p1 << 8) + p2 of one segment's three plane dots: the exact
// integer sum of w * q (|.| < 2^31 for 16 weights <= 15 and |q| <= QMAX + 1).
// Plain C on purpose: the operands are MFMA results, and only the compiler's
// hazard recognizer inserts the wait states a VALU read of them needs.
__device__ __forceinline__ float mq_combine(const mq_v4i &d) {
    const uint32_t t = ((uint32_t)d[0] << 8) + (uint32_t)d[1];
    return (float)(int32_t)((t << 8) + (uint32_t)d[2]);
}

// What a lane needs besides its weights for one block: the LDS base, the
// byte offset of its A operand in the block record (plane p of the block on
// the A lanes, the zero area elsewhere), and the block's 16 segment scales
// xs and offset sums gv (gs or gq, per format).
struct MqCtx {
    const uint8_t *lds0;
    uint32_t abase;
    const float *xsb, *gvb;
    const uint8_t *tab;   // the format's codebook in LDS (IQ formats)
};
// A operand of the segment starting at column col of the block (col a
// multiple of 16): segment col / 16 of the record, 48 bytes each.
__device__ __forceinline__ mq_v4i mq_a(const MqCtx &x, int col) {
    return *(const mq_v4i *)(x.lds0 + x.abase + 3u * (uint32_t)col);
}
__device__ __forceinline__ mq_v4i mq_mfma(const mq_v4i &a, const mq_v4i &b) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, mq_v4i{0, 0, 0, 0}, 0, 0, 0);
}

template <int T> struct MQ;

// ---------------------------------------------------------------- Q2_K
// Block {scales[16]@0, qs[64]@16, d@80, dmin@82} (ggml block_q2_K). Unit
// u = (h = u >> 1, u' = u & 1): qs bytes 32h + 16u' + i, i < 16; bit pair s
// of that byte is the weight of column 128h + 32s + 16u' + i, in group
// 8h + 2s + u' whose scale byte holds (min << 4 | scale).
// Block value: d * sum sc (q . x) - dmin * sum m (sum x).
// Words: 0 = scales, 1..4 = qs, 5 = bytes 68..83 (d | dmin in its .w).
template <> struct MQ<ST_Q2_K> {
    static constexpr int bytes = 84, W = 6, Wp = 7, sum_sel = 1;
    static constexpr uint32_t table_bytes = 0;
    static constexpr bool has_pre = true;
    __device__ static uint32_t shift(uint32_t) { return 0u; }
    __device__ static uint32_t word(int k) { return k < 5 ? 16u * (uint32_t)k : 68u; }
    // Segment s: s = 0 mask 0x03, s = 1 mask 0x0C (4 q), s = 2 and 3 the same
    // on q >> 4 -- so segments 1 and 3 enter the MFMA scaled by 4.
    __device__ static mq_v4i bop(const uint4 &q, int s) {
        const uint32_t m = (s & 1) ? 0x0C0C0C0Cu : 0x03030303u;
        const uint32_t sh = (s & 2) ? 4u : 0u;
        return mq_v4i{(int32_t)((q.x >> sh) & m), (int32_t)((q.y >> sh) & m), (int32_t)((q.z >> sh) & m),
                      (int32_t)((q.w >> sh) & m)};
    }
    __device__ static float block(const uint4 (&w)[W], uint32_t, const MqCtx &x) {
        float acc = 0.0f, mn = 0.0f;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            float xs[8], gv[8];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                xs[i] = x.xsb[8 * h + i];
                gv[i] = x.gvb[8 * h + i];
            }
            const uint32_t s_lo = h ? w[0].z : w[0].x, s_hi = h ? w[0].w : w[0].y;
#pragma unroll
            for (int up = 0; up < 2; up++) {
                const uint4 q = w[1 + 2 * h + up];
                mq_v4i D[4];
#pragma unroll
                for (int s = 0; s < 4; s++) D[s] = mq_mfma(mq_a(x, 128 * h + 32 * s + 16 * up), bop(q, s));
                // scale bytes 2s + u' of the half's 8 bytes, gathered in s order
                const uint32_t sb = __builtin_amdgcn_perm(s_hi, s_lo, up ? 0x07050301u : 0x06040200u);
                const uint32_t scw = sb & 0x0F0F0F0Fu, mw = (sb >> 4) & 0x0F0F0F0Fu;
                const float a1 = __builtin_fmaf(mq_combine(D[0]), mq_ubyte<0>(scw) * xs[up],
                                                mq_combine(D[2]) * (mq_ubyte<2>(scw) * xs[4 + up]));
                const float a4 = __builtin_fmaf(mq_combine(D[1]), mq_ubyte<1>(scw) * xs[2 + up],
                                                mq_combine(D[3]) * (mq_ubyte<3>(scw) * xs[6 + up]));
                acc += __builtin_fmaf(0.25f, a4, a1);
                float m = mq_ubyte<0>(mw) * gv[up];
                m = __builtin_fmaf(mq_ubyte<1>(mw), gv[2 + up], m);
                m = __builtin_fmaf(mq_ubyte<2>(mw), gv[4 + up], m);
                mn += __builtin_fmaf(mq_ubyte<3>(mw), gv[6 + up], m);
            }
        }
        return __builtin_fmaf(mq_half_lo(w[5].w), acc, -(mq_half_hi(w[5].w) * mn));
    }
    // block() in two halves: pre() needs only the weights (B operands and
    // scales), post() the vector; the same operations in the same order.
    struct Pre {
        mq_v4i b[16];
        uint32_t scw[4], mw[4];
        uint32_t dd;
    };
    __device__ static Pre pre(const uint4 (&w)[W], uint32_t) {
        Pre r;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t s_lo = h ? w[0].z : w[0].x, s_hi = h ? w[0].w : w[0].y;
#pragma unroll
            for (int up = 0; up < 2; up++) {
                const uint4 q = w[1 + 2 * h + up];
#pragma unroll
                for (int s = 0; s < 4; s++) r.b[4 * (2 * h + up) + s] = bop(q, s);
                const uint32_t sb = __builtin_amdgcn_perm(s_hi, s_lo, up ? 0x07050301u : 0x06040200u);
                r.scw[2 * h + up] = sb & 0x0F0F0F0Fu;
                r.mw[2 * h + up] = (sb >> 4) & 0x0F0F0F0Fu;
            }
        }
        r.dd = w[5].w;
        return r;
    }
    __device__ static float post(const Pre &r, const MqCtx &x) {
        float acc = 0.0f, mn = 0.0f;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            float xs[8], gv[8];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                xs[i] = x.xsb[8 * h + i];
                gv[i] = x.gvb[8 * h + i];
            }
#pragma unroll
            for (int up = 0; up < 2; up++) {
                mq_v4i D[4];
#pragma unroll
                for (int s = 0; s < 4; s++) D[s] = mq_mfma(mq_a(x, 128 * h + 32 * s + 16 * up), r.b[4 * (2 * h + up) + s]);
                const uint32_t scw = r.scw[2 * h + up], mw = r.mw[2 * h + up];
                const float a1 = __builtin_fmaf(mq_combine(D[0]), mq_ubyte<0>(scw) * xs[up],
                                                mq_combine(D[2]) * (mq_ubyte<2>(scw) * xs[4 + up]));
                const float a4 = __builtin_fmaf(mq_combine(D[1]), mq_ubyte<1>(scw) * xs[2 + up],
                                                mq_combine(D[3]) * (mq_ubyte<3>(scw) * xs[6 + up]));
                acc += __builtin_fmaf(0.25f, a4, a1);
                float m = mq_ubyte<0>(mw) * gv[up];
                m = __builtin_fmaf(mq_ubyte<1>(mw), gv[2 + up], m);
                m = __builtin_fmaf(mq_ubyte<2>(mw), gv[4 + up], m);
                mn += __builtin_fmaf(mq_ubyte<3>(mw), gv[6 + up], m);
            }
        }
        return __builtin_fmaf(mq_half_lo(r.dd), acc, -(mq_half_hi(r.dd) * mn));
    }
};

// ---------------------------------------------------------------- Q3_K
// Block {hmask[32]@0, qs[64]@32, scales[12]@96, d@108}: 110 bytes, so
// every other block of a row starts 2 bytes past a 4-byte boundary. A lane
// fetches the 112 bytes from the 4-byte boundary at or below its block
// (shift sh = 0 or 2) and realigns with v_alignbyte; the block after an
// aligned one is never the last of a row (rows hold a multiple of 4
// blocks), so the fetch never leaves the matrix.
// Unit u = (h, u') as Q2_K: weight 128h + 32s + 16u' + i has low bits
// (qs[32h + 16u' + i] >> 2s) & 3 and is lowered by 4 unless bit 4h + s of
// hmask[16u' + i] is set; its group 8h + 2s + u' has a 6-bit scale stored
// +32 (low nibble in bytes 0..7, top two bits in bytes 8..11, ggml's
// kmask1/kmask2 packing). The B operand holds q + 4 * hbit in 0..7; the -4
// returns through the segment sum:
// contribution = d * sum_s (sc_s - 32) * ((q + 4 hbit) . x^ - 4 sum x^)_s.
template <> struct MQ<ST_Q3_K> {
    static constexpr int bytes = 110, W = 7, Wp = 7, sum_sel = 2;   // the -4 is part of the weight: gq
    static constexpr uint32_t table_bytes = 0;
    static constexpr bool has_pre = true;
    __device__ static uint32_t shift(uint32_t boff) { return boff & 3u; }
    __device__ static uint32_t word(int k) { return 16u * (uint32_t)k; }
    __device__ static float block(const uint4 (&w)[W], uint32_t sh, const MqCtx &x) {
        uint32_t raw[4 * W + 1];
#pragma unroll
        for (int k = 0; k < W; k++) {
            raw[4 * k] = w[k].x;
            raw[4 * k + 1] = w[k].y;
            raw[4 * k + 2] = w[k].z;
            raw[4 * k + 3] = w[k].w;
        }
        raw[4 * W] = 0u;
        // dword m of the block itself
        auto L = [&](int m) { return __builtin_amdgcn_alignbyte(raw[m + 1], raw[m], sh); };
        const uint32_t c0 = L(24), c1 = L(25), c2 = L(26), c3 = L(27);   // scales[12], d (low half of c3)
        float acc = 0.0f;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            float xs[8], gv[8];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                xs[i] = x.xsb[8 * h + i];
                gv[i] = x.gvb[8 * h + i];
            }
#pragma unroll
            for (int up = 0; up < 2; up++) {
                const int u = 2 * h + up;
                mq_v4i D[4];
#pragma unroll
                for (int s = 0; s < 4; s++) {
                    mq_v4i b;
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        const uint32_t qw = L(8 + 4 * u + t), hw = L(4 * up + t);
                        // hmask bits 4h.. moved to bit 2: << 2 for h = 0, >> 2 for h = 1
                        const uint32_t hf = h ? (hw >> 2) : (hw << 2);
                        b[t] = (int32_t)(((qw >> (2 * s)) & 0x03030303u) | ((hf >> s) & 0x04040404u));
                    }
                    D[s] = mq_mfma(mq_a(x, 128 * h + 32 * s + 16 * up), b);
                }
                const uint32_t base = 8u * (uint32_t)up + 4u * (uint32_t)h;
#pragma unroll
                for (int s = 0; s < 4; s++) {
                    const uint32_t lw = (s < 2) ? c0 : c1;
                    const uint32_t low4 = __builtin_amdgcn_ubfe(lw, 16u * (s & 1) + base, 4u);
                    const uint32_t top2 = __builtin_amdgcn_ubfe(c2, 16u * (s & 1) + 2u * (s >> 1) + base, 2u);
                    const float scf = (float)((int32_t)(low4 | (top2 << 4)) - 32);
                    const int li = 2 * s + up;
                    acc = __builtin_fmaf(scf, __builtin_fmaf(-4.0f, gv[li], mq_combine(D[s]) * xs[li]), acc);
                }
            }
        }
        return mq_half_lo(c3) * acc;
    }
    // block() in two halves (see MQ<ST_Q2_K>::Pre).
    struct Pre {
        mq_v4i b[16];
        float sc[16];
        uint32_t dd;
    };
    __device__ static Pre pre(const uint4 (&w)[W], uint32_t sh) {
        uint32_t raw[4 * W + 1];
#pragma unroll
        for (int k = 0; k < W; k++) {
            raw[4 * k] = w[k].x;
            raw[4 * k + 1] = w[k].y;
            raw[4 * k + 2] = w[k].z;
            raw[4 * k + 3] = w[k].w;
        }
        raw[4 * W] = 0u;
        auto L = [&](int m) { return __builtin_amdgcn_alignbyte(raw[m + 1], raw[m], sh); };
        const uint32_t c0 = L(24), c1 = L(25), c2 = L(26), c3 = L(27);
        Pre r;
#pragma unroll
        for (int h = 0; h < 2; h++) {
#pragma unroll
            for (int up = 0; up < 2; up++) {
                const int u = 2 * h + up;
#pragma unroll
                for (int s = 0; s < 4; s++) {
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        const uint32_t qw = L(8 + 4 * u + t), hw = L(4 * up + t);
                        const uint32_t hf = h ? (hw >> 2) : (hw << 2);
                        r.b[4 * u + s][t] = (int32_t)(((qw >> (2 * s)) & 0x03030303u) | ((hf >> s) & 0x04040404u));
                    }
                }
                const uint32_t base = 8u * (uint32_t)up + 4u * (uint32_t)h;
#pragma unroll
                for (int s = 0; s < 4; s++) {
                    const uint32_t lw = (s < 2) ? c0 : c1;
                    const uint32_t low4 = __builtin_amdgcn_ubfe(lw, 16u * (s & 1) + base, 4u);
                    const uint32_t top2 = __builtin_amdgcn_ubfe(c2, 16u * (s & 1) + 2u * (s >> 1) + base, 2u);
                    r.sc[4 * u + s] = (float)((int32_t)(low4 | (top2 << 4)) - 32);
                }
            }
        }
        r.dd = c3;
        return r;
    }
    __device__ static float post(const Pre &r, const MqCtx &x) {
        float acc = 0.0f;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            float xs[8], gv[8];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                xs[i] = x.xsb[8 * h + i];
                gv[i] = x.gvb[8 * h + i];
            }
#pragma unroll
            for (int up = 0; up < 2; up++) {
                const int u = 2 * h + up;
                mq_v4i D[4];
#pragma unroll
                for (int s = 0; s < 4; s++) D[s] = mq_mfma(mq_a(x, 128 * h + 32 * s + 16 * up), r.b[4 * u + s]);
#pragma unroll
                for (int s = 0; s < 4; s++) {
                    const int li = 2 * s + up;
                    acc = __builtin_fmaf(r.sc[4 * u + s], __builtin_fmaf(-4.0f, gv[li], mq_combine(D[s]) * xs[li]), acc);
                }
            }
        }
        return mq_half_lo(r.dd) * acc;
    }
};

// ---------------------------------------------------------------- Q4_K
// Block {d@0, dmin@2, scales[12]@4, qs[128]@16}. Unit u = 64-weight chunk:
// low nibbles of qs[32u .. 32u+31] are sub-block 2u (columns 64u .. 64u+31),
// high nibbles sub-block 2u+1 (64u+32 .. 64u+63). Segment s: s = 0 low
// nibbles of bytes 0..15, s = 1 low of 16..31, s = 2 high of 0..15, s = 3
// high of 16..31. y = d*sc*q - dmin*m with the 6-bit (sc, m) of sub-block j
// unpacked as reference src/quants.c:96-102.
// Words: 0 = d | dmin, scales[12]; 1..8 = qs.
template <> struct MQ<ST_Q4_K> {
    static constexpr int bytes = 144, W = 9, Wp = 9, sum_sel = 1;
    static constexpr uint32_t table_bytes = 0;
    static constexpr bool has_pre = true;
    __device__ static uint32_t shift(uint32_t) { return 0u; }
    __device__ static uint32_t word(int k) { return 16u * (uint32_t)k; }
    // (scale, min) of sub-block j = 2u + half. For j < 4 both are the low 6
    // bits of bytes j and j + 4; for j >= 4 (jj = j - 4) the low nibbles come
    // from byte 8 + jj and the top two bits from the top of bytes jj, jj + 4.
    __device__ static void scale_min(const uint4 &c, int u, int half, float &sc, float &mn) {
        const uint32_t hi = (uint32_t)(u >> 1);
        const uint32_t jj = (uint32_t)(2 * (u & 1) + half);
        const uint32_t wid = hi ? 4u : 6u, top = hi ? 2u : 0u;
        const uint32_t s0 = c.y, s1 = c.z, s2 = c.w;
        const uint32_t sl = __builtin_amdgcn_ubfe(hi ? s2 : s0, 8u * jj, wid);
        const uint32_t st = __builtin_amdgcn_ubfe(s0, 8u * jj + 6u, top);
        const uint32_t ml = __builtin_amdgcn_ubfe(hi ? s2 : s1, 8u * jj + 4u * hi, wid);
        const uint32_t mt = __builtin_amdgcn_ubfe(s1, 8u * jj + 6u, top);
        sc = (float)(sl | (st << 4));
        mn = (float)(ml | (mt << 4));
    }
    __device__ static float block(const uint4 (&w)[W], uint32_t, const MqCtx &x) {
        float acc = 0.0f, mn = 0.0f;
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const uint4 a = w[1 + 2 * u], b = w[2 + 2 * u];
            mq_v4i D[4];
#pragma unroll
            for (int s = 0; s < 4; s++) {
                const uint4 q = (s & 1) ? b : a;
                const uint32_t sh = (s & 2) ? 4u : 0u, m = 0x0F0F0F0Fu;
                D[s] = mq_mfma(mq_a(x, 64 * u + 16 * s),
                               mq_v4i{(int32_t)((q.x >> sh) & m), (int32_t)((q.y >> sh) & m),
                                      (int32_t)((q.z >> sh) & m), (int32_t)((q.w >> sh) & m)});
            }
            float xs[4], gv[4];
#pragma unroll
            for (int s = 0; s < 4; s++) {
                xs[s] = x.xsb[4 * u + s];
                gv[s] = x.gvb[4 * u + s];
            }
            float sc0, mn0, sc1, mn1;
            scale_min(w[0], u, 0, sc0, mn0);
            scale_min(w[0], u, 1, sc1, mn1);
            const float sub0 = __builtin_fmaf(mq_combine(D[0]), xs[0], mq_combine(D[1]) * xs[1]);
            const float sub1 = __builtin_fmaf(mq_combine(D[2]), xs[2], mq_combine(D[3]) * xs[3]);
            acc += __builtin_fmaf(sc0, sub0, sc1 * sub1);
            mn += __builtin_fmaf(mn0, gv[0] + gv[1], mn1 * (gv[2] + gv[3]));
        }
        return __builtin_fmaf(mq_half_lo(w[0].x), acc, -(mq_half_hi(w[0].x) * mn));
    }
    // block() in two halves (see MQ<ST_Q2_K>::Pre).
    struct Pre {
        mq_v4i b[16];
        float sc[8], mn[8];
        uint32_t dd;
    };
    __device__ static Pre pre(const uint4 (&w)[W], uint32_t) {
        Pre r;
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const uint4 a = w[1 + 2 * u], b = w[2 + 2 * u];
#pragma unroll
            for (int s = 0; s < 4; s++) {
                const uint4 q = (s & 1) ? b : a;
                const uint32_t sh = (s & 2) ? 4u : 0u, m = 0x0F0F0F0Fu;
                r.b[4 * u + s] = mq_v4i{(int32_t)((q.x >> sh) & m), (int32_t)((q.y >> sh) & m),
                                        (int32_t)((q.z >> sh) & m), (int32_t)((q.w >> sh) & m)};
            }
            scale_min(w[0], u, 0, r.sc[2 * u], r.mn[2 * u]);
            scale_min(w[0], u, 1, r.sc[2 * u + 1], r.mn[2 * u + 1]);
        }
        r.dd = w[0].x;
        return r;
    }
    __device__ static float post(const Pre &r, const MqCtx &x) {
        float acc = 0.0f, mn = 0.0f;
#pragma unroll
        for (int u = 0; u < 4; u++) {
            mq_v4i D[4];
#pragma unroll
            for (int s = 0; s < 4; s++) D[s] = mq_mfma(mq_a(x, 64 * u + 16 * s), r.b[4 * u + s]);
            float xs[4], gv[4];
#pragma unroll
            for (int s = 0; s < 4; s++) {
                xs[s] = x.xsb[4 * u + s];
                gv[s] = x.gvb[4 * u + s];
            }
            const float sub0 = __builtin_fmaf(mq_combine(D[0]), xs[0], mq_combine(D[1]) * xs[1]);
            const float sub1 = __builtin_fmaf(mq_combine(D[2]), xs[2], mq_combine(D[3]) * xs[3]);
            acc += __builtin_fmaf(r.sc[2 * u], sub0, r.sc[2 * u + 1] * sub1);
            mn += __builtin_fmaf(r.mn[2 * u], gv[0] + gv[1], r.mn[2 * u + 1] * (gv[2] + gv[3]));
        }
        return __builtin_fmaf(mq_half_lo(r.dd), acc, -(mq_half_hi(r.dd) * mn));
    }
};

// ------------------------------------------------------------- IQ formats
// Weights are a codebook entry (small positive bytes), a sign and a scale
// per 16 (IQ2_XS) or 32 (IQ3_XXS) weights: the signed codebook bytes are the
// B operand, exact in int8, and the scale multiplies the segment dot. The
// codebook sits in LDS (MqCtx::tab). Both block sizes leave every other
// block 2 bytes past a 4-byte boundary: the lane fetches W words from the
// boundary at or below (shift 0 or 2) and realigns as Q3_K does.
// The last word of a fetch comes from the end of the window (overlapping
// the word before), so a window ends at its block's end when the block is 2
// bytes off a boundary (the last block of a row always is) and 2 bytes after
// it otherwise: no bytes of the next block are read twice.
// Signs: bit j of the sign byte negates weight j (iq_signs adds the parity
// bit). The 128 sign indices' permute selectors (8 bytes each: byte j is j,
// or j + 4 where weight j is negative) follow the codebook in LDS, so a
// sign index is one 8-byte read and four signed codes are one v_perm_b32
// of a codebook word and its bytewise negation. IQ3_XXS keeps each word's
// negation beside it in LDS; IQ2_XS computes it (one subtract: no codebook
// byte is 0, so 0x01010100 - g negates every byte without a borrow).
// The three plane dots of a segment combined in f32: with codebook weights
// up to 62 the exact integer can pass 2^31 (mq_combine holds it for weights
// <= 15 only); each term is exact in f32, their sum rounds once or twice.
// 256 d1 + d2 stays exact in i32 (|d_p| <= 16 * 127 * 128 per segment), and
// one convert rounds it exactly as the f32 fma of d1, 256 and d2 would.
__device__ __forceinline__ float mq_combine_f(const mq_v4i &d) {
    return __builtin_fmaf((float)d[0], 65536.0f, (float)(int32_t)(((uint32_t)d[1] << 8) + (uint32_t)d[2]));
}
// The four signed codes of codebook word g (ng: its bytewise negation) by
// the selector word sel.
__device__ __forceinline__ uint32_t mq_iq_signed(uint32_t g, uint32_t ng, uint32_t sel) {
    return __builtin_amdgcn_perm(ng, g, sel);
}
// Permute selectors of sign index idx7 (0..127) from the table at st.
__device__ __forceinline__ uint2 mq_iq_mask(const uint8_t *st, uint32_t idx7) {
    return *(const uint2 *)(st + 8u * idx7);
}

// IQ2_XS {d@0, u16 qs[32]@2, scales[8]@66} (74 bytes, reference
// src/quants.c:179-201): 32-weight group ib has 4 entries qs[4 ib + l]
// (9-bit index into the 512 x 8-byte codebook, 7-bit sign index) and the
// scale nibble (l < 2: low, else high): w = d (0.5 + nibble) / 4 * entry.
// Segment sg = 2 ib + half covers entries l = 2 half, 2 half + 1.
template <> struct MQ<ST_IQ2_XS> {
    static constexpr int bytes = 74, W = 5, Wp = 5, sum_sel = 1;
    static constexpr uint32_t grid_bytes = 512 * 8, table_bytes = grid_bytes + 128 * 8;
    static constexpr bool has_pre = false;
    __device__ static uint32_t shift(uint32_t boff) { return boff & 3u; }
    // window bytes 0..75: words at 0, 16, 32, 48 and 60
    __device__ static uint32_t word(int k) { return k < 4 ? 16u * (uint32_t)k : 60u; }
    __device__ static float block(const uint4 (&w)[W], uint32_t sh, const MqCtx &x) {
        uint32_t raw[20];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            raw[4 * k] = w[k].x;
            raw[4 * k + 1] = w[k].y;
            raw[4 * k + 2] = w[k].z;
            raw[4 * k + 3] = w[k].w;
        }
        raw[16] = w[4].y;   // window dwords 16..18 (w[4].x repeats dword 15)
        raw[17] = w[4].z;
        raw[18] = w[4].w;
        raw[19] = 0u;
        auto L = [&](int m) { return __builtin_amdgcn_alignbyte(raw[m + 1], raw[m], sh); };
        const float d = mq_half_lo(L(0)), d4 = 0.25f * d, d8 = 0.125f * d;
        // scales bytes 66..73: the 8 nibble pairs
        const uint32_t sc_lo = __builtin_amdgcn_alignbyte(L(17), L(16), 2u), sc_hi = __builtin_amdgcn_alignbyte(L(18), L(17), 2u);
        float acc = 0.0f;
#pragma unroll
        for (int sg = 0; sg < 16; sg++) {
            const int ib = sg >> 1, half = sg & 1;
            // u16 entries 4 ib + 2 half and + 1: bytes 2 + 8 ib + 4 half .. + 3
            const uint32_t e = __builtin_amdgcn_alignbyte(L(2 * ib + half + 1), L(2 * ib + half), 2u);
            const uint32_t v0 = e & 0xFFFFu, v1 = e >> 16;
            const uint2 g0 = *(const uint2 *)(x.tab + 8u * (v0 & 511u));
            const uint2 g1 = *(const uint2 *)(x.tab + 8u * (v1 & 511u));
            const uint2 m0 = mq_iq_mask(x.tab + grid_bytes, v0 >> 9), m1 = mq_iq_mask(x.tab + grid_bytes, v1 >> 9);
            const mq_v4i b = {(int32_t)mq_iq_signed(g0.x, 0x01010100u - g0.x, m0.x),
                              (int32_t)mq_iq_signed(g0.y, 0x01010100u - g0.y, m0.y),
                              (int32_t)mq_iq_signed(g1.x, 0x01010100u - g1.x, m1.x),
                              (int32_t)mq_iq_signed(g1.y, 0x01010100u - g1.y, m1.y)};
            const mq_v4i D = mq_mfma(mq_a(x, 16 * sg), b);
            const uint32_t scb = ((ib < 4 ? sc_lo : sc_hi) >> (8 * (ib & 3))) & 0xFFu;
            const float nib = (float)(half ? (scb >> 4) : (scb & 15u));
            // d (0.5 + nib) / 4 as one fma: the quarter and eighth of d are
            // exact, so the single rounding gives the same float
            const float db = __builtin_fmaf(nib, d4, d8);
            acc = __builtin_fmaf(db * x.xsb[sg], mq_combine_f(D), acc);
        }
        return acc;
    }
};

// IQ3_XXS {d@0, qs[64]@2, scales_signs[32]@66} (98 bytes, reference
// src/quants.c:203-226): group ib has the word aux = scales_signs[4 ib ..]
// (4 x 7-bit sign indices, 4-bit scale on top) and bytes qs[8 ib .. 8 ib +
// 7] (indices into the 256-entry codebook, two per 8 weights; in LDS each
// 4-byte entry is followed by its negation):
// w = d (0.5 + aux >> 28) / 2 * entry. Segment sg = 2 ib + half covers
// index bytes 8 ib + 4 half .. + 3 and sign indices 2 half, 2 half + 1.
template <> struct MQ<ST_IQ3_XXS> {
    static constexpr int bytes = 98, W = 7, Wp = 7, sum_sel = 1;
    static constexpr uint32_t grid_bytes = 256 * 8, table_bytes = grid_bytes + 128 * 8;
    static constexpr bool has_pre = false;
    __device__ static uint32_t shift(uint32_t boff) { return boff & 3u; }
    // window bytes 0..99: words at 0, 16, ..., 80 and 84
    __device__ static uint32_t word(int k) { return k < 6 ? 16u * (uint32_t)k : 84u; }
    __device__ static float block(const uint4 (&w)[W], uint32_t sh, const MqCtx &x) {
        uint32_t raw[26];
#pragma unroll
        for (int k = 0; k < 6; k++) {
            raw[4 * k] = w[k].x;
            raw[4 * k + 1] = w[k].y;
            raw[4 * k + 2] = w[k].z;
            raw[4 * k + 3] = w[k].w;
        }
        raw[24] = w[6].w;   // window dword 24 (w[6].x .. .z repeat dwords 21..23)
        raw[25] = 0u;
        auto L = [&](int m) { return __builtin_amdgcn_alignbyte(raw[m + 1], raw[m], sh); };
        const float d = mq_half_lo(L(0)), d2 = 0.5f * d, d4 = 0.25f * d;
        float acc = 0.0f;
#pragma unroll
        for (int ib = 0; ib < 8; ib++) {
            const uint32_t aux = __builtin_amdgcn_alignbyte(L(17 + ib), L(16 + ib), 2u);
            // d (0.5 + aux >> 28) / 2 as one fma (half and quarter of d exact)
            const float db = __builtin_fmaf((float)(aux >> 28), d2, d4);
#pragma unroll
            for (int half = 0; half < 2; half++) {
                const int sg = 2 * ib + half;
                const uint32_t idx = __builtin_amdgcn_alignbyte(L(2 * ib + half + 1), L(2 * ib + half), 2u);
                const uint2 ma = mq_iq_mask(x.tab + grid_bytes, (aux >> (14 * half)) & 127u);
                const uint2 mb = mq_iq_mask(x.tab + grid_bytes, (aux >> (14 * half + 7)) & 127u);
                const uint2 *tab = (const uint2 *)x.tab;
                const uint2 t0 = tab[idx & 0xFFu], t1 = tab[(idx >> 8) & 0xFFu], t2 = tab[(idx >> 16) & 0xFFu],
                            t3 = tab[idx >> 24];
                const mq_v4i b = {(int32_t)mq_iq_signed(t0.x, t0.y, ma.x), (int32_t)mq_iq_signed(t1.x, t1.y, ma.y),
                                  (int32_t)mq_iq_signed(t2.x, t2.y, mb.x), (int32_t)mq_iq_signed(t3.x, t3.y, mb.y)};
                const mq_v4i D = mq_mfma(mq_a(x, 16 * sg), b);
                acc = __builtin_fmaf(db * x.xsb[sg], mq_combine_f(D), acc);
            }
        }
        return acc;
    }
};

// ------------------------------------------- Q5_K, Q6_K, IQ4_XS, Q8_0
// Codes above 15 (Q5_K 0..31, Q6_K 0..63, IQ4_XS and Q8_0 int8): the plane
// dots combine in f32 (mq_combine_f).

// Q5_K {d@0, dmin@2, scales[12]@4, qh[32]@16, qs[128]@48} (176 bytes = 11
// words, reference src/quants.c:127-151). As Q4_K with a fifth bit: the low
// nibble of qs[32u + l] (sub-block 2u) adds 16 when bit 2u of qh[l] is set,
// the high nibble (sub-block 2u + 1) with bit 2u + 1. Segment s of unit u as
// Q4_K: s & 1 picks bytes 16..31 of the unit (and of qh), s & 2 the high
// nibbles.
// Words: 0 = d | dmin, scales[12]; 1, 2 = qh; 3..10 = qs.
template <> struct MQ<ST_Q5_K> {
    static constexpr int bytes = 176, W = 11, Wp = 11, sum_sel = 1;
    static constexpr uint32_t table_bytes = 0;
    static constexpr bool has_pre = false;
    __device__ static uint32_t shift(uint32_t) { return 0u; }
    __device__ static uint32_t word(int k) { return 16u * (uint32_t)k; }
    __device__ static float block(const uint4 (&w)[W], uint32_t, const MqCtx &x) {
        float acc = 0.0f, mn = 0.0f;
#pragma unroll
        for (int u = 0; u < 4; u++) {
            mq_v4i D[4];
#pragma unroll
            for (int s = 0; s < 4; s++) {
                const uint4 q = w[3 + 2 * u + (s & 1)], qh = w[1 + (s & 1)];
                const uint32_t sh = (s & 2) ? 4u : 0u, hb = 2u * (uint32_t)u + (uint32_t)(s >> 1);
                const uint32_t m = 0x0F0F0F0Fu, m1 = 0x01010101u;
                D[s] = mq_mfma(mq_a(x, 64 * u + 16 * s),
                               mq_v4i{(int32_t)(((q.x >> sh) & m) | (((qh.x >> hb) & m1) << 4)),
                                      (int32_t)(((q.y >> sh) & m) | (((qh.y >> hb) & m1) << 4)),
                                      (int32_t)(((q.z >> sh) & m) | (((qh.z >> hb) & m1) << 4)),
                                      (int32_t)(((q.w >> sh) & m) | (((qh.w >> hb) & m1) << 4))});
            }
            float xs[4], gv[4];
#pragma unroll
            for (int s = 0; s < 4; s++) {
                xs[s] = x.xsb[4 * u + s];
                gv[s] = x.gvb[4 * u + s];
            }
            float sc0, mn0, sc1, mn1;
            MQ<ST_Q4_K>::scale_min(w[0], u, 0, sc0, mn0);
            MQ<ST_Q4_K>::scale_min(w[0], u, 1, sc1, mn1);
            const float sub0 = __builtin_fmaf(mq_combine_f(D[0]), xs[0], mq_combine_f(D[1]) * xs[1]);
            const float sub1 = __builtin_fmaf(mq_combine_f(D[2]), xs[2], mq_combine_f(D[3]) * xs[3]);
            acc += __builtin_fmaf(sc0, sub0, sc1 * sub1);
            mn += __builtin_fmaf(mn0, gv[0] + gv[1], mn1 * (gv[2] + gv[3]));
        }
        return __builtin_fmaf(mq_half_lo(w[0].x), acc, -(mq_half_hi(w[0].x) * mn));
    }
};

// Q6_K {ql[128]@0, qh[64]@128, scales[16]@192 (int8), d@208} (210 bytes,
// reference src/quants.c:153-176). Every other block of a row starts 2 bytes
// past a 4-byte boundary: fetched from the boundary at or below and
// realigned as Q3_K. The last word comes from bytes 196..211 of the fetch
// (overlapping the one before), so a fetch ends at its block's end when the
// block is 2 bytes off (the last block of a row always is: rows hold a
// multiple of 4 blocks) and 2 bytes after it otherwise.
// Column 128 hf + 32 r + 16 i + t (r < 4; i < 2; t < 16) has the code
// q = ((ql[64 hf + 32 (r & 1) + 16 i + t] >> 4 (r >> 1)) & 15) |
// ((qh[32 hf + 16 i + t] >> 2 r) & 3) << 4 and the weight d sc (q - 32),
// sc the int8 scale of its 16 columns: scales[col / 16]. The B operand
// holds q (0..63); the -32 returns through the segment sum of x^ (gq), as
// Q3_K's -4 does.
template <> struct MQ<ST_Q6_K> {
    static constexpr int bytes = 210, W = 14, Wp = 15, sum_sel = 2;
    static constexpr uint32_t table_bytes = 0;
    static constexpr bool has_pre = false;
    __device__ static uint32_t shift(uint32_t boff) { return boff & 3u; }
    __device__ static uint32_t word(int k) { return k < 13 ? 16u * (uint32_t)k : 196u; }
    __device__ static float block(const uint4 (&w)[W], uint32_t sh, const MqCtx &x) {
        uint32_t raw[54];
#pragma unroll
        for (int k = 0; k < 13; k++) {
            raw[4 * k] = w[k].x;
            raw[4 * k + 1] = w[k].y;
            raw[4 * k + 2] = w[k].z;
            raw[4 * k + 3] = w[k].w;
        }
        raw[52] = w[13].w;   // fetch bytes 208..211
        raw[53] = 0u;
        auto L = [&](int m) { return __builtin_amdgcn_alignbyte(raw[m + 1], raw[m], sh); };
        float acc = 0.0f;
        // groups (hf, i) of four segments share their qh dwords and, two by
        // two, their ql dwords; a group's words die before the next starts
        // (the scheduling barrier keeps the groups apart, which keeps the
        // block within the registers of 16 waves)
#pragma unroll
        for (int gi = 0; gi < 4; gi++) {
            const int hf = gi >> 1, i = gi & 1;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int sg = 8 * hf + 2 * r + i;
                const uint32_t nsh = 4u * (uint32_t)(r >> 1), hsh = 2u * (uint32_t)r;
                mq_v4i b;
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const uint32_t ql = L(16 * hf + 8 * (r & 1) + 4 * i + t), qh = L(32 + 8 * hf + 4 * i + t);
                    b[t] = (int32_t)(((ql >> nsh) & 0x0F0F0F0Fu) | (((qh >> hsh) & 0x03030303u) << 4));
                }
                const mq_v4i D = mq_mfma(mq_a(x, 16 * sg), b);
                // the int8 scale as (byte ^ 0x80) - 128 from an unsigned byte
                // convert: a signed byte extract feeding the convert was
                // folded into v_cvt_f32_u32 of the sign-extended byte, which
                // turns a negative scale into about 2^32
                const uint32_t scb = (L(48 + (sg >> 2)) >> (8 * (sg & 3))) & 0xFFu;
                const float sc = (float)(scb ^ 0x80u) - 128.0f;
                acc = __builtin_fmaf(sc, __builtin_fmaf(-32.0f, x.gvb[sg], mq_combine_f(D) * x.xsb[sg]), acc);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        return mq_half_lo(L(52)) * acc;
    }
};

// IQ4_XS {d@0, scales_h@2 (u16), scales_l[4]@4, qs[128]@8} (136 bytes,
// reference src/quants.c:228-249): group ib of 32 columns has the 6-bit
// scale ls = nibble ib of scales_l | (bits 2 ib, 2 ib + 1 of scales_h) << 4
// and the codes of qs[16 ib + j]: low nibble column 32 ib + j, high nibble
// column 32 ib + 16 + j; w = d (ls - 32) values[code] with the 16 int8
// levels of the IQ4 non-linear table. Segment sg = 2 ib + half. Blocks are
// 4-byte aligned; the last word comes from bytes 120..135 (overlapping the
// one before), so the fetch ends at the block's end.
// Four codes at a time become their levels by byte permutes: code & 7
// selects a byte of the table's first and of its second half (two
// v_perm_b32 over two table dwords each), and a third permute keeps the
// first or the second by bit 3.
__device__ __forceinline__ constexpr uint32_t mq_iq4_word(int k) {
    constexpr int8_t v[16] = SEPIA_IQ4NL_VALUES_INIT;
    return (uint32_t)(uint8_t)v[4 * k] | ((uint32_t)(uint8_t)v[4 * k + 1] << 8) |
           ((uint32_t)(uint8_t)v[4 * k + 2] << 16) | ((uint32_t)(uint8_t)v[4 * k + 3] << 24);
}
// Levels of the four codes in the low nibbles of the bytes of c.
__device__ __forceinline__ uint32_t mq_iq4_levels(uint32_t c) {
    constexpr uint32_t T0 = mq_iq4_word(0), T1 = mq_iq4_word(1), T2 = mq_iq4_word(2), T3 = mq_iq4_word(3);
    const uint32_t sel = c & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(T1, T0, sel), hi = __builtin_amdgcn_perm(T3, T2, sel);
    // byte k of the result: byte k of lo (selector k) or of hi (k + 4, bit 3 of the code moved to bit 2)
    return __builtin_amdgcn_perm(hi, lo, ((c >> 1) & 0x04040404u) | 0x03020100u);
}
template <> struct MQ<ST_IQ4_XS> {
    static constexpr int bytes = 136, W = 9, Wp = 9, sum_sel = 1;
    static constexpr uint32_t table_bytes = 0;
    static constexpr bool has_pre = false;
    __device__ static uint32_t shift(uint32_t) { return 0u; }
    __device__ static uint32_t word(int k) { return k < 8 ? 16u * (uint32_t)k : 120u; }
    __device__ static float block(const uint4 (&w)[W], uint32_t, const MqCtx &x) {
        uint32_t raw[34];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            raw[4 * k] = w[k].x;
            raw[4 * k + 1] = w[k].y;
            raw[4 * k + 2] = w[k].z;
            raw[4 * k + 3] = w[k].w;
        }
        raw[32] = w[8].z;   // block bytes 128..135
        raw[33] = w[8].w;
        const float d = mq_half_lo(raw[0]);
        const uint32_t sh_hi = raw[0] >> 16, sl = raw[1];
        float acc = 0.0f;
#pragma unroll
        for (int ib = 0; ib < 8; ib++) {
            const uint32_t ls = ((sl >> (4 * ib)) & 15u) | (((sh_hi >> (2 * ib)) & 3u) << 4);
            const float dl = d * (float)((int32_t)ls - 32);
            mq_v4i D[2];
#pragma unroll
            for (int half = 0; half < 2; half++) {
                mq_v4i b;
#pragma unroll
                for (int t = 0; t < 4; t++) b[t] = (int32_t)mq_iq4_levels(raw[2 + 4 * ib + t] >> (4 * half));
                D[half] = mq_mfma(mq_a(x, 32 * ib + 16 * half), b);
            }
            acc = __builtin_fmaf(dl, __builtin_fmaf(mq_combine_f(D[0]), x.xsb[2 * ib], mq_combine_f(D[1]) * x.xsb[2 * ib + 1]),
                                 acc);
        }
        return acc;
    }
};

// Q8_0 in super-blocks of 8 blocks {d@0, qs[32]@2} (34 bytes each,
// reference src/quants.c:85-94): 272 bytes = 17 words and 256 columns, so a
// row of a multiple of 1024 columns steps in the K-quants' quads of four
// super-blocks (the host counts such rows in super-blocks). Block k sits at
// byte 34 k: for even k its qs start 2 bytes past a 4-byte boundary (realigned
// with v_alignbyte) and d is the low half of dword 34 k / 4; for odd k the
// qs are aligned and d is the high half of dword (34 k - 2) / 4.
template <> struct MQ<ST_Q8_0> {
    static constexpr int bytes = 272, W = 17, Wp = 17, sum_sel = 1;
    static constexpr uint32_t table_bytes = 0;
    static constexpr bool has_pre = false;
    // Read and decoded in two parts of 9 words (the whole block does not
    // fit the registers of 16 waves beside the pipeline): words 0..8 hold
    // blocks 0..3 (bytes 0..135), words 8..16 blocks 4..7 (bytes 136..271).
    static constexpr int W1 = 9, O2 = 8;
    __device__ static uint32_t shift(uint32_t) { return 0u; }
    __device__ static uint32_t word(int k) { return 16u * (uint32_t)k; }
    // Blocks 4 H .. 4 H + 3 from words 8 H .. 8 H + 8 (dword m of the
    // super-block is raw[m - 32 H]).
    template <int H>
    __device__ static float part(const uint4 (&w)[9], const MqCtx &x) {
        uint32_t raw[36];
#pragma unroll
        for (int k = 0; k < 9; k++) {
            raw[4 * k] = w[k].x;
            raw[4 * k + 1] = w[k].y;
            raw[4 * k + 2] = w[k].z;
            raw[4 * k + 3] = w[k].w;
        }
        constexpr int o = 32 * H;
        float acc = 0.0f;
#pragma unroll
        for (int k = 4 * H; k < 4 * H + 4; k++) {
            const float d = (k & 1) ? mq_half_hi(raw[(34 * k - 2) / 4 - o]) : mq_half_lo(raw[34 * k / 4 - o]);
            mq_v4i D[2];
#pragma unroll
            for (int half = 0; half < 2; half++) {
                const int m = (34 * k + 2 + 16 * half) / 4 - o;
                mq_v4i b;
#pragma unroll
                for (int t = 0; t < 4; t++)
                    b[t] = (int32_t)((k & 1) ? raw[m + t] : __builtin_amdgcn_alignbyte(raw[m + t + 1], raw[m + t], 2u));
                D[half] = mq_mfma(mq_a(x, 32 * k + 16 * half), b);
            }
            acc = __builtin_fmaf(d, __builtin_fmaf(mq_combine_f(D[0]), x.xsb[2 * k], mq_combine_f(D[1]) * x.xsb[2 * k + 1]),
                                 acc);
            if (k & 1) __builtin_amdgcn_sched_barrier(0);   // two blocks at a time
        }
        return acc;
    }
};

// Formats read in two parts declare W1 (words of the first part) and O2
// (first word of the second, which runs to W - 1); the others read their
// W words at once (W1 = 0).
template <class M, class = void> struct MqSplit {
    static constexpr int W1 = 0, O2 = 0;
};
template <class M> struct MqSplit<M, decltype((void)M::W1)> {
    static constexpr int W1 = M::W1, O2 = M::O2;
};

// LDS codebook bytes of a format, by type code.
__device__ __forceinline__ uint32_t mq_table_bytes(int32_t type) {
    return type == ST_IQ2_XS ? MQ<ST_IQ2_XS>::table_bytes : type == ST_IQ3_XXS ? MQ<ST_IQ3_XXS>::table_bytes : 0u;
}
// The format's codebook into LDS at tab (IQ formats; nothing for the
// others). Published by the caller's next barrier.
// IQ formats: the codebook (IQ3_XXS: each word followed by its bytewise
// negation), then the permute selectors of the 128 sign indices (8 bytes
// each: byte j is j mod 4, plus 4 when bit j of iq_signs(index) is set).
__device__ __forceinline__ uint32_t mq_neg_bytes(uint32_t g) {
    uint32_t r = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) r |= ((256u - ((g >> (8 * j)) & 0xFFu)) & 0xFFu) << (8 * j);
    return r;
}
template <int T>
__device__ __forceinline__ void mq_fill_signs(uint8_t *st) {
    for (int i = threadIdx.x; i < 128; i += blockDim.x) {
        const uint32_t s = iq_signs((uint32_t)i);
        uint2 m;
        m.x = 0x03020100u | ((s & 1u) << 2) | ((s & 2u) << 9) | ((s & 4u) << 16) | ((s & 8u) << 23);
        m.y = 0x03020100u | ((s & 16u) >> 2) | ((s & 32u) << 5) | ((s & 64u) << 12) | ((s & 128u) << 19);
        ((uint2 *)st)[i] = m;
    }
}
template <int T>
__device__ __forceinline__ void mq_fill_table(uint8_t *tab) {
    if constexpr (T == ST_IQ2_XS) {
        for (int i = threadIdx.x; i < 512; i += blockDim.x) ((uint64_t *)tab)[i] = c_iq2xs_grid[i];
        mq_fill_signs<T>(tab + MQ<T>::grid_bytes);
    } else if constexpr (T == ST_IQ3_XXS) {
        for (int i = threadIdx.x; i < 256; i += blockDim.x) {
            const uint32_t g = c_iq3xxs_grid[i];
            ((uint2 *)tab)[i] = make_uint2(g, mq_neg_bytes(g));
        }
        mq_fill_signs<T>(tab + MQ<T>::grid_bytes);
    }
}

// ------------------------------------------------------------ the waves ---
struct MqLane {
    int lane, g, p;
    bool a_lane;   // lane 20g + p, p < 3: carries digit plane p of block g's x
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

// ------------------------------------------- vector by converter waves ----
// Wait until the LDS counter c reaches target (acquire), bounded in time:
// sepia_wait_ticks of s_memrealtime (100 MHz; 2 s unless the host sets
// another bound). On expiry the wave goes on and code 5 goes to err, or
// else to the library's device error word, which the host checks when the
// batch ends: the launch's outputs are then invalid.
// The elapsed time is compared in 32 bits (bounds up to 2^32 - 1 ticks, 42
// s): a scalar compare, where a 64-bit one needs a VGPR copy of the bound
// that can make the poll loop wait for the wave's outstanding loads.
__device__ __forceinline__ void mq_waves_wait(uint32_t *c, uint32_t target, int lane, uint32_t *err) {
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    const uint64_t b64 = sepia_wait_ticks;
    const uint32_t bound = b64 > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)b64;
    while (__hip_atomic_load(c, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < target) {
        __builtin_amdgcn_s_sleep(1);
        if ((uint32_t)(__builtin_amdgcn_s_memrealtime() - t0) > bound) {
            sepia_report_error(err, 5u, lane);
            return;
        }
    }
}

// Waves first .. first + count - 1 of the workgroup wait for one another:
// arrival k of each (k = 1, 2, ...) completes when the counter at c
// reaches k * count. Bounded in time (error code 5 on expiry).
__device__ __forceinline__ void mq_waves_sync(uint32_t *c, uint32_t target, int lane, uint32_t *err) {
    if (lane == 0) __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    mq_waves_wait(c, target, lane, err);
}

// The n-float vector x becomes its XQ form at LDS offset xoff, in place,
// by the waves of threads first .. first + count - 1 (count a multiple of
// 64) alone: they DMA x (1 KB a wave instruction), wait for their own
// DMAs, then four lanes per 16-column segment -- lane j of a quad holds
// columns 4j .. 4j + 3 and writes word j of each digit plane, the segment's
// max and sums by quad exchanges -- in up to MQ_XQP passes of count / 4
// segments (n / 16 <= MQ_XQP count / 4). The same XQ as xq_segment but for
// the order of the gs sum. Every float is read before any byte is written.
// Three arrivals at the counter c (landed, read, written): other waves may
// use the XQ vector once it reaches 3 (count / 64). Clears the zero area.
#define MQ_XQP 8
__device__ __forceinline__ void mq_xq_dma_by(const float *src, int n, uint8_t *lds0, uint32_t xoff, int first,
                                             int count) {
    const int nw = count >> 6, w = mq_wave_id() - (first >> 6);
    const uint32_t lane = threadIdx.x & 63, raw = mq_lds_addr(lds0 + xoff);
    // the conversion gates every gate/up wave: these waves go first on the
    // SIMDs until it is written (back to 0 at its end)
    __builtin_amdgcn_s_setprio(3);
    for (int c = w; c < (n >> 8); c += nw) mq_dma16((const uint8_t *)src, (uint32_t)c * 1024u + 16u * lane, raw + (uint32_t)c * 1024u);
}
__device__ __forceinline__ void mq_xq_in_place_by(int n, uint8_t *lds0, uint32_t xoff, int first, int count,
                                                  uint32_t *c, uint32_t *err, bool waited = false) {
    const int t = (int)threadIdx.x - first, segs = n >> 4, per = count >> 2, lane = t & 63;
    const uint32_t nw = (uint32_t)(count >> 6);
    const int j = t & 3, s0 = t >> 2;
    if (!waited) __builtin_amdgcn_s_waitcnt(mq_wc_vm(0));   // this wave's DMAs of x (or the caller waited)
    mq_waves_sync(c, nw, lane, err);
    float4 v[MQ_XQP];
#pragma unroll
    for (int k = 0; k < MQ_XQP; k++) {
        const int seg = s0 + k * per;
        v[k] = ((const float4 *)(lds0 + xoff))[4 * (seg < segs ? seg : segs - 1) + j];
    }
    if (t < MQ_ZERO / 16) ((uint4 *)(lds0))[t] = make_uint4(0, 0, 0, 0);
    mq_waves_sync(c, 2 * nw, lane, err);
    float *xsv = (float *)(lds0 + xoff + mq_xq_planes(n));
    // straight-line passes (a segment past the end converts a copy of the
    // last and stores nothing), so that they interleave
    XqQuad r[MQ_XQP];
#pragma unroll
    for (int k = 0; k < MQ_XQP; k++) {
        const float a[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
        r[k] = mq_xq_quad(a);
    }
#pragma unroll
    for (int k = 0; k < MQ_XQP; k++) {
        const int seg = s0 + k * per;
        if (seg < segs) {
            uint8_t *pl = lds0 + xoff + (seg >> 4) * MQ_BREC + (seg & 15) * 48 + 4 * j;
            *(uint32_t *)(pl) = r[k].p0;
            *(uint32_t *)(pl + 16) = r[k].p1;
            *(uint32_t *)(pl + 32) = r[k].p2;
            if (j == 0) {
                xsv[seg] = r[k].xs;
                xsv[segs + seg] = r[k].gs;
                xsv[2 * segs + seg] = r[k].gq;
            }
        }
    }
    if (lane == 0) __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    __builtin_amdgcn_s_setprio(0);
}

// Row sum over the four block lanes (l, l + 16, l + 32, l + 48) of a wave.
__device__ __forceinline__ float mq_sum_units(float v) {
    v += __shfl_xor(v, 16, SEPIA_WAVE);
    v += __shfl_xor(v, 32, SEPIA_WAVE);
    return v;
}

// One item: 16 rows (row0 .. row0 + 15, those >= rows repeat the last row
// and are discarded) of a matrix at base (row r at base + r * row_bytes),
// against the XQ vector at LDS offset xoff; its row sums go to red slot
// `red` (in units of P partial vectors of 16 floats).
struct MqItem {
    const uint8_t *base;
    int64_t row0, rows;
    uint32_t xoff;
    int32_t red;
};

// Workgroup geometry: nw = C * P waves; wave w is part p = w % P of items
// c = w / P, c + C, ...: of each such item it takes the quads p, p + P, ...
// of the row's nq = nb / 4 quads. Every wave has a private ring of `ring`
// bytes at LDS offset rings + w * ring, which holds S = min(4, ring / Wp KB)
// stages of a format of Wp padded words.
// xraw: LDS offset of a raw f32 copy of the workgroup's vector (0: the
// vector is read from global memory directly), orings: LDS offset of the
// rings (for the kernels whose LDS layout the host plans). conv > 0: the
// last conv waves of the workgroup DMA the vector straight into its XQ
// place and convert it there while the others stream and decode their
// first step; xraw is then the LDS offset of 16 bytes of control words.
// conv < 0: the first -conv stepping waves do that conversion before they
// issue their own weight prologue, while the other waves issue theirs (no
// waves of its own, and the vector is in XQ form long before the weight
// stream has been issued in full).
// nw: the stepping waves (C x P); a launch may run more waves than that
// (its other kind of workgroup needs more), which then take no items and no
// ring.
// C: items side by side (nw / P); S: ring stages, min(4, ring / Wp KB);
// step: the stride between a workgroup's items (the launch's workgroups per
// slot, or the matvec's grid). mP, mC, mstep: their reciprocals for mq_div,
// computed by the host, so that no wave runs a division sequence.
struct MqGeo {
    int32_t P, ring, xraw, orings, conv, nw;
    int32_t C, S, step;
    uint32_t mP, mC, mstep;
};
// floor(n / d) for n < 2^31 / d, with m = ceil(2^31 / d) from the host.
__device__ __forceinline__ uint32_t mq_div(uint32_t n, uint32_t m) { return (uint32_t)(((uint64_t)n * m) >> 31); }

// The pipeline of one wave over n_items items of format T, in two halves:
// prologue() issues the first S stages (before the workgroup stages its XQ
// vectors, so that both overlap), run() computes every step and writes the
// wave's partial row sums to red[item.red * P + p][16].
template <int T, class ItemFn>
struct MqWave {
    static constexpr int W = MQ<T>::W, Wp = MQ<T>::Wp;
    const ItemFn &item_of;
    int n_items, nq, n;        // items, quads per row, XQ columns
    uint32_t rb;               // row bytes
    int c, C, p, P, S;
    uint32_t ring;             // LDS address of this wave's ring
    const uint8_t *ringp;      // the same as a pointer
    MqLane L;
    int nqw, Tn;               // quads per item and steps of this wave
    int ik, im, islot;         // issue cursor: item, quad, ring slot
    const uint8_t *tab = nullptr;   // codebook in LDS (IQ formats)

    // Waves first, first + 1, ..., first + geo.nw - 1 share the items as
    // geo.C columns of geo.P parts; other waves get none. Wave first + k
    // keeps ring k.
    __device__ __forceinline__ MqWave(const ItemFn &f, int n_items_, int nq_, int n_, uint32_t rb_, MqGeo geo,
                                      uint8_t *ring_lds, int first = 0)
        : item_of(f), n_items(n_items_), nq(nq_), n(n_), rb(rb_) {
        const int w = mq_wave_id(), wk = w - first;
        P = geo.P;
        S = geo.S;
        C = geo.C;
        c = wk >= 0 ? (int)mq_div((uint32_t)wk, geo.mP) : 0;
        p = wk - c * P;
        ringp = ring_lds + (ptrdiff_t)wk * geo.ring;
        ring = mq_lds_addr(ringp);
        L = mq_lane();
        const int ni = (wk >= 0 && wk < C * P && n_items > c) ? (int)mq_div((uint32_t)(n_items - c + C - 1), geo.mC) : 0;
        nqw = nq > p ? (int)mq_div((uint32_t)(nq - p + P - 1), geo.mP) : 0;
        Tn = ni * nqw;
        ik = im = islot = 0;
    }
    // DMA d of a step fills stage pieces 64 d .. 64 d + 63; piece i is word
    // i % Wp (the pad word repeats the last one) of compute lane i / Wp.
    __device__ __forceinline__ void issue() {
        const MqItem it = item_of(c + ik * C);
        const uint32_t q4 = 4u * (uint32_t)(p + im * P);
        const uint32_t dst = ring + (uint32_t)islot * (uint32_t)(Wp * 1024);
        const uint32_t rmax = (uint32_t)(it.rows - 1 - it.row0);   // last valid row of the item
        const uint32_t rbase = (uint32_t)it.row0 * rb;
        // For the widest formats the lane number is made opaque here, so
        // that the per-lane parts of the Wp offsets are recomputed at each
        // issue instead of being held in registers across the whole loop
        // (an empty asm statement: it emits nothing).
        uint32_t lane = (uint32_t)L.lane;
        if constexpr (Wp >= 15) asm volatile("" : "+v"(lane));
#pragma unroll
        for (int d = 0; d < Wp; d++) {
            const uint32_t i = 64u * (uint32_t)d + lane;
            const uint32_t cl = i / (uint32_t)Wp, k = i - cl * (uint32_t)Wp;
            const uint32_t j = cl & 15u, r = j < rmax ? j : rmax;
            const uint32_t boff = (uint32_t)MQ<T>::bytes * (q4 + (cl >> 4));
            const uint32_t off = rbase + r * rb + boff - MQ<T>::shift(boff) + MQ<T>::word(k < (uint32_t)W ? k : W - 1);
            mq_dma16(it.base, off, dst + 1024u * (uint32_t)d);
        }
        if (++im == nqw) {
            im = 0;
            ++ik;
        }
        if (++islot == S) islot = 0;
    }
    __device__ __forceinline__ void prologue() {
        for (int t = 0; t < S && t < Tn; t++) issue();
    }
    // Wait for this wave's memory operations older than its prologue.
    __device__ __forceinline__ void wait_before_prologue() const { mq_wait_stages<Wp>(S < Tn ? S : Tn); }
    // The workgroup's vector: from global memory, or (geo.xraw) by LDS DMA
    // ahead of the prologue and converted once it has landed, so that the
    // vector does not queue behind the workgroup's weight stream.
    // x_issued: the caller already DMA'd the vector into the raw copy (a
    // mode-1 geometry) before work of its own, e.g. the expert selection.
    bool x_issued = false;
    // xq_ready: the workgroup already holds the XQ vector (converted in
    // place while wave 0 selected the experts); go() then only issues the
    // prologue and runs.
    bool xq_ready = false;
    __device__ __forceinline__ void start(const float *src, const MqGeo &geo, uint8_t *lds0, uint32_t xoff) {
        if (geo.xraw) {
            if (!x_issued) mq_dma_vec(src, n, mq_lds_addr(lds0 + geo.xraw));
            // every wave's vector DMAs are issued before any weight DMA, so
            // the CU's queue holds the whole vector ahead of the weights
            // (a bare s_barrier: nothing waits for the loads here)
            __builtin_amdgcn_s_barrier();
            prologue();
            wait_before_prologue();
            __syncthreads();
            mq_stage_xq_lds((const float *)(lds0 + geo.xraw), n, lds0, xoff);
        } else {
            prologue();
            mq_stage_xq(src, 0, 1, n, lds0, xoff, 0u);
        }
    }
    // The first step split around the wait for the vector: pre_first()
    // waits for its stage, refills the slot and decodes the weights (no x
    // needed); run_after() finishes it once the XQ vector is in LDS and runs
    // the remaining steps as run() does. Only for Tn >= 1.
    template <int TT = T>
    __device__ __forceinline__ typename MQ<TT>::Pre pre_first() {
        mq_wait_stages<Wp>((S < Tn ? S : Tn) - 1);
        uint4 w[W];
        const uint8_t *src = ringp + 16 * Wp * L.lane;
#pragma unroll
        for (int k = 0; k < W; k++) w[k] = *(const uint4 *)(src + 16 * k);
        __builtin_amdgcn_s_waitcnt(MQ_WC_LGKM0);
        if (S < Tn) issue();
        const uint32_t b = 4u * (uint32_t)p + (uint32_t)L.g;
        return MQ<TT>::pre(w, MQ<TT>::shift((uint32_t)MQ<TT>::bytes * b));
    }
    template <int TT = T>
    __device__ __forceinline__ void run_after(const uint8_t *lds0, float *red, const typename MQ<TT>::Pre &pr) {
        float acc;
        {
            const MqItem it = item_of(c);
            const uint32_t b = 4u * (uint32_t)p + (uint32_t)L.g;
            MqCtx x;
            x.lds0 = lds0;
            x.abase = L.a_lane ? it.xoff + MQ_BREC * b + 16u * (uint32_t)L.p : 0u;
            x.xsb = (const float *)(lds0 + it.xoff + mq_xq_planes(n)) + 16u * b;
            x.gvb = x.xsb + MQ<T>::sum_sel * (n >> 4);
            x.tab = tab;
            acc = MQ<TT>::post(pr, x);
        }
        steps(lds0, red, 1, acc);
    }
    __device__ __forceinline__ void run(const uint8_t *lds0, float *red) { steps(lds0, red, 0, 0.0f); }
    // start() and run() in one. With geo.conv the last geo.conv waves turn
    // the vector into XQ (at raised priority) while the others issue their
    // weights and decode their first step, and wait only for the XQ vector
    // to finish it; the converter waves return at once after. Every wave of
    // the workgroup calls this. CONV false compiles that path out (the host
    // never plans it for such a kernel), which keeps the kernel's registers
    // for its own pipeline.
    // SCONV: the kernel may be planned with conv < 0 (the FFN gate/up
    // launch only; compiled out of the others, which keeps their registers).
    template <bool CONV = true, bool SCONV = false>
    __device__ __forceinline__ void go(const float *src, const MqGeo &geo, uint8_t *lds0, uint32_t xoff, float *red) {
        if (xq_ready) {
            prologue();
            // a codebook the caller wrote after the vector's barrier
            if constexpr (MQ<T>::table_bytes > 0) __syncthreads();
            run(lds0, red);
            return;
        }
        if (!CONV || geo.conv == 0) {
            start(src, geo, lds0, xoff);
            run(lds0, red);
            return;
        }
        if (SCONV && geo.conv < 0) {
            const int nconv = -64 * geo.conv;
            uint32_t *ctl = (uint32_t *)(lds0 + geo.xraw);
            const bool cv = (int)threadIdx.x < nconv;
            if (threadIdx.x == 0) ctl[0] = 0u;
            if (cv) mq_xq_dma_by(src, n, lds0, xoff, 0, nconv);
            // a bare barrier: the vector's DMAs are queued ahead of every
            // weight DMA, and the control word is written
            __builtin_amdgcn_s_waitcnt(MQ_WC_LGKM0);
            __builtin_amdgcn_s_barrier();
            const uint32_t ready = 3u * (uint32_t)(-geo.conv);
            if (cv) {
                mq_xq_in_place_by(n, lds0, xoff, 0, nconv, ctl, nullptr);
                prologue();
                mq_waves_wait(ctl, ready, L.lane, nullptr);
                run(lds0, red);
                return;
            }
            prologue();
            if constexpr (MQ<T>::has_pre) {
                if (Tn > 0) {
                    const typename MQ<T>::Pre pr = pre_first();
                    mq_waves_wait(ctl, ready, L.lane, nullptr);
                    run_after(lds0, red, pr);
                }
            } else {
                mq_waves_wait(ctl, ready, L.lane, nullptr);
                run(lds0, red);
            }
            return;
        }
        const int nconv = 64 * geo.conv, first = (int)blockDim.x - nconv;
        uint32_t *ctl = (uint32_t *)(lds0 + geo.xraw);
        const bool cv = (int)threadIdx.x >= first;
        if (threadIdx.x == 0) ctl[0] = 0u;
        if (cv) mq_xq_dma_by(src, n, lds0, xoff, first, nconv);
        // a bare barrier: the vector's DMAs are queued ahead of every weight
        // DMA, and the control word (and any table in LDS) is written
        __builtin_amdgcn_s_waitcnt(MQ_WC_LGKM0);
        __builtin_amdgcn_s_barrier();
        if (cv) {
            mq_xq_in_place_by(n, lds0, xoff, first, nconv, ctl, nullptr);
            return;
        }
        prologue();
        const uint32_t ready = 3u * (uint32_t)geo.conv;
        if constexpr (!CONV) {
            return;
        } else if constexpr (MQ<T>::has_pre) {
            if (Tn > 0) {
                const typename MQ<T>::Pre pr = pre_first();
                mq_waves_wait(ctl, ready, L.lane, nullptr);
                run_after(lds0, red, pr);
            }
        } else {
            mq_waves_wait(ctl, ready, L.lane, nullptr);
            run(lds0, red);
        }
    }
    // Steps t0 .. Tn - 1 (t0 <= 1), acc0 the sum so far of step 0's item.
    __device__ __forceinline__ void steps(const uint8_t *lds0, float *red, int t0, float acc0) {
        int ck = 0, cm = 0, cslot = 0;
        float acc = acc0;
        if (t0 == 1) {
            if (++cm == nqw) {
                cm = 0;
                acc = mq_sum_units(acc);
                if (L.lane < 16) red[((int64_t)item_of(c).red * P + p) * 16 + L.lane] = acc;
                acc = 0.0f;
                ++ck;
            }
            if (++cslot == S) cslot = 0;
        }
        for (int t = t0; t < Tn; t++) {
            const int after = (Tn - 1 - t) < (S - 1) ? (Tn - 1 - t) : (S - 1);
            mq_wait_stages<Wp>(after);
            const uint8_t *src = ringp + (size_t)cslot * (Wp * 1024) + 16 * Wp * L.lane;
            const MqItem it = item_of(c + ck * C);
            const uint32_t b = 4u * (uint32_t)(p + cm * P) + (uint32_t)L.g;
            MqCtx x;
            x.lds0 = lds0;
            x.abase = L.a_lane ? it.xoff + MQ_BREC * b + 16u * (uint32_t)L.p : 0u;
            x.xsb = (const float *)(lds0 + it.xoff + mq_xq_planes(n)) + 16u * b;
            x.gvb = x.xsb + MQ<T>::sum_sel * (n >> 4);
            x.tab = tab;
            if constexpr (MqSplit<MQ<T>>::W1 > 0) {
                constexpr int W1 = MqSplit<MQ<T>>::W1, O2 = MqSplit<MQ<T>>::O2;
                uint4 wa[W1];
#pragma unroll
                for (int k = 0; k < W1; k++) wa[k] = *(const uint4 *)(src + 16 * k);
                const float a0 = MQ<T>::template part<0>(wa, x);
                // the second part's words are read only after the first is done with
                __builtin_amdgcn_sched_barrier(0);
                uint4 wb[W - O2];
#pragma unroll
                for (int k = 0; k < W - O2; k++) wb[k] = *(const uint4 *)(src + 16 * (O2 + k));
                __builtin_amdgcn_s_waitcnt(MQ_WC_LGKM0);
                if (t + S < Tn) issue();
                acc += a0 + MQ<T>::template part<1>(wb, x);
            } else {
                uint4 w[W];
#pragma unroll
                for (int k = 0; k < W; k++) w[k] = *(const uint4 *)(src + 16 * k);
                // the slot is refilled only after its words are in registers
                __builtin_amdgcn_s_waitcnt(MQ_WC_LGKM0);
                if (t + S < Tn) issue();
                acc += MQ<T>::block(w, MQ<T>::shift((uint32_t)MQ<T>::bytes * b), x);
            }
            if (++cm == nqw) {
                cm = 0;
                acc = mq_sum_units(acc);
                if (L.lane < 16) red[((int64_t)it.red * P + p) * 16 + L.lane] = acc;
                acc = 0.0f;
                ++ck;
            }
            if (++cslot == S) cslot = 0;
        }
    }
};

// Sum of the P partial vectors of red slot i, element t.
__device__ __forceinline__ float mq_red_sum(const float *red, int i, int P, int t) {
    float s = 0.0f;
    for (int p = 0; p < P; p++) s += red[((int64_t)i * P + p) * 16 + t];
    return s;
}

// ------------------------------------------------------------ matvec ------
// y = W x for one matrix of nb blocks per row (nb % 4 == 0). Workgroup k
// owns row groups rg = k, k + G, ... (G = gridDim.x), one item each.
// LDS: [zero][XQ of x][codebook (IQ formats)][red: nk x P x 16 f32][raw x, if geo.xraw]
//      [rings at geo.orings].
template <int T>
__device__ __forceinline__ void mq_mv(const uint8_t *__restrict__ W, uint64_t row_bytes, int64_t rows, int32_t nb,
                                      const float *__restrict__ x, float *__restrict__ y, MqGeo geo) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int n = 256 * nb;
    const int64_t tiles = (rows + 15) >> 4, G = geo.step;   // the grid
    const int nk = tiles > blockIdx.x ? (int)mq_div((uint32_t)(tiles - blockIdx.x + G - 1), geo.mstep) : 0;
    const uint32_t xoff = MQ_ZERO;
    uint8_t *tab = smem + xoff + mq_xq_bytes(n);   // codebook (IQ formats), then the row sums
    float *red = (float *)(tab + MQ<T>::table_bytes);
    uint8_t *rings = smem + geo.orings;
    mq_fill_table<T>(tab);
    auto item_of = [&](int i) {
        MqItem it;
        it.base = W;
        it.row0 = ((int64_t)blockIdx.x + (int64_t)i * G) * 16;
        it.rows = rows;
        it.xoff = xoff;
        it.red = i;
        return it;
    };
    MqWave<T, decltype(item_of)> wv(item_of, nk, nb >> 2, n, (uint32_t)row_bytes, geo, rings, 0);
    wv.tab = tab;
    wv.go(x, geo, smem, xoff, red);   // its first barrier also publishes the codebook
    __syncthreads();
    for (int i = threadIdx.x; i < nk * 16; i += blockDim.x) {
        const int64_t r = ((int64_t)blockIdx.x + (int64_t)(i >> 4) * G) * 16 + (i & 15);
        if (r < rows) y[r] = mq_red_sum(red, i >> 4, geo.P, i & 15);
    }
}

#define SEPIA_MQ_MV(name, T)                                                                              \
    extern "C" __global__ __launch_bounds__(1024) void sepia_mq_mv_##name(                               \
        const uint8_t *__restrict__ W, uint64_t row_bytes, int64_t rows, int32_t nb,                      \
        const float *__restrict__ x, float *__restrict__ y, MqGeo geo) {                                  \
        sepia_kernarg_warm<320>();                                                                        \
        mq_mv<T>(W, row_bytes, rows, nb, x, y, geo);                                                      \
    }

// --------------------------------------------------------- expert FFN ------
// One projection family of a stack of experts: expert e's quant rows start
// at base + e * stride, row r at + r * row_bytes; n_blocks counts 256-column
// blocks (Q8_0: super-blocks of 8 blocks).
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

// Gate/up of one slot: the workgroup owns row groups j0, j0 + jstep, ... of
// the slot's inter rows; item 2k is the gate rows of its k-th row group,
// item 2k + 1 the up rows. h[r] = silu(gate_r . x) * (up_r . x) (f32).
// LDS: [zero][XQ of x][selection: 64 i32 + 64 f32][codebook (IQ formats)]
//      [red: 2 nk x P x 16 f32][raw x][rings].
// The selection area: 64 i32 expert indices, 64 f32 weights, 16 bytes of
// control words.
#define MQ_SEL_BYTES 528
template <int T>
__device__ __forceinline__ void mq_gateup_slot(const uint8_t *Wg, const uint8_t *Wu, uint64_t row_bytes, int32_t nb,
                                               int32_t inter, int32_t j0, int32_t jstep, const float *__restrict__ x,
                                               float *__restrict__ h, MqGeo geo, bool x_issued, bool xq_ready) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int n = 256 * nb;
    const int tiles = (inter + 15) >> 4;   // jstep == geo.step
    const int nk = j0 < tiles ? (int)mq_div((uint32_t)(tiles - j0 + jstep - 1), geo.mstep) : 0;
    const uint32_t xoff = MQ_ZERO;
    uint8_t *tab = smem + xoff + mq_xq_bytes(n) + MQ_SEL_BYTES;   // codebook (IQ formats), then the row sums
    float *red = (float *)(tab + MQ<T>::table_bytes);
    uint8_t *rings = smem + geo.orings;
    mq_fill_table<T>(tab);
    auto item_of = [&](int i) {
        MqItem it;
        it.base = (i & 1) ? Wu : Wg;
        it.row0 = ((int64_t)j0 + (int64_t)(i >> 1) * jstep) * 16;
        it.rows = inter;
        it.xoff = xoff;
        it.red = i;
        return it;
    };
    MqWave<T, decltype(item_of)> wv(item_of, 2 * nk, nb >> 2, n, (uint32_t)row_bytes, geo, rings, 0);
    wv.x_issued = x_issued;
    wv.xq_ready = xq_ready;
    wv.tab = tab;
    wv.template go<true, true>(x, geo, smem, xoff, red);
    __syncthreads();
    for (int i = threadIdx.x; i < nk * 16; i += blockDim.x) {
        const int k = i >> 4, t = i & 15;
        const int64_t r = ((int64_t)j0 + (int64_t)k * jstep) * 16 + t;
        if (r < inter) h[r] = silu_f32(mq_red_sum(red, 2 * k, geo.P, t)) * mq_red_sum(red, 2 * k + 1, geo.P, t);
    }
}

// In-kernel selection for the MoE decode: with logits set, every routed
// workgroup selects from the router's logits (route.h, one wave) and
// workgroup 0 publishes the selection to idx_out / w_out for the down
// launch; with logits NULL the experts come from sel_idx (or fixed + slot).
struct MqRoute {
    const float *logits;
    const float *bias;
    int32_t n_routed, n_shared;
    float route_scale, global_scale;
    int32_t *idx_out;
    float *w_out;
};

// Workgroups [0, topk * wps_r) serve the routed slots, wps_r each
// (workgroup k: slot k / wps_r, row groups k % wps_r, + wps_r, ...), the
// next n_shared * wps_s the shared slots, wps_s each; bid is the
// workgroup's index among them. Routed slots take their expert from the
// selection, sel_idx or fixed + slot; shared slot topk + i is shared expert
// i. h is [n_slots][inter] f32. Each kind has its own geometry (geo_r,
// geo_s), planned for its format, so the rings of routed workgroups hold
// steps of the routed format, not of the larger shared one.
__device__ __forceinline__ void mq_gateup(const MqProj &gate, const MqProj &up, const MqProj &s_gate,
                                          const MqProj &s_up, const int32_t *__restrict__ sel_idx, int32_t fixed,
                                          int32_t topk, int32_t inter, int32_t wps_r, int32_t wps_s,
                                          const float *__restrict__ x, float *__restrict__ h, const MqGeo &geo_r,
                                          const MqGeo &geo_s, const MqRoute &rt, int32_t bid) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const bool rk = bid < topk * wps_r;
    const MqGeo geo = rk ? geo_r : geo_s;
    const int32_t wps = rk ? wps_r : wps_s;   // == geo.step
    const int32_t k0 = rk ? bid : bid - topk * wps_r;
    const int32_t kq = (int32_t)mq_div((uint32_t)k0, geo.mstep);
    const int32_t slot = (rk ? 0 : topk) + kq, j0 = k0 - kq * wps;
    int64_t e;
    bool x_issued = false, xq_ready = false;
    // With the selection in this launch, one workgroup publishes it with its
    // weights: the first shared one, which has time to spare (its slot needs
    // no selection), or workgroup 0 without shared experts. The other routed
    // workgroups select without the weights.
    const bool publisher = rt.n_shared > 0 ? bid == topk * wps_r : bid == 0;
    if (rt.logits && (slot < topk || publisher)) {
        const int n = (int)(256 * gate.n_blocks);
        int32_t *si = (int32_t *)(smem + MQ_ZERO + mq_xq_bytes(n));
        float *sw = (float *)(si + 64);
        uint32_t *ctl = (uint32_t *)(sw + 64);
        // A routed workgroup's waves 1.. DMA x straight into its XQ place
        // and convert it there while wave 0 selects, so the weight prologue
        // is the only thing left once the expert is known.
        const int conv = (int)blockDim.x - SEPIA_WAVE;
        xq_ready = slot < topk && conv >= 64 && (n >> 4) <= MQ_XQP * (conv >> 2);
        if (xq_ready) {
            if (threadIdx.x == 0) ctl[0] = 0u;
            __syncthreads();
            if ((int)threadIdx.x >= SEPIA_WAVE) {
                mq_xq_dma_by(x, n, smem, MQ_ZERO, SEPIA_WAVE, conv);
                // the selection is the longer chain: wave 0 goes first
                __builtin_amdgcn_s_setprio(0);
            } else {
                __builtin_amdgcn_s_setprio(3);
            }
        } else if (geo.xraw && geo.conv == 0) {
            // the vector does not depend on the selection: its DMA goes out
            // first and lands while wave 0 selects
            mq_dma_vec(x, n, mq_lds_addr(smem + geo.xraw));
            x_issued = true;
        }
        if (threadIdx.x < SEPIA_WAVE)
            route_pick_any<false>(rt.logits, rt.bias, rt.n_routed, rt.n_shared, topk, rt.route_scale,
                                  rt.global_scale, si, publisher ? sw : nullptr);
        else if (xq_ready)
            mq_xq_in_place_by(n, smem, MQ_ZERO, SEPIA_WAVE, conv, ctl, nullptr);
        __builtin_amdgcn_s_setprio(0);
        __syncthreads();
        if (publisher && threadIdx.x < topk + rt.n_shared) {
            if ((int)threadIdx.x < topk) rt.idx_out[threadIdx.x] = si[threadIdx.x];
            rt.w_out[threadIdx.x] = sw[threadIdx.x];
        }
        e = slot < topk ? (int64_t)__builtin_amdgcn_readfirstlane(si[slot]) : (int64_t)(slot - topk);
    } else {
        e = mq_slot_expert(sel_idx, fixed, slot, topk);
    }
    const MqProj &G = slot < topk ? gate : s_gate;
    const MqProj &U = slot < topk ? up : s_up;
    const uint8_t *wg = G.base + e * G.stride, *wu = U.base + e * U.stride;
    float *hs = h + (int64_t)slot * inter;
    const int32_t nb = (int32_t)G.n_blocks;
#define MQ_GU_CASE(T) \
    case T: mq_gateup_slot<T>(wg, wu, G.row_bytes, nb, inter, j0, wps, x, hs, geo, x_issued, xq_ready); break;
    switch (G.type) {
        MQ_GU_CASE(ST_Q2_K)
        MQ_GU_CASE(ST_Q3_K)
        MQ_GU_CASE(ST_Q5_K)
        MQ_GU_CASE(ST_Q6_K)
        MQ_GU_CASE(ST_Q8_0)
        MQ_GU_CASE(ST_IQ2_XS)
        MQ_GU_CASE(ST_IQ3_XXS)
        MQ_GU_CASE(ST_IQ4_XS)
    default: mq_gateup_slot<ST_Q4_K>(wg, wu, G.row_bytes, nb, inter, j0, wps, x, hs, geo, x_issued, xq_ready); break;
    }
#undef MQ_GU_CASE
}

#define SEPIA_MQ_GATEUP()                                                                                \
    extern "C" __global__ __launch_bounds__(1024) void sepia_mq_gateup(                                  \
        MqProj gate, MqProj up, MqProj s_gate, MqProj s_up, const int32_t *__restrict__ sel_idx,         \
        int32_t fixed, int32_t topk, int32_t inter, int32_t wps_r, int32_t wps_s,                        \
        const float *__restrict__ x, float *__restrict__ h, MqGeo geo_r, MqGeo geo_s, MqRoute rt) {      \
        sepia_kernarg_warm<512>();                                                                       \
        mq_gateup(gate, up, s_gate, s_up, sel_idx, fixed, topk, inter, wps_r, wps_s, x, h, geo_r, geo_s, \
                  rt, (int32_t)blockIdx.x);                                                              \
    }

// Down, one slot per workgroup: workgroups [0, topk * wps_r) serve the
// routed slots (wps_r each), the next ones the shared slots (wps_s each);
// bid is the workgroup's index among them. A workgroup owns row groups j0,
// j0 + jstep, ... of y for its slot (one item each) and stages only its
// slot's h as XQ. With a single slot (the expert FFN) it stores w * its rows
// into y. Otherwise it publishes its rows to ypart[slot] (agent-scope
// stores, waited for); with n_count > 0 it then bumps each of its row
// groups' arrival counters, and the workgroup whose arrival is the
// n_count-th adds the n_sum partial rows in slot order, weighted by sel_w
// (routed weights, then the shared gammas; the shared gamma scales the down
// output as src/sepia.c:3953-3957 does), into y and puts the counter back to
// zero -- deterministic whatever the arrival order. n_count < n_sum: the
// other slots' partial rows were published by an earlier launch.
// LDS: [zero][XQ of h_slot][codebook (IQ formats)][red: nk x P x 16 f32][flags: nk i32][raw h]
//      [rings].
template <int T>
__device__ __forceinline__ void mq_dn_slot(const uint8_t *Wd, uint64_t row_bytes, int32_t nb, int32_t inter,
                                           int64_t hidden, int32_t j0, int32_t jstep, int nk,
                                           const float *__restrict__ hs, MqGeo geo, float *red, uint8_t *rings,
                                           uint8_t *lds0) {
    uint8_t *tab = lds0 + MQ_ZERO + mq_xq_bytes(inter);
    mq_fill_table<T>(tab);
    auto item_of = [&](int i) {
        MqItem it;
        it.base = Wd;
        it.row0 = ((int64_t)j0 + (int64_t)i * jstep) * 16;
        it.rows = hidden;
        it.xoff = MQ_ZERO;
        it.red = i;
        return it;
    };
    MqWave<T, decltype(item_of)> wv(item_of, nk, nb >> 2, inter, (uint32_t)row_bytes, geo, rings, 0);
    wv.tab = tab;
    wv.template go<true>(hs, geo, lds0, MQ_ZERO, red);
}

__device__ __forceinline__ void mq_down(const MqProj &down, const MqProj &s_down, const int32_t *__restrict__ sel_idx,
                                        const float *__restrict__ sel_w, int32_t fixed, int32_t topk,
                                        int32_t n_count, int32_t n_sum, int32_t inter, int64_t hidden,
                                        const float *__restrict__ h, float *__restrict__ y, const MqGeo &geo_r,
                                        const MqGeo &geo_s, int32_t wps_r, int32_t wps_s, float *__restrict__ ypart,
                                        uint32_t *__restrict__ cnt, int32_t bid) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const bool routed = bid < topk * wps_r;
    const MqGeo geo = routed ? geo_r : geo_s;
    const int32_t jstep = routed ? wps_r : wps_s;   // == geo.step
    const int32_t k0 = routed ? bid : bid - topk * wps_r;
    const int32_t kq = (int32_t)mq_div((uint32_t)k0, geo.mstep);
    const int32_t slot = (routed ? 0 : topk) + kq, j0 = k0 - kq * jstep;
    const int64_t e = mq_slot_expert(sel_idx, fixed, slot, topk);
    const MqProj &Pj = routed ? down : s_down;
    const uint8_t *Wd = Pj.base + e * Pj.stride;
    const int tiles = (int)((hidden + 15) >> 4);
    const int nk = j0 < tiles ? (int)mq_div((uint32_t)(tiles - j0 + jstep - 1), geo.mstep) : 0;
    const size_t o_red = MQ_ZERO + mq_xq_bytes(inter) + mq_table_bytes(Pj.type);
    float *red = (float *)(smem + o_red);
    int32_t *flag = (int32_t *)(smem + o_red + (size_t)nk * geo.P * 64);
    uint8_t *rings = smem + geo.orings;
    const float *hs = h + (int64_t)slot * inter;
    const int32_t nb = (int32_t)Pj.n_blocks;
#define MQ_DN_CASE(T) \
    case T: mq_dn_slot<T>(Wd, Pj.row_bytes, nb, inter, hidden, j0, jstep, nk, hs, geo, red, rings, smem); break;
    switch (Pj.type) {
        MQ_DN_CASE(ST_Q2_K)
        MQ_DN_CASE(ST_Q3_K)
        MQ_DN_CASE(ST_Q5_K)
        MQ_DN_CASE(ST_Q6_K)
        MQ_DN_CASE(ST_Q8_0)
        MQ_DN_CASE(ST_IQ2_XS)
        MQ_DN_CASE(ST_IQ3_XXS)
        MQ_DN_CASE(ST_IQ4_XS)
    default: mq_dn_slot<ST_Q4_K>(Wd, Pj.row_bytes, nb, inter, hidden, j0, jstep, nk, hs, geo, red, rings, smem); break;
    }
#undef MQ_DN_CASE
    __syncthreads();
    if (n_sum == 1) {
        const float w = sel_w ? sel_w[0] : 1.0f;
        for (int i = threadIdx.x; i < nk * 16; i += blockDim.x) {
            const int64_t r = ((int64_t)j0 + (int64_t)(i >> 4) * jstep) * 16 + (i & 15);
            if (r < hidden) y[r] = w * mq_red_sum(red, i >> 4, geo.P, i & 15);
        }
        return;
    }
    for (int i = threadIdx.x; i < nk * 16; i += blockDim.x) {
        const int64_t r = ((int64_t)j0 + (int64_t)(i >> 4) * jstep) * 16 + (i & 15);
        if (r < hidden)
            __hip_atomic_store(&ypart[(int64_t)slot * hidden + r], mq_red_sum(red, i >> 4, geo.P, i & 15),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (n_count == 0) return;
    // Publication without release/acquire fences. Every datum that crosses
    // workgroups here is an agent-scope atomic: the partial rows are stored
    // and loaded, and the counter incremented, with relaxed agent-scope
    // atomics, which gfx950 performs at the agent's coherence point (sc1
    // stores and loads, L2-coherent atomics; the LLVM AMDGPU memory model's
    // code sequences for relaxed agent-scope atomics). What the fences would
    // add is ordering, and the hardware gives it here: s_waitcnt vmcnt(0)
    // returns only once this thread's stores are acknowledged at that point,
    // the barrier then orders them before the counter increment, and the
    // last arriver's loads are issued after it has read the final count. An
    // agent-scope release fence would also write back the whole L2 (buffer
    // write-back), which measured 0.6-1.3 us more per down launch at C3.
    __builtin_amdgcn_s_waitcnt(0);   // this thread's partial stores have completed
    __syncthreads();
    for (int k = threadIdx.x; k < nk; k += blockDim.x) {
        const uint32_t prev =
            __hip_atomic_fetch_add(&cnt[j0 + k * jstep], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        flag[k] = prev == (uint32_t)(n_count - 1);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < nk * 16; i += blockDim.x) {
        if (!flag[i >> 4]) continue;
        const int64_t r = ((int64_t)j0 + (int64_t)(i >> 4) * jstep) * 16 + (i & 15);
        if (r >= hidden) continue;
        // eight slots' loads in flight at a time, added in slot order
        float acc = 0.0f;
        for (int s0 = 0; s0 < n_sum; s0 += 8) {
            float v[8], wv[8];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const bool on = s0 + k < n_sum;
                v[k] = on ? __hip_atomic_load(&ypart[(int64_t)(s0 + k) * hidden + r], __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT)
                          : 0.0f;
                wv[k] = on && sel_w ? sel_w[s0 + k] : 1.0f;
            }
#pragma unroll
            for (int k = 0; k < 8; k++)
                if (s0 + k < n_sum) acc = __builtin_fmaf(wv[k], v[k], acc);
        }
        y[r] = acc;
    }
    for (int k = threadIdx.x; k < nk; k += blockDim.x)
        if (flag[k]) __hip_atomic_store(&cnt[j0 + k * jstep], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

#define SEPIA_MQ_DOWN()                                                                                  \
    extern "C" __global__ __launch_bounds__(1024) void sepia_mq_down(                                    \
        MqProj down, MqProj s_down, const int32_t *__restrict__ sel_idx, const float *__restrict__ sel_w, \
        int32_t fixed, int32_t topk, int32_t n_count, int32_t n_sum, int32_t inter, int64_t hidden,      \
        const float *__restrict__ h, float *__restrict__ y, MqGeo geo_r, MqGeo geo_s, int32_t wps_r,     \
        int32_t wps_s, float *__restrict__ ypart, uint32_t *__restrict__ cnt) {                          \
        sepia_kernarg_warm<448>();                                                                       \
        mq_down(down, s_down, sel_idx, sel_w, fixed, topk, n_count, n_sum, inter, hidden, h, y, geo_r,   \
                geo_s, wps_r, wps_s, ypart, cnt, (int32_t)blockIdx.x);                                   \
    }

