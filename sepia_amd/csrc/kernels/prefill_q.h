// prefill_q.h -- the prefill MoE projections of the K-quant formats Q2_K,
// Q3_K and Q4_K on the int8 matrix cores (the batched layer of prefill.h
// with these formats: the same grouping, units and combine).
//
// Activations (x per token for gate/up, h per pair for down) travel as "PQ"
// rows: per row one f32 scale s = max|v| / MQ_QMAX and per column the
// integer q = round(v / s), |q| <= MQ_QMAX + 1, written as three signed
// base-256 digits q = 65536 p0 + 256 p1 + p2 exactly as the decode path's
// XQ digits (mq.h); v^ = s q is within s / 2 + 2^-22 |v| of v (a 23-bit
// representation relative to the row's largest |v|). A 256-column block of
// a row is an 832-byte record: the digit planes p0, p1, p2 (256 bytes each,
// column order), then the sixteen 16-column sums S_j = sum of q as bf16 hi +
// lo (hi + lo within 2^-16 |S_j| of S_j) in four 16-byte groups: group g
// holds hi of S_4g .. S_4g+3, then their lo.
//
// The weights' integer codes are the B operand of v_mfma_i32_16x16x64_i8:
// Q2_K as sc * q (0..45) and Q3_K as (32 - sc) * (q - 4) (-128..124), the
// 16-weight sub-block scale folded in, each read from a per-sub-block table
// by v_perm_b32 with the 2- or 3-bit codes as the selectors; Q4_K as two
// operands q * (sc & 7) and q * (sc >> 3) whose sums combine as lo + 8 hi
// (sc * q needs 10 bits). Per weight row n and
// 256-column block (src/quants.c:104-125 and the ggml layouts of Q2_K and
// Q3_K), with C the i32 dot of the codes with q:
//   Q2_K  sum_k w_k v^_k = s (d_n C - dmin_n sum_j m_j S_j)
//   Q3_K  sum_k w_k v^_k = -s d_n C
//   Q4_K  sum_k w_k v^_k = s (d_n C - dmin_n sum_j m_j (S_2j + S_2j+1))
// C = 65536 C0 + 256 C1 + C2 over the digit planes, each plane's sum an
// exact i32 (|C_p| <= 256 * 128 * 128 = 2^22, so 256 C1 + C2 is exact too);
// the block's C goes to f32 as fma(C0, 65536, 256 C1 + C2) and accumulates
// in f32 with d_n. The min terms are 16x16x16 bf16 MFMAs over the sixteen
// sums (m exact in bf16, S as hi + lo). The row scale s multiplies the
// result once at the end.
//
// Workgroup: one unit (<= 32 pairs of one expert) x 256 weight rows (gate/up:
// 128 rows of gate and the same 128 rows of up), 8 waves; wave w computes
// 32 rows (two 16-row N tiles) x the unit's one or two 16-pair M tiles, so a
// decoded B fragment feeds 3 (or 6) MFMAs per M tile and an A fragment
// 2 N tiles. Each 256-column block arrives by LDS DMA one block ahead (two
// stages): the unit's 32 PQ records (padded to 848 bytes, so the 16 pair
// rows of an A read hit 16 bank groups) and each weight row's 16-byte-aligned
// window that holds the block (an odd number of 16-byte pieces per row).
#pragma once
#include "prefill.h"

#define PQ_REC 832                     // bytes of a 256-column PQ record
#define PQ_ROWS 256                    // weight rows of a workgroup
#define PQ_LDS_TOP (PF_LDS_BYTES - 3 * PF_MT * 4)   // row tables: roff, pair, scale

template <int T> struct PqFmt;
// BB: block bytes; PW: 16-byte pieces of a staged weight row; RP: pieces of
// a PQ record the format reads (the planes, and the sums where it has min
// terms); AP: pieces of a staged record (RP, then padding); SW: weight
// stages (LDS: 2 record stages + SW weight stages of 256 rows within 160
// KB). Each row's block is staged from the 4-byte boundary at or below its
// start (every format here: rows of 4-byte multiples, so the offset o of
// the block in its staged row is the same for every row of a block: 0, or 0
// and 2 for Q3_K), so a K step's codes are one (Q3_K: two) aligned 16-byte
// reads. Strides: on gfx950, 16-byte reads of 16 rows at a stride of 2 mod
// 4 pieces measured free of bank conflicts (odd strides two-way), so AP and
// PW are 2 mod 4.
template <> struct PqFmt<ST_Q2_K> { static constexpr int BB = 84, PW = 6, RP = 52, AP = 54, SW = 3; };
template <> struct PqFmt<ST_Q3_K> { static constexpr int BB = 110, PW = 10, RP = 48, AP = 50, SW = 2; };
template <> struct PqFmt<ST_Q4_K> { static constexpr int BB = 144, PW = 10, RP = 52, AP = 54, SW = 2; };

// ------------------------------------------------------------- rows -> PQ --
// Wave max over 64 lanes.
__device__ __forceinline__ float pq_wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// One workgroup per row: src row r (K floats at src + r * ld) into its PQ
// records at pq + r * ldq and its scale at scale[r].
extern "C" __global__ __launch_bounds__(256) void sepia_pf_quant(const float *__restrict__ src, int64_t ld,
                                                                 int64_t K, uint8_t *__restrict__ pq, int64_t ldq,
                                                                 float *__restrict__ scale) {
    __shared__ float red[4];
    const int64_t r = blockIdx.x;
    const float *row = src + r * ld;
    float m = 0.0f;
    for (int64_t c = 4 * (int64_t)threadIdx.x; c < K; c += 1024) {
        const float4 v = *(const float4 *)(row + c);
        // a NaN or an infinity makes the row's scale infinite (mq_nonfinite_max)
        m = mq_nonfinite_max(fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)))),
                             (v.x + v.y) + (v.z + v.w));
    }
    m = pq_wave_max(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    // |v * inv| <= QMAX (1 + 2^-22): rcp is within 1 ulp
    const float inv = (m > 0.0f) ? MQ_QMAX * __builtin_amdgcn_rcpf(m) : 0.0f;
    if (threadIdx.x == 0) scale[r] = m * (1.0f / MQ_QMAX);
    uint8_t *out = pq + r * ldq;
    for (int64_t seg = threadIdx.x; seg < K / 16; seg += 256) {
        const float4 *x4 = (const float4 *)(row + 16 * seg);
        uint32_t q[16];
        int32_t sum = 0;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const float4 t = x4[c];
            const float a[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int32_t v = mq_round(a[i] * inv);
                sum += v;
                q[4 * c + i] = (uint32_t)v + 0x8080u;
            }
        }
        uint32_t w0[4], w1[4], w2[4];
#pragma unroll
        for (int w = 0; w < 4; w++) {
            // as xq_segment (mq.h): byte 2 of q + 0x8080 is p0, bytes 1 and 0 are p1 + 128, p2 + 128
            const uint32_t t01 = __builtin_amdgcn_perm(q[4 * w + 1], q[4 * w], 0x05010400u);
            const uint32_t t23 = __builtin_amdgcn_perm(q[4 * w + 3], q[4 * w + 2], 0x05010400u);
            const uint32_t u01 = __builtin_amdgcn_perm(q[4 * w + 1], q[4 * w], 0x06020602u);
            const uint32_t u23 = __builtin_amdgcn_perm(q[4 * w + 3], q[4 * w + 2], 0x06020602u);
            w2[w] = __builtin_amdgcn_perm(t23, t01, 0x05040100u) ^ 0x80808080u;
            w1[w] = __builtin_amdgcn_perm(t23, t01, 0x07060302u) ^ 0x80808080u;
            w0[w] = __builtin_amdgcn_perm(u23, u01, 0x05040100u);
        }
        uint8_t *rec = out + (seg >> 4) * PQ_REC;
        const int j = (int)(seg & 15);
        *(uint4 *)(rec + 16 * j) = make_uint4(w0[0], w0[1], w0[2], w0[3]);
        *(uint4 *)(rec + 256 + 16 * j) = make_uint4(w1[0], w1[1], w1[2], w1[3]);
        *(uint4 *)(rec + 512 + 16 * j) = make_uint4(w2[0], w2[1], w2[2], w2[3]);
        // S = hi + lo: hi = bf16(S), lo = bf16 of the exact integer remainder
        const __bf16 hi = (__bf16)(float)sum;
        const __bf16 lo = (__bf16)(float)(sum - (int32_t)(float)hi);
        *(__bf16 *)(rec + 768 + 16 * (j >> 2) + 2 * (j & 3)) = hi;
        *(__bf16 *)(rec + 776 + 16 * (j >> 2) + 2 * (j & 3)) = lo;
    }
}

// --------------------------------------------------------------- staging --
// LDS: [records of block b: 2 stages][weight windows of block b: SW stages]
// [row tables]. A record stage holds the unit's PQ records of the block
// (record m at 16 AP m: its first RP pieces of 16 bytes, then padding
// pieces, piece 0 again). A weight stage holds each weight row's block at
// 16 PW k + o for row k, in PW pieces from the 4-byte boundary at or below
// the block's start (the offset o). A piece that would end more than 2
// bytes past the block takes the block's last 16 bytes instead (Q2_K: bytes
// 68..83 at 80, so d and dmin sit at 92 and 94); pieces past the block's
// end take piece 0 again. So no read passes the 4-byte word that holds the
// block's last byte (Q3_K reads at most 2 bytes past it, within that word).
// Gate/up stages carry 128 gate rows, then the same 128 up rows; down
// stages 256 rows. A wave instruction moves 64 pieces (1 KB) of
// one stage; wave w issues instructions w, w + 8, ... of each. Their lane
// offsets are fixed for the workgroup but for the block term, so they are
// computed once.
template <int T, bool GU>
struct PqDma {
    static constexpr int BB = PqFmt<T>::BB, PW = PqFmt<T>::PW, AP = PqFmt<T>::AP, RP = PqFmt<T>::RP;
    static constexpr int NA = (PF_MT * AP + 63) / 64, KA = (NA + 7) / 8;
    static constexpr int NW = PQ_ROWS * PW / 64, KW = NW / 8;   // NW: 24, 40, 40
    // wave w issues weight instructions KW w .. KW w + KW - 1: exactly the
    // stage rows 32 w .. 32 w + 31 it decodes, so no other wave reads them
    static_assert(NW % 8 == 0 && 64 * KW == 32 * PW, "a wave stages its own 32 rows");
    static_assert(PF_MT * AP % 64 == 0, "a record stage is whole DMA instructions");
    uint32_t a[KA];            // record piece offsets at block 0
    uint32_t r[KW], c16[KW];   // row offset from the matrix base; offset of the lane's piece
    __device__ __forceinline__ void init(const uint32_t *roff, const uint8_t *W0, const uint8_t *W1,
                                         uint64_t row_bytes, int64_t r0) {
        const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
        for (int k = 0; k < KA; k++) {
            const int q = 64 * (w + 8 * k) + lane, m = q / AP, c = q - m * AP;
            a[k] = q < PF_MT * AP ? roff[m] + 16u * (uint32_t)(c < RP ? c : 0) : 0u;
        }
#pragma unroll
        for (int k = 0; k < KW; k++) {
            const int jj = KW * w + k;
            const int mat = GU ? jj / (NW / 2) : 0, j1 = GU ? jj - mat * (NW / 2) : jj;
            const int q = 64 * j1 + lane, kr = q / PW, c = q - kr * PW;
            r[k] = (uint32_t)((uint64_t)(r0 + kr) * row_bytes);
            c16[k] = 16 * c >= BB ? 0u : 16 * c + 16 <= BB + 2 ? 16u * (uint32_t)c : (uint32_t)(BB - 16);
        }
    }
    // this wave's weight instructions per block
    static __device__ __forceinline__ int n_w() { return KW; }
    __device__ __forceinline__ void issue_a(int64_t b, uint8_t *As, const uint8_t *pq) const {
        const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
        const uint32_t ab = (uint32_t)b * PQ_REC;
#pragma unroll
        for (int k = 0; k < KA; k++) {
            const int jj = w + 8 * k;
            if (jj < NA) pf_dma16(pq, a[k] + ab, pf_lds(As + 1024 * jj));
        }
    }
    __device__ __forceinline__ void issue_w(int64_t b, uint8_t *Ws, const uint8_t *W0, const uint8_t *W1) const {
        const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
        const uint32_t wb = (uint32_t)b * BB;
#pragma unroll
        for (int k = 0; k < KW; k++) {
            const int jj = KW * w + k;
            pf_dma16((GU && jj >= NW / 2) ? W1 : W0, ((r[k] + wb) & ~3u) + c16[k], pf_lds(Ws + 1024 * jj));
        }
    }
};

// ------------------------------------------------------------- decoders --
typedef const __attribute__((address_space(3))) uint32_t pq_lds_u32;
typedef const __attribute__((address_space(3))) uint16_t pq_lds_u16;
typedef const __attribute__((address_space(3))) uint8_t pq_lds_u8;
__device__ __forceinline__ uint32_t pq_u8(const uint8_t *p) { return *(pq_lds_u8 *)(size_t)pf_lds(p); }
__device__ __forceinline__ uint32_t pq_u16(const uint8_t *p) { return *(pq_lds_u16 *)(size_t)pf_lds(p); }
__device__ __forceinline__ float pq_h2f(const uint8_t *p) { return f16_bits_to_f32(pq_u16(p)); }
// Five dwords from the dword holding p, for p at most 3 bytes past a
// 16-byte boundary (two aligned 16-byte reads): with sh = 8 (p & 3), the
// funnel shift of (D[i + 1], D[i]) by sh + t is bytes 4 i .. 4 i + 3 from
// p, moved down t bits.
struct PqWin {
    uint32_t d[5];
    uint32_t sh;
};
typedef uint32_t pq_u4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ PqWin pq_win(const uint8_t *p) {
    const uint32_t a = pf_lds(p), a16 = a & ~15u;
    const pq_u4 lo = *(const __attribute__((address_space(3))) pq_u4 *)(size_t)a16;
    const pq_u4 hi = *(const __attribute__((address_space(3))) pq_u4 *)(size_t)(a16 + 16u);
    PqWin r;
#pragma unroll
    for (int i = 0; i < 4; i++) r.d[i] = lo[i];
    r.d[4] = hi[0];
    r.sh = 8u * (a & 3u);
    return r;
}
__device__ __forceinline__ uint32_t pq_fsh(uint32_t hi, uint32_t lo, uint32_t n) {
    return __builtin_amdgcn_alignbit(hi, lo, n);
}
// 16 bytes at a 16-byte-aligned LDS address (one ds_read_b128); u32 at a
// 4-byte-aligned one.
__device__ __forceinline__ pq_u4 pq_b128(const uint8_t *p) {
    return *(const __attribute__((address_space(3))) pq_u4 *)(size_t)pf_lds(p);
}
__device__ __forceinline__ uint32_t pq_u32(const uint8_t *p) { return *(pq_lds_u32 *)(size_t)pf_lds(p); }

// Q2_K (ggml): weight k = 128 h + 32 s + 16 g' + l: q = (qs[32 h + 16 g' + l]
// >> 2 s) & 3, sub-block k / 16 with scale byte (sc lo nibble, m hi nibble).
// K step j (64 columns), lane group g: h = j >> 1, s = 2 (j & 1) + (g >> 1),
// g' = g & 1, sub-block 4 j + g. Codes sc * q by v_perm from the table
// [0, sc, 2 sc, 3 sc] (selector q picks its byte q). The decoders take
// their LDS bytes as arguments: the block loop reads a K step's window
// ahead of the matrix ops of the step before (pq_block). The staged block
// is 16-byte aligned: a window is one 16-byte read.
__device__ __forceinline__ pq_u4 pq_w_q2k(const uint8_t *blk, int j, int g) {
    return pq_b128(blk + 16 + 32 * (j >> 1) + 16 * (g & 1));
}
// sc4: scale bytes 0..15; wq: pq_w_q2k(blk, j, g)
__device__ __forceinline__ mq_v4i pq_b_q2k(const pq_u4 &sc4, const pq_u4 &wq, int j, int g) {
    const uint32_t sc = __builtin_amdgcn_ubfe(sc4[j], 8u * (uint32_t)g, 4u);   // byte 4 j + g, low nibble
    // [0, sc, 2 sc, 3 sc]: the 24-bit product [sc, 2 sc, 3 sc, 0] moved up a byte by v_perm
    // (a shift would fold into a 32-bit constant and a full-width multiply)
    const uint32_t t3 = (uint32_t)__umul24(sc, 0x030201u);
    const uint32_t tab = __builtin_amdgcn_perm(t3, t3, 0x0201000cu);
    const uint32_t sh = 2u * (uint32_t)(2 * (j & 1) + (g >> 1));
    mq_v4i r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        // selectors 0..3 pick bytes of the second operand, the table
        r[i] = (int32_t)__builtin_amdgcn_perm(0u, tab, (wq[i] >> sh) & 0x03030303u);
    }
    return r;
}
// Q3_K (ggml): Q2_K's indexing of qs (at 32); the high bit of q is bit
// (4 h + s) of hmask[16 g' + l] (at 0), q - 4 unless it is set; 6-bit scale
// sc of sub-block 4 j + g (q3_scale's packing, at 96). Codes (32 - sc) *
// (u - 4), u = low bits | high bit << 2, by v_perm from the 8-byte table
// a * (u - 4), a = 32 - sc.
__device__ __forceinline__ PqWin pq_w_q3k(const uint8_t *blk, int j, int g) {
    return pq_win(blk + 32 + 32 * (j >> 1) + 16 * (g & 1));
}
// lb: scale byte 96 + 4 (j & 1) + g; hb: byte 104 + g; wq: pq_w_q3k(blk, j,
// g); wh: the hmask window pq_win(blk + 16 (g & 1))
__device__ __forceinline__ mq_v4i pq_b_q3k(uint32_t lb, uint32_t hb, const PqWin &wq, const PqWin &wh, int j,
                                           int g) {
    const uint32_t lo4 = (lb >> (4 * (j >> 1))) & 15u;
    const uint32_t hi2 = (hb >> (2 * j)) & 3u;
    const uint32_t a = 32u - (lo4 | (hi2 << 4));           // two's complement of a, a in [-31, 32]
    const uint32_t a8 = a & 255u, na8 = (0u - a) & 255u;   // a and -a mod 256
    const uint32_t t01 = a8 << 16, t23 = (uint32_t)__umul24(a8, 0x030002u);
    const uint32_t t45 = (uint32_t)__umul24(na8, 0x030004u), t67 = (uint32_t)__umul24(na8, 0x010002u);
    const uint32_t thi = __builtin_amdgcn_perm(t23, t01, 0x06040200u);   // a * [0, 1, 2, 3]
    const uint32_t tlo = __builtin_amdgcn_perm(t67, t45, 0x06040200u);   // a * [-4, -3, -2, -1]
    const int s = 2 * (j & 1) + (g >> 1), bit = 4 * (j >> 1) + s;
    const uint32_t shq = wq.sh + 2u * (uint32_t)s;
    // bit `bit` of each hmask byte to bit 2: a right funnel shift by
    // sh + bit - 2, or (sh = 0, bit < 2) a left rotate; the bits a rotate or
    // shift brings in never reach bit 2 of a byte
    const int hs = (int)wh.sh + bit - 2;
    mq_v4i r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t hsrc = (hs >= 0) ? wh.d[i + 1] : wh.d[i];
        const uint32_t hb = pq_fsh(hsrc, wh.d[i], (uint32_t)hs & 31u);
        const uint32_t u = (pq_fsh(wq.d[i + 1], wq.d[i], shq) & 0x03030303u) | (hb & 0x04040404u);
        r[i] = (int32_t)__builtin_amdgcn_perm(thi, tlo, u);
    }
    return r;
}
// Q4_K (src/quants.c:104-125): weight k = 64 p + 32 n + l: nibble n of
// qs[32 p + l] (at 16), 32-weight sub-block 2 p + n with its 6-bit (sc, m)
// pair. K step j, lane group g: codes k = 64 j + 16 g + l = nibble g >> 1
// of qs[32 j + 16 (g & 1) + l], sub-block 2 j + (g >> 1). sc * q needs 10
// bits, so the codes go in as two operands, q * (sc & 7) and q * (sc >> 3)
// (each <= 105; the products of a byte never carry into the next, so a
// packed 16-bit multiply makes them), whose i32 sums combine as lo + 8 hi.
struct PqQ4 {
    mq_v4i lo, hi;
};
typedef unsigned short pq_u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pq_mul16(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(pq_u16x2, a) * __builtin_bit_cast(pq_u16x2, b));
}
__device__ __forceinline__ pq_u4 pq_w_q4k(const uint8_t *blk, int j, int g) {
    return pq_b128(blk + 16 + 32 * j + 16 * (g & 1));
}
// wq: pq_w_q4k(blk, j, g) (16-byte-aligned staging); sc: the 6-bit scale of
// sub-block 2 j + (g >> 1)
__device__ __forceinline__ PqQ4 pq_b_q4k(const pq_u4 &wq, int g, uint32_t sc) {
    const uint32_t sh = 4u * (uint32_t)(g >> 1);
    const uint32_t slo = (uint32_t)__umul24(sc & 7u, 0x10001u), shi = (uint32_t)__umul24(sc >> 3, 0x10001u);
    PqQ4 r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t q = (wq[i] >> sh) & 0x0F0F0F0Fu;
        r.lo[i] = (int32_t)pq_mul16(q, slo);
        r.hi[i] = (int32_t)pq_mul16(q, shi);
    }
    return r;
}
// 6-bit (sc, m) of Q4_K sub-block jj (k4_scale_min) from the block's first
// 16 bytes p0 (d, dmin, then the 12 scale bytes: dwords 1..3).
__device__ __forceinline__ void pq_q4k_sm(const pq_u4 &p0, int jj, uint32_t &sc, uint32_t &mn) {
    if (jj < 4) {
        sc = __builtin_amdgcn_ubfe(p0[1], 8u * (uint32_t)jj, 6u);
        mn = __builtin_amdgcn_ubfe(p0[2], 8u * (uint32_t)jj, 6u);
    } else {
        const uint32_t o = 8u * (uint32_t)(jj - 4);
        sc = __builtin_amdgcn_ubfe(p0[3], o, 4u) | (__builtin_amdgcn_ubfe(p0[1], o + 6u, 2u) << 4);
        mn = __builtin_amdgcn_ubfe(p0[3], o + 4u, 4u) | (__builtin_amdgcn_ubfe(p0[2], o + 6u, 2u) << 4);
    }
}

// ----------------------------------------------------------- projection --
// acc (+)= this block's share for both N tiles and MT M tiles.
typedef short pq_s16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t pq_u2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ pq_s16x4 pq_bf4(float a, float b, float c, float d) {
    __bf16 h[4] = {(__bf16)a, (__bf16)b, (__bf16)c, (__bf16)d};
    return *(const pq_s16x4 *)h;
}
// 256 C1 + C2 is exact in i32; the sum goes to f32 once.
__device__ __forceinline__ float pq_comb(int32_t c0, int32_t c1, int32_t c2) {
    return __builtin_fmaf((float)c0, 65536.0f, (float)(int32_t)(((uint32_t)c1 << 8) + (uint32_t)c2));
}

// A block's first LDS reads of the lane's two weight rows (scales and the
// first K steps' windows): the wave staged those rows itself, so pq_proj
// issues them before the block's barrier.
struct PqHead {
    pq_u4 a[2], b[2];         // Q2_K: scale bytes, window 0; Q4_K: first 16 bytes, window 0
    PqWin wq[2], wh[2];       // Q3_K: window 0, hmask window
    uint32_t sb[2][2], hb[2];   // Q3_K scale bytes 96 + g, 100 + g and hmask bits byte 104 + g
    uint32_t sc[2];           // Q4_K: 6-bit scale of sub-block g >> 1
};
template <int T>
__device__ __forceinline__ PqHead pq_head(const uint8_t *blk0, const uint8_t *blk1) {
    const int g = (threadIdx.x & 63) >> 4;
    const uint8_t *blk[2] = {blk0, blk1};
    PqHead h;
#pragma unroll
    for (int t = 0; t < 2; t++) {
        if constexpr (T == ST_Q2_K) {
            h.a[t] = pq_b128(blk[t]);
            h.b[t] = pq_w_q2k(blk[t], 0, g);
        } else if constexpr (T == ST_Q3_K) {
            h.sb[t][0] = pq_u8(blk[t] + 96 + g);
            h.sb[t][1] = pq_u8(blk[t] + 100 + g);
            h.hb[t] = pq_u8(blk[t] + 104 + g);
            h.wh[t] = pq_win(blk[t] + 16 * (g & 1));
            h.wq[t] = pq_w_q3k(blk[t], 0, g);
        } else {
            uint32_t mn;
            h.a[t] = pq_b128(blk[t]);
            pq_q4k_sm(h.a[t], g >> 1, h.sc[t], mn);
            h.b[t] = pq_w_q4k(blk[t], 0, g);
        }
    }
    return h;
}

template <int T, int MT>
__device__ __forceinline__ void pq_block(pf_f32x4 (&acc)[2][2], const uint8_t *As, const uint8_t *blk0,
                                         const uint8_t *blk1, const PqHead &hd) {
    const int l = threadIdx.x & 63, n = l & 15, g = l >> 4;
    const uint8_t *blk[2] = {blk0, blk1};
    // A fragment of plane p, M tile mt, columns c0 .. (lane: pair 16 mt + n, 16 or 8 bytes at group g)
    constexpr int APB = 16 * PqFmt<T>::AP;
    auto a_at = [&](int mt, int p, int col) { return As + (16 * mt + n) * APB + 256 * p + col; };
    if constexpr (T == ST_Q2_K || T == ST_Q3_K) {
        mq_v4i C[2][MT][3];
        // the block's scale bytes and first window come in the head; a
        // window serves two K steps, and the second is read after step 1's
        // decode, ahead of step 1's matrix ops
        uint32_t sb[2][2], hb[2];
        pq_u4 sc4[2], w2[2];
        PqWin wq[2], wh[2];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            sc4[t] = hd.a[t];
            w2[t] = hd.b[t];
            sb[t][0] = hd.sb[t][0];
            sb[t][1] = hd.sb[t][1];
            hb[t] = hd.hb[t];
            wh[t] = hd.wh[t];
            wq[t] = hd.wq[t];
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            mq_v4i B[2];
#pragma unroll
            for (int t = 0; t < 2; t++) {
                if constexpr (T == ST_Q2_K) B[t] = pq_b_q2k(sc4[t], w2[t], j, g);
                else B[t] = pq_b_q3k(sb[t][j & 1], hb[t], wq[t], wh[t], j, g);
            }
            if (j == 1) {
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    if constexpr (T == ST_Q2_K) w2[t] = pq_w_q2k(blk[t], 2, g);
                    else wq[t] = pq_w_q3k(blk[t], 2, g);
                }
                __builtin_amdgcn_sched_barrier(0);   // keep the reads ahead of the matrix ops
            }
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
#pragma unroll
                for (int p = 0; p < 3; p++) {
                    const mq_v4i a = *(const mq_v4i *)a_at(mt, p, 64 * j + 16 * g);
#pragma unroll
                    for (int t = 0; t < 2; t++)
                        C[t][mt][p] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, B[t], j ? C[t][mt][p] : mq_v4i{0, 0, 0, 0},
                                                                           0, 0, 0);
                }
            }
        }
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const float d = pq_h2f(blk[t] + (T == ST_Q2_K ? 92 : 108)), dn = T == ST_Q2_K ? d : -d;
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    acc[t][mt][i] = __builtin_fmaf(dn, pq_comb(C[t][mt][0][i], C[t][mt][1][i], C[t][mt][2][i]),
                                                   acc[t][mt][i]);
        }
    } else {   // Q4_K
        mq_v4i C[2][MT][3][2];
        // step j + 1's window and scale are read after step j's decode,
        // ahead of step j's matrix ops
        pq_u4 wq[2], p0[2];   // p0: the block's first 16 bytes (d, dmin, scales)
        uint32_t sc[2];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            p0[t] = hd.a[t];
            sc[t] = hd.sc[t];
            wq[t] = hd.b[t];
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            PqQ4 B[2];
#pragma unroll
            for (int t = 0; t < 2; t++) B[t] = pq_b_q4k(wq[t], g, sc[t]);
            if (j < 3) {
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    uint32_t mn;
                    pq_q4k_sm(p0[t], 2 * (j + 1) + (g >> 1), sc[t], mn);
                    wq[t] = pq_w_q4k(blk[t], j + 1, g);
                }
                __builtin_amdgcn_sched_barrier(0);   // keep the reads ahead of the matrix ops
            }
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
#pragma unroll
                for (int p = 0; p < 3; p++) {
                    const mq_v4i a = *(const mq_v4i *)a_at(mt, p, 64 * j + 16 * g);
#pragma unroll
                    for (int t = 0; t < 2; t++) {
                        C[t][mt][p][0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                            a, B[t].lo, j ? C[t][mt][p][0] : mq_v4i{0, 0, 0, 0}, 0, 0, 0);
                        C[t][mt][p][1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                            a, B[t].hi, j ? C[t][mt][p][1] : mq_v4i{0, 0, 0, 0}, 0, 0, 0);
                    }
                }
            }
        }
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const float d = pq_h2f(blk[t]);
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    // plane sums lo + 8 hi: |.| <= 9 * 256 * 105 * 128 < 2^25, each to f32 on its own
                    float c[3];
#pragma unroll
                    for (int p = 0; p < 3; p++)
                        c[p] = (float)(int32_t)(((uint32_t)C[t][mt][p][1][i] << 3) + (uint32_t)C[t][mt][p][0][i]);
                    const float f = __builtin_fmaf(c[0], 65536.0f, __builtin_fmaf(c[1], 256.0f, c[2]));
                    acc[t][mt][i] = __builtin_fmaf(d, f, acc[t][mt][i]);
                }
        }
    }
    if constexpr (T == ST_Q2_K || T == ST_Q4_K) {
        // min terms: B[k = sub-block 4 g + i][n] = m (Q4_K: m of 32-column sub-block k / 2)
#pragma unroll
        for (int t = 0; t < 2; t++) {
            pq_s16x4 bm;
            float dmin;
            if constexpr (T == ST_Q2_K) {
                const uint32_t v = pq_u32(blk[t] + 4 * g) >> 4;
                bm = pq_bf4((float)(v & 15u), (float)((v >> 8) & 15u), (float)((v >> 16) & 15u), (float)((v >> 24) & 15u));
                dmin = pq_h2f(blk[t] + 94);
            } else {
                uint32_t s0, m0, s1, m1;
                const pq_u4 p0 = pq_b128(blk[t]);
                pq_q4k_sm(p0, 2 * g, s0, m0);
                pq_q4k_sm(p0, 2 * g + 1, s1, m1);
                bm = pq_bf4((float)m0, (float)m0, (float)m1, (float)m1);
                dmin = pq_h2f(blk[t] + 2);
            }
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                // group g of the sums: hi of S_4g .. S_4g+3, then their lo
                const pq_u4 sv = pq_b128(As + (16 * mt + n) * APB + 768 + 16 * g);
                const pq_s16x4 shi = __builtin_bit_cast(pq_s16x4, (pq_u2){sv[0], sv[1]});
                const pq_s16x4 slo = __builtin_bit_cast(pq_s16x4, (pq_u2){sv[2], sv[3]});
                pf_f32x4 cm = {0.0f, 0.0f, 0.0f, 0.0f};
                cm = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(shi, bm, cm, 0, 0, 0);
                cm = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(slo, bm, cm, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; i++) acc[t][mt][i] = __builtin_fmaf(-dmin, cm[i], acc[t][mt][i]);
            }
        }
    }
}

// s_waitcnt vmcnt(n) for a wave-uniform n <= MAX (a short compare chain
// instead of pf_wait_vm's switch over every count).
template <int MAX>
__device__ __forceinline__ void pq_wait_vm(int n) {
    if constexpr (MAX <= 0) {
        __builtin_amdgcn_s_waitcnt(mq_wc_vm(0));
    } else {
        if (n >= MAX) __builtin_amdgcn_s_waitcnt(mq_wc_vm(MAX));
        else pq_wait_vm<MAX - 1>(n);
    }
}

// One projection workgroup (see the top of the file). GU: rows r0 .. r0 +
// 127 of gate (W0) and up (W1), h[pair][row] = silu(gate) * up in f32;
// down: rows r0 .. r0 + 255 of W0, out[pair][row] in f32. ld_out: floats
// per output row (I for h, H for the down partials).
template <int T, bool GU, int MT>
__device__ __forceinline__ void pq_proj(uint8_t *smem, const uint8_t *W0, const uint8_t *W1, uint64_t row_bytes,
                                        int64_t nb, const uint8_t *pq, const uint32_t *roff, const int32_t *pair,
                                        const float *srow, int nv, int64_t r0, float *__restrict__ out,
                                        int64_t ld_out) {
    constexpr int BB = PqFmt<T>::BB, PW = PqFmt<T>::PW, SW = PqFmt<T>::SW;
    constexpr uint32_t a_bytes = PF_MT * 16 * PqFmt<T>::AP, w_bytes = PQ_ROWS * PW * 16;
    static_assert(2 * a_bytes + SW * w_bytes <= PQ_LDS_TOP, "LDS stages");
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63, n = l & 15, g = l >> 4;
    const int mat = GU ? (w >> 2) : 0;
    const int rho0 = GU ? 128 * mat + 32 * (w & 3) : 32 * w;   // stage row of N tile 0
    const int64_t grow0 = r0 + (GU ? 32 * (w & 3) : 32 * w);   // its global row
    auto a_stage = [&](int b) { return smem + (uint32_t)(b & 1) * a_bytes; };
    auto w_stage = [&](int b) { return smem + 2 * a_bytes + (uint32_t)b % SW * w_bytes; };
    PqDma<T, GU> dma;
    dma.init(roff, W0, W1, row_bytes, r0);
    const int nwi = PqDma<T, GU>::n_w();
    pf_f32x4 acc[2][2];
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int mt = 0; mt < 2; mt++) acc[t][mt] = pf_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // records one block ahead, weights SW - 1 blocks ahead; in issue order
    // the DMAs of a block b are A_b, then W_(b + SW - 2)
    const int nbi = (int)nb;   // 256-column blocks of a row (K / 256)
    dma.issue_a(0, a_stage(0), pq);
    for (int c = 0; c < SW - 1 && c < nbi; c++) dma.issue_w(c, w_stage(c), W0, W1);
    for (int b = 0; b < nbi; b++) {
        // everything up to A_b and W_b; the weights of blocks b + 1 .. b + SW - 2 may fly
        const int ahead = (nbi - 1 - b) < (SW - 2) ? (nbi - 1 - b) : (SW - 2);
        pq_wait_vm<PqDma<T, GU>::KW * (SW - 2)>(nwi * ahead);
        const uint8_t *Ws = w_stage(b);
        const uint8_t *blk[2];
#pragma unroll
        for (int t = 0; t < 2; t++)   // the block at offset o of its staged row (rows of 4-byte multiples)
            blk[t] = Ws + (uint32_t)(rho0 + 16 * t + n) * (PW * 16) + (((uint32_t)b * BB) & 3u);
        // this wave's own weight rows have landed: their first reads go out
        // before the barrier, which then covers only the records (A_b staged
        // by every wave; block b - 1's reads of the stage A_(b+1) refills are
        // all used, so complete). The asm statements keep the compiler from
        // moving memory accesses across the bare barrier.
        const PqHead hd = pq_head<T>(blk[0], blk[1]);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (b + 1 < nbi) dma.issue_a(b + 1, a_stage(b + 1), pq);
        if (b + SW - 1 < nbi) dma.issue_w(b + SW - 1, w_stage(b + SW - 1), W0, W1);
        pq_block<T, MT>(acc, a_stage(b), blk[0], blk[1], hd);
    }
    // y = s_pair * acc; lane: pairs 16 mt + 4 g + i, rows grow0 + 16 t + n
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float s = srow[16 * mt + 4 * g + i];
#pragma unroll
            for (int t = 0; t < 2; t++) acc[t][mt][i] *= s;
        }
    if constexpr (GU) {
        __syncthreads();   // every wave is done with the stages
        float *xch = (float *)smem + ((w & 3) * 64 + l) * 16;
        if (mat) {
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int mt = 0; mt < 2; mt++) *(pf_f32x4 *)(xch + 8 * t + 4 * mt) = acc[t][mt];
        }
        __syncthreads();
        if (mat) return;
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const pf_f32x4 u = *(const pf_f32x4 *)(xch + 8 * t + 4 * mt);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int m = 16 * mt + 4 * g + i;
                    if (m < nv) out[(int64_t)pair[m] * ld_out + grow0 + 16 * t + n] = silu_f32(acc[t][mt][i]) * u[i];
                }
            }
    } else {
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int m = 16 * mt + 4 * g + i;
                    if (m < nv) out[(int64_t)pair[m] * ld_out + grow0 + 16 * t + n] = acc[t][mt][i];
                }
    }
}

// The unit's tables at the top of the LDS: roff[m] = byte offset of pair
// m's PQ row (rows past nv repeat pair 0's), pair[m], srow[m] = its scale.
__device__ __forceinline__ void pq_unit_rows(const int32_t *pairs, int nv, bool by_token, int32_t n_sel,
                                             int64_t ldq, const float *scale, uint8_t *smem, uint32_t *&roff,
                                             int32_t *&pair, float *&srow) {
    roff = (uint32_t *)(smem + PQ_LDS_TOP);
    pair = (int32_t *)(roff + PF_MT);
    srow = (float *)(pair + PF_MT);
    if (threadIdx.x < PF_MT) {
        const int m = threadIdx.x < (unsigned)nv ? (int)threadIdx.x : 0;
        const int32_t p = pairs[m];
        const int64_t row = by_token ? (int64_t)(p / n_sel) : (int64_t)p;
        pair[threadIdx.x] = p;
        roff[threadIdx.x] = (uint32_t)(row * ldq);
        srow[threadIdx.x] = scale[row];
    }
    __syncthreads();
}

#define PQ_DISPATCH(TYPE, GU, ...)                                                                   \
    do {                                                                                             \
        if (nv > 16) {                                                                               \
            switch (TYPE) {                                                                          \
            case ST_Q2_K: pq_proj<ST_Q2_K, GU, 2>(__VA_ARGS__); break;                               \
            case ST_Q3_K: pq_proj<ST_Q3_K, GU, 2>(__VA_ARGS__); break;                               \
            case ST_Q4_K: pq_proj<ST_Q4_K, GU, 2>(__VA_ARGS__); break;                               \
            default: break;                                                                          \
            }                                                                                        \
        } else {                                                                                     \
            switch (TYPE) {                                                                          \
            case ST_Q2_K: pq_proj<ST_Q2_K, GU, 1>(__VA_ARGS__); break;                               \
            case ST_Q3_K: pq_proj<ST_Q3_K, GU, 1>(__VA_ARGS__); break;                               \
            case ST_Q4_K: pq_proj<ST_Q4_K, GU, 1>(__VA_ARGS__); break;                               \
            default: break;                                                                          \
            }                                                                                        \
        }                                                                                            \
    } while (0)

// Gate/up: workgroup (rows 128 bx .. 128 bx + 127 of I, unit by); hf[p][row]
// = silu(gate . x_t) * (up . x_t) in f32 for the unit's pairs p (token t =
// p / n_sel). The host launches it only when every projection of the layer
// is Q2_K, Q3_K or Q4_K and I is a multiple of 128.
extern "C" __global__ __launch_bounds__(512) void sepia_pf_gateup_q(
    PfProj gate, PfProj up, PfProj s_gate, PfProj s_up, int32_t n_routed, int32_t n_sel, int64_t I, int64_t H,
    const uint8_t *__restrict__ pqx, const float *__restrict__ pqxs, const int32_t *__restrict__ list,
    const int32_t *__restrict__ units, const int32_t *__restrict__ n_units, float *__restrict__ hf) {
    if ((int32_t)blockIdx.y >= n_units[0]) return;
    extern __shared__ __attribute__((aligned(16))) uint8_t pf_smem[];
    uint8_t *smem = pf_smem;
    const int32_t *un = units + 3 * blockIdx.y;
    const int32_t e = un[0], nv = un[2];
    const bool routed = e < n_routed;
    const PfProj &G = routed ? gate : s_gate, &U = routed ? up : s_up;
    const int64_t ei = routed ? e : e - n_routed;
    const uint8_t *wg = G.base + ei * G.stride, *wu = U.base + ei * U.stride;
    const int64_t r0 = (int64_t)blockIdx.x * 128;
    uint32_t *roff;
    int32_t *pair;
    float *srow;
    pq_unit_rows(list + un[1], nv, true, n_sel, (H / 256) * PQ_REC, pqxs, smem, roff, pair, srow);
    PQ_DISPATCH(G.type, true, smem, wg, wu, G.row_bytes, G.n_blocks, pqx, roff, pair, srow, nv, r0, hf, I);
}

// Down: workgroup (rows 256 bx .. 256 bx + 255 of H, unit by); yp[p][row] =
// down_e . h_p in f32 (h_p the PQ row p). Same launch conditions, H a
// multiple of 256.
extern "C" __global__ __launch_bounds__(512) void sepia_pf_down_q(
    PfProj down, PfProj s_down, int32_t n_routed, int64_t I, int64_t H, const uint8_t *__restrict__ pqh,
    const float *__restrict__ pqhs, const int32_t *__restrict__ list, const int32_t *__restrict__ units,
    const int32_t *__restrict__ n_units, float *__restrict__ yp) {
    if ((int32_t)blockIdx.y >= n_units[0]) return;
    extern __shared__ __attribute__((aligned(16))) uint8_t pf_smem[];
    uint8_t *smem = pf_smem;
    const int32_t *un = units + 3 * blockIdx.y;
    const int32_t e = un[0], nv = un[2];
    const bool routed = e < n_routed;
    const PfProj &D = routed ? down : s_down;
    const int64_t ei = routed ? e : e - n_routed;
    const uint8_t *wd = D.base + ei * D.stride;
    const int64_t r0 = (int64_t)blockIdx.x * 256;
    uint32_t *roff;
    int32_t *pair;
    float *srow;
    pq_unit_rows(list + un[1], nv, false, 1, (I / 256) * PQ_REC, pqhs, smem, roff, pair, srow);
    PQ_DISPATCH(D.type, false, smem, wd, nullptr, D.row_bytes, D.n_blocks, pqh, roff, pair, srow, nv, r0, yp, H);
}
