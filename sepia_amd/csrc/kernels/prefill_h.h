// prefill_h.h -- the prefill MoE projections of the real checkpoint's
// formats (IQ2_XS, IQ3_XXS, IQ4_XS routed; Q5_K, Q6_K, Q8_0 shared) on the
// f16 matrix cores: the batched layer of prefill.h with the same grouping,
// units and combine, for layers whose six projections all have one of
// these formats.
//
// Activations (x per token for gate/up, h per pair for down) travel as "PH"
// rows: per row a power-of-two scale s > max|v| (s = 1 for a zero row,
// +inf when the row holds a NaN or an infinity, which then makes every
// output of the row non-finite), and per column v' = v / s (|v'| < 1,
// exact) as two f16 planes, hi = f16(v') and lo = f16(v' - hi): together
// within 2^-23 of v' (lo's rounding, or the f16 subnormal spacing 2^-24).
// A 256-column block of a row is a 1056-byte record: hi (256 f16, column
// order), lo (256 f16), then the eight 32-column sums of v' (f32, column
// order) that the Q5_K min terms use.
//
// Weights enter v_mfma_f32_16x16x32_f16 as exact f16 integer codes, decoded
// from the raw blocks in registers (the products hi * code and lo * code are
// exact in f32; the matrix cores add them in f32). Per weight row n and
// 256-column block, with C the f32 dot of the codes with v' (x is the
// v' the record holds, w the weights of src/quants.c's dequant):
//   IQ2_XS   code = +-grid * (2 s + 1) * 2^-14, s the 4-bit scale of its
//            16 weights (|code| <= 43 * 31 * 2^-14),
//            sum w x = d C 2^14 / 8                     (quants.c:179-201)
//   IQ3_XXS  code = +-grid * (2 s + 1) * 2^-14, 4-bit s per 32 weights
//            (|code| <= 62 * 31 * 2^-14), sum w x = d C 2^14 / 4
//            (quants.c:203-226)
//   Q5_K     code = q * sc, 6-bit sc per 32 (<= 31 * 63);
//            sum w x = d C - dmin sum_j m_j S_j, S_j the record's sums
//            (quants.c:127-151)
//   Q6_K     int8 sc per 16 weights split as 16 a + b (b in 0..15):
//            codes (q - 32) b and (q - 32) a, sum w x = d (C_b + 16 C_a)
//            (quants.c:153-177)
//   IQ4_XS   code = level (int8 table), per 32 columns
//            sum w x = sum_32 d (ls - 32) C_32          (quants.c:228-248)
//   Q8_0     code = q, per 32 columns sum w x = sum_32 d_32 C_32
//            (quants.c:85-94)
// Every code is an integer of magnitude < 2048 (the IQ codes times 2^-14),
// so exact in f16. The K-quant codes come from the byte b by a permute that
// makes the half 0x64bb (1024 + b, exact) and a packed f16 add or
// multiply-add that removes the 1024 and applies the scale. The IQ codes
// come from the grid byte b and a sign byte (0x80 or 0x00, a table per sign
// index) by one permute per two codes that makes the half +-b 2^-24 (the
// f16 subnormal with mantissa b), then one packed f16 multiply by
// (2 s + 1) 2^10: every intermediate exact. (The multiply reads the
// subnormal as such: f16 denormals are on in the kernels' default FP mode,
// and a flush would zero every IQ code, which every IQ parity case shows.)
//
// Workgroup: one unit (<= 32 pairs of one expert) x R weight rows (R = 256:
// gate/up 128 gate + the same 128 up rows; R = 128 for the formats whose
// staged blocks are too large for 256 rows: Q6_K, Q8_0), 16 waves; wave
// w < R / (16 NT) computes 16 NT rows (NT N tiles: 2 for the 256-row
// formats, so each activation read feeds two, else 1) x the unit's one or
// two 16-pair M tiles; the other waves only stage records. Records are double-buffered; weights SW-buffered, and
// a stepping wave stages exactly the weight rows it decodes (each row's block from
// the 4-byte boundary at or below its start, PW 16-byte pieces), so only
// the records need the per-block barrier.
#pragma once
#include "prefill_q.h"

#define PH_REC 1056                    // bytes of a 256-column PH record
#define PH_AP 66                       // its 16-byte pieces (2 mod 4: no LDS bank conflicts)
#define PH_ABYTES (PF_MT * PH_REC)     // a record stage: the unit's 32 rows
#define PH_WAVES 16                    // waves of a workgroup

typedef _Float16 ph_h2 __attribute__((ext_vector_type(2)));
typedef _Float16 ph_h8 __attribute__((ext_vector_type(8)));
typedef uint32_t ph_u4 __attribute__((ext_vector_type(4)));

// BB: block bytes (256 columns); PW: 16-byte pieces of a staged row (the
// block from the 4-byte boundary at or below its start, at most 2 bytes
// earlier); SW: weight stages; R: weight rows of a workgroup; NT: 16-row N
// tiles of a stepping wave; STEP: scale per 32-column step applied in f32
// (else once per block).
template <int T> struct PhFmt;
template <> struct PhFmt<ST_IQ2_XS> { static constexpr int BB = 74, PW = 6, SW = 3, R = 256, NT = 2; static constexpr bool STEP = false; };
template <> struct PhFmt<ST_IQ3_XXS> { static constexpr int BB = 98, PW = 10, SW = 2, R = 256, NT = 2; static constexpr bool STEP = false; };
template <> struct PhFmt<ST_IQ4_XS> { static constexpr int BB = 136, PW = 10, SW = 2, R = 256, NT = 2; static constexpr bool STEP = true; };
template <> struct PhFmt<ST_Q5_K> { static constexpr int BB = 176, PW = 11, SW = 2, R = 256, NT = 2; static constexpr bool STEP = false; };
template <> struct PhFmt<ST_Q6_K> { static constexpr int BB = 210, PW = 14, SW = 2, R = 128, NT = 1; static constexpr bool STEP = false; };
template <> struct PhFmt<ST_Q8_0> { static constexpr int BB = 272, PW = 17, SW = 2, R = 128, NT = 1; static constexpr bool STEP = true; };

// LDS: [record stages 2 x PH_ABYTES][weight stages SW x R x PW x 16]
//      [tables: IQ2_XS grid 4 KB / IQ3_XXS grid 1 KB, then 128 x 8 sign
//       bytes][... row tables at PQ_LDS_TOP]
template <int T> struct PhLds {
    static constexpr uint32_t W = (uint32_t)PhFmt<T>::R * PhFmt<T>::PW * 16;
    static constexpr uint32_t TAB = 2 * PH_ABYTES + PhFmt<T>::SW * W;
    static constexpr uint32_t GRID = T == ST_IQ2_XS ? 4096u : T == ST_IQ3_XXS ? 1024u : 0u;
    static constexpr uint32_t SIGNS = TAB + GRID;
    static constexpr uint32_t END = SIGNS + (GRID ? 1024u : 0u);
    static_assert(END <= PQ_LDS_TOP, "LDS of a PH projection");
};

// --------------------------------------------------------- rows -> PH ----
// One workgroup per row: src row r (K floats at src + r * ld) into its
// records at rec + r * ldr and its scale at scale[r]. Thread i converts the
// 32-column groups i, i + 256, ...
extern "C" __global__ __launch_bounds__(256) void sepia_ph_quant(const float *__restrict__ src, int64_t ld,
                                                                 int64_t K, uint8_t *__restrict__ rec, int64_t ldr,
                                                                 float *__restrict__ scale) {
    __shared__ float red[4];
    const int64_t r = blockIdx.x;
    const float *row = src + r * ld;
    float m = 0.0f;
    for (int64_t c = 4 * (int64_t)threadIdx.x; c < K; c += 1024) {
        const float4 v = *(const float4 *)(row + c);
        m = mq_nonfinite_max(fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)))),
                             (v.x + v.y) + (v.z + v.w));
    }
    m = pq_wave_max(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    // s = 2^e > m (exact scaling): e = the exponent of m's leading bit + 1
    const bool fin = m <= 3.0e38f;
    int e = 0;
    if (fin && m > 0.0f) (void)frexpf(m, &e);
    e = e < 127 ? e : 127;   // 2^127 <= m < 2^128: |v'| < 2, still exact in f16 hi + lo
    const float s = !fin ? INFINITY : ldexpf(1.0f, e), inv = fin ? ldexpf(1.0f, -e) : 0.0f;
    if (threadIdx.x == 0) scale[r] = s;
    uint8_t *out = rec + r * ldr;
    for (int64_t gi = threadIdx.x; gi < K / 32; gi += 256) {
        const float4 *x4 = (const float4 *)(row + 32 * gi);
        uint8_t *blk = out + (gi >> 3) * PH_REC;
        const int j = (int)(gi & 7);
        float sum = 0.0f;
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const float4 t = x4[c];
            const float a[4] = {t.x * inv, t.y * inv, t.z * inv, t.w * inv};
            _Float16 h[4], l[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                sum += a[i];
                h[i] = (_Float16)a[i];
                l[i] = (_Float16)(a[i] - (float)h[i]);
            }
            *(uint2 *)(blk + 64 * j + 8 * c) = *(const uint2 *)h;
            *(uint2 *)(blk + 512 + 64 * j + 8 * c) = *(const uint2 *)l;
        }
        *(float *)(blk + 1024 + 4 * j) = fin ? sum : 0.0f;
    }
}

// ------------------------------------------------------------- staging --
// Record pieces: the unit's records of a block (its nv <= 32 pairs, 66
// pieces each, record m at 1056 m) by up to 33 wave instructions over the 16
// waves. Weight pieces:
// stepping wave w (w < R / RW, RW = 16 NT) stages its RW rows, piece c of
// row k at 16 (PW (RW w + k) + c); a piece that starts past the block's bytes (plus
// the 2 of the 4-byte alignment) takes piece 0's bytes again. The last
// piece that holds block bytes may run up to 14 bytes past the block: into
// the row's next block, the next row, or, after a matrix's last row, the
// 256 bytes every device buffer of the library carries past its data
// (dev_bytes in sepia_hip.c).
template <int T, bool GU>
struct PhDma {
    static constexpr int BB = PhFmt<T>::BB, PW = PhFmt<T>::PW, R = PhFmt<T>::R, RW = 16 * PhFmt<T>::NT, AW = R / RW;
    static constexpr int NA = (PF_MT * PH_AP + 63) / 64, KA = (NA + PH_WAVES - 1) / PH_WAVES;
    static constexpr int NW = RW * PW, KW = (NW + 63) / 64;   // a stepping wave's weight pieces and instructions
    uint32_t a[KA];            // record piece offsets at block 0
    uint32_t r[KW], c16[KW];   // row offset from the matrix base; offset of the lane's piece in the window
    bool aon[KA], won[KW];
    // nr: the records the unit's M tiles read (its pairs; the rest of the
    // stage is not staged, and the M tile rows past the pairs are discarded)
    __device__ __forceinline__ void init(const uint32_t *roff, uint64_t row_bytes, int64_t r0, int nr) {
        const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
        for (int k = 0; k < KA; k++) {
            const int q = 64 * (w + PH_WAVES * k) + lane, m = q / PH_AP, c = q - m * PH_AP;
            aon[k] = w + PH_WAVES * k < NA && q < PF_MT * PH_AP && m < nr;
            a[k] = aon[k] ? roff[m] + 16u * (uint32_t)c : 0u;
        }
        // stepping waves 0 .. AW - 1 take RW rows each; GU: the first half
        // the gate rows, the second half the same up rows
        const bool on = w < AW;
        const int64_t rw0 = r0 + (int64_t)(RW * (GU ? w % (AW / 2) : w));
#pragma unroll
        for (int k = 0; k < KW; k++) {
            const int q = 64 * k + lane, kr = q / PW, c = q - kr * PW;
            won[k] = on && q < NW;
            r[k] = won[k] ? (uint32_t)((uint64_t)(rw0 + kr) * row_bytes) : 0u;
            c16[k] = 16 * c < BB + 2 ? 16u * (uint32_t)c : 0u;
        }
    }
    __device__ __forceinline__ void issue_a(int64_t b, uint8_t *As, const uint8_t *rec) const {
        const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
        const uint32_t ab = (uint32_t)b * PH_REC;
#pragma unroll
        for (int k = 0; k < KA; k++) {
            const int jj = w + PH_WAVES * k;
            if (jj < NA && aon[k]) pf_dma16(rec, a[k] + ab, pf_lds(As + 1024 * jj));
        }
    }
    // a stepping wave's weight instructions of one block (other waves: none)
    __device__ __forceinline__ void issue_w(int64_t b, uint8_t *Ws, const uint8_t *Wm) const {
        const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
        if (w >= AW) return;
        const uint32_t wb = (uint32_t)b * BB;
        uint8_t *dst = Ws + 16 * NW * w;
#pragma unroll
        for (int k = 0; k < KW; k++)
            if (won[k]) pf_dma16(Wm, ((r[k] + wb) & ~3u) + c16[k], pf_lds(dst + 1024 * k));
    }
};

// ------------------------------------------------------------- decoders --
typedef const __attribute__((address_space(3))) uint32_t ph_lds_u32;
typedef const __attribute__((address_space(3))) uint16_t ph_lds_u16;
typedef const __attribute__((address_space(3))) uint8_t ph_lds_u8;
__device__ __forceinline__ uint32_t ph_u8(const uint8_t *p) { return *(ph_lds_u8 *)(size_t)pf_lds(p); }
__device__ __forceinline__ uint32_t ph_u16(const uint8_t *p) { return *(ph_lds_u16 *)(size_t)pf_lds(p); }
__device__ __forceinline__ float ph_h2f(const uint8_t *p) { return f16_bits_to_f32(ph_u16(p)); }
// 4 bytes at a 2-byte-aligned LDS address: the two aligned dwords around
// it, funnel-shifted
__device__ __forceinline__ uint32_t ph_u32(const uint8_t *p) {
    const uint32_t a = pf_lds(p), a4 = a & ~3u;
    const uint32_t lo = *(ph_lds_u32 *)(size_t)a4, hi = *(ph_lds_u32 *)(size_t)(a4 + 4u);
    return __builtin_amdgcn_alignbit(hi, lo, 8u * (a & 3u));
}
// 8 bytes at a 2-byte-aligned LDS address
__device__ __forceinline__ uint2 ph_u64(const uint8_t *p) {
    const uint32_t a = pf_lds(p), a4 = a & ~3u, sh = 8u * (a & 3u);
    const uint32_t d0 = *(ph_lds_u32 *)(size_t)a4, d1 = *(ph_lds_u32 *)(size_t)(a4 + 4u),
                   d2 = *(ph_lds_u32 *)(size_t)(a4 + 8u);
    return make_uint2(__builtin_amdgcn_alignbit(d1, d0, sh), __builtin_amdgcn_alignbit(d2, d1, sh));
}

// Bytes 0, 1 (sel 0x04010400) or 2, 3 (sel 0x04030402) of v as the halves
// 0x64bb: 1024 + b, exact.
__device__ __forceinline__ ph_h2 ph_bias2(uint32_t v, uint32_t sel) {
    return __builtin_bit_cast(ph_h2, __builtin_amdgcn_perm(0x64646464u, v, sel));
}
#define PH_SEL_LO 0x04010400u
#define PH_SEL_HI 0x04030402u
// 8 codes b - off from the 8 bytes of g (exact f16 integers)
__device__ __forceinline__ ph_h8 ph_codes_sub(uint2 g, ph_h2 off) {
    ph_h2 c[4] = {ph_bias2(g.x, PH_SEL_LO) - off, ph_bias2(g.x, PH_SEL_HI) - off, ph_bias2(g.y, PH_SEL_LO) - off,
                  ph_bias2(g.y, PH_SEL_HI) - off};
    return __builtin_bit_cast(ph_h8, c);
}
__device__ __forceinline__ ph_h2 ph_splat(float v) {
    const _Float16 h = (_Float16)v;
    return ph_h2{h, h};
}
// A small integer's exact f16 in both halves (a direct 16-bit integer to f16
// convert, no f32 step): |v| <= 2048.
__device__ __forceinline__ ph_h2 ph_splat_u(uint32_t v) {
    const _Float16 h = (_Float16)(uint16_t)v;
    return ph_h2{h, h};
}
// The sign bytes of the 128 IQ sign indices, 8 bytes each: byte j 0x80
// where bit j of iq_signs(index) is set (code j negative), else 0x00.
__device__ __forceinline__ void ph_fill_signs(uint8_t *st) {
    for (int i = threadIdx.x; i < 128; i += blockDim.x) {
        const uint32_t s = iq_signs((uint32_t)i);
        uint2 m = make_uint2(0u, 0u);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            m.x |= ((s >> j) & 1u) << (8 * j + 7);
            m.y |= ((s >> (j + 4)) & 1u) << (8 * j + 7);
        }
        *(uint2 *)(st + 8 * i) = m;
    }
}
// 8 IQ codes from the grid bytes g and the sign bytes sg (codes 0..3 in .x,
// 4..7 in .y): the halves +-b 2^-24 (low byte the grid byte, high byte the
// sign byte) times s2 = (2 s + 1) 2^10
__device__ __forceinline__ ph_h8 ph_codes_iq(uint2 g, uint2 sg, ph_h2 s2) {
    const ph_h2 c[4] = {__builtin_bit_cast(ph_h2, __builtin_amdgcn_perm(sg.x, g.x, 0x05010400u)) * s2,
                        __builtin_bit_cast(ph_h2, __builtin_amdgcn_perm(sg.x, g.x, 0x07030602u)) * s2,
                        __builtin_bit_cast(ph_h2, __builtin_amdgcn_perm(sg.y, g.y, 0x05010400u)) * s2,
                        __builtin_bit_cast(ph_h2, __builtin_amdgcn_perm(sg.y, g.y, 0x07030602u)) * s2};
    return __builtin_bit_cast(ph_h8, c);
}
template <int T>
__device__ __forceinline__ void ph_fill_tables(uint8_t *smem) {
    if constexpr (T == ST_IQ2_XS) {
        for (int i = threadIdx.x; i < 512; i += blockDim.x) ((uint64_t *)(smem + PhLds<T>::TAB))[i] = c_iq2xs_grid[i];
        ph_fill_signs(smem + PhLds<T>::SIGNS);
    } else if constexpr (T == ST_IQ3_XXS) {
        for (int i = threadIdx.x; i < 256; i += blockDim.x) ((uint32_t *)(smem + PhLds<T>::TAB))[i] = c_iq3xxs_grid[i];
        ph_fill_signs(smem + PhLds<T>::SIGNS);
    }
}

// The IQ4 levels + 128 as bytes (0..241), for the biased conversion.
__device__ __forceinline__ constexpr uint32_t ph_iq4_word(int k) {
    constexpr int8_t v[16] = SEPIA_IQ4NL_VALUES_INIT;
    return (uint32_t)(uint8_t)(v[4 * k] + 128) | ((uint32_t)(uint8_t)(v[4 * k + 1] + 128) << 8) |
           ((uint32_t)(uint8_t)(v[4 * k + 2] + 128) << 16) | ((uint32_t)(uint8_t)(v[4 * k + 3] + 128) << 24);
}
// levels + 128 of the four codes in the low nibbles of the bytes of c
__device__ __forceinline__ uint32_t ph_iq4_levels(uint32_t c) {
    constexpr uint32_t T0 = ph_iq4_word(0), T1 = ph_iq4_word(1), T2 = ph_iq4_word(2), T3 = ph_iq4_word(3);
    const uint32_t sel = c & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(T1, T0, sel), hi = __builtin_amdgcn_perm(T3, T2, sel);
    return __builtin_amdgcn_perm(hi, lo, ((c >> 1) & 0x04040404u) | 0x03020100u);
}

// Q5_K's 6-bit scale and min of sub-block j from the 12 scale bytes at p
// (the packing of get_scale_min_k4, src/quants.c:96-102).
__device__ __forceinline__ uint32_t k_scale_6(const uint8_t *p, int j) {
    return j < 4 ? ph_u8(p + j) & 63u : (ph_u8(p + j + 4) & 15u) | ((ph_u8(p + j - 4) >> 6) << 4);
}
__device__ __forceinline__ uint32_t k_min_6(const uint8_t *p, int j) {
    return j < 4 ? ph_u8(p + j + 4) & 63u : (ph_u8(p + j + 4) >> 4) | ((ph_u8(p + j) >> 6) << 4);
}

// What a lane decodes for K step s (columns 32 s .. 32 s + 31 of the block;
// lane group g takes columns 32 s + 8 g .. + 7) of its row's block: the 8
// codes (two operands for Q6_K) and, for the STEP formats, the step's scale.
struct PhB {
    ph_h8 b, b2;
    float sc;
};
template <int T>
__device__ __forceinline__ PhB ph_decode(const uint8_t *blk, const uint8_t *tab, const uint8_t *signs, int s, int g) {
    PhB r;
    if constexpr (T == ST_IQ2_XS) {
        // qs u16 [4 s + g] at 2: grid index (9 bits), sign index (7 bits);
        // 4-bit scale: nibble g >> 1 of byte 66 + s
        const uint32_t v = ph_u16(blk + 2 + 2 * (4 * s + g));
        const uint32_t sc = 2u * ((ph_u8(blk + 66 + s) >> (4 * (g >> 1))) & 15u) + 1u;
        const uint2 gr = *(const __attribute__((address_space(3))) uint2 *)(size_t)pf_lds(tab + 8 * (v & 511u));
        const uint2 sg = *(const __attribute__((address_space(3))) uint2 *)(size_t)pf_lds(signs + 8 * (v >> 9));
        r.b = ph_codes_iq(gr, sg, ph_splat_u(sc << 10));
    } else if constexpr (T == ST_IQ3_XXS) {
        // qs bytes 8 s + 2 g, + 1 at 2 (grid indices, 4 bytes each); aux32 of
        // step s at 66 + 4 s: sign index g at bit 7 g, 4-bit scale at 28
        const uint32_t aux = ph_u32(blk + 66 + 4 * s);
        const uint32_t ix = ph_u16(blk + 2 + 8 * s + 2 * g);
        const uint32_t sc = 2u * (aux >> 28) + 1u;
        uint2 gr;
        gr.x = *(const __attribute__((address_space(3))) uint32_t *)(size_t)pf_lds(tab + 4 * (ix & 255u));
        gr.y = *(const __attribute__((address_space(3))) uint32_t *)(size_t)pf_lds(tab + 4 * (ix >> 8));
        const uint2 sg =
            *(const __attribute__((address_space(3))) uint2 *)(size_t)pf_lds(signs + 8 * ((aux >> (7 * g)) & 127u));
        r.b = ph_codes_iq(gr, sg, ph_splat_u(sc << 10));
    } else if constexpr (T == ST_IQ4_XS) {
        // qs[16 s + 8 (g & 1) + i] at 8, nibble g >> 1; 6-bit scale ls
        const uint2 q = ph_u64(blk + 8 + 16 * s + 8 * (g & 1));
        const uint32_t sh = 4u * (uint32_t)(g >> 1);
        const uint2 lv = make_uint2(ph_iq4_levels(q.x >> sh), ph_iq4_levels(q.y >> sh));
        r.b = ph_codes_sub(lv, ph_splat(1152.0f));
        const uint32_t ls = ((ph_u8(blk + 4 + (s >> 1)) >> (4 * (s & 1))) & 15u) |
                            (((ph_u16(blk + 2) >> (2 * s)) & 3u) << 4);
        r.sc = ph_h2f(blk) * (float)((int32_t)ls - 32);
    } else if constexpr (T == ST_Q5_K) {
        // step s: 64-weight chunk j = s >> 1, nibble s & 1 of qs[32 j + l]
        // (at 48) and bit s of qh[l] (at 16), l = 8 g .. 8 g + 7; 6-bit
        // scale of sub-block s
        const uint2 q = ph_u64(blk + 48 + 32 * (s >> 1) + 8 * g), h = ph_u64(blk + 16 + 8 * g);
        const uint32_t nsh = 4u * (uint32_t)(s & 1);
        const uint32_t c0 = ((q.x >> nsh) & 0x0F0F0F0Fu) | (((h.x >> s) & 0x01010101u) << 4);
        const uint32_t c1 = ((q.y >> nsh) & 0x0F0F0F0Fu) | (((h.y >> s) & 0x01010101u) << 4);
        const uint32_t sc = k_scale_6(blk + 4, s);
        r.b = ph_codes_sub(make_uint2(c0, c1), ph_splat(1024.0f)) * (_Float16)(uint16_t)sc;
    } else if constexpr (T == ST_Q6_K) {
        // 128-half n6 = s >> 2, quarter qq = s & 3: low 4 bits from
        // ql[64 n6 + 32 (qq & 1) + l] (nibble qq >> 1), high 2 bits from
        // qh[32 n6 + l] bits 2 qq (at 128), l = 8 g .. 8 g + 7; int8 scale
        // sc[8 n6 + 2 qq + (g >> 1)] (at 192) split as 16 a + b
        const int n6 = s >> 2, qq = s & 3;
        const uint2 q = ph_u64(blk + 64 * n6 + 32 * (qq & 1) + 8 * g), h = ph_u64(blk + 128 + 32 * n6 + 8 * g);
        const uint32_t nsh = 4u * (uint32_t)(qq >> 1), hsh = 2u * (uint32_t)qq;
        const uint32_t c0 = ((q.x >> nsh) & 0x0F0F0F0Fu) | (((h.x >> hsh) & 0x03030303u) << 4);
        const uint32_t c1 = ((q.y >> nsh) & 0x0F0F0F0Fu) | (((h.y >> hsh) & 0x03030303u) << 4);
        const int32_t sc = (int32_t)(int8_t)ph_u8(blk + 192 + 8 * n6 + 2 * qq + (g >> 1));
        const ph_h8 q32 = ph_codes_sub(make_uint2(c0, c1), ph_splat(1056.0f));   // q - 32
        r.b = q32 * (_Float16)(int16_t)(sc & 15);                               // (q - 32) b
        r.b2 = q32 * (_Float16)(int16_t)(sc >> 4);                              // (q - 32) a
    } else {   // Q8_0: block s (34 bytes at 34 s): d, then int8 qs
        const uint2 q = ph_u64(blk + 34 * s + 2 + 8 * g);
        r.b = ph_codes_sub(make_uint2(q.x ^ 0x80808080u, q.y ^ 0x80808080u), ph_splat(1152.0f));
        r.sc = ph_h2f(blk + 34 * s);
    }
    return r;
}

// ----------------------------------------------------------- projection --
// One projection workgroup (see the top of the file). GU: rows r0 .. r0 +
// R / 2 - 1 of gate (W0) and up (W1), h[pair][row] = silu(gate) * up in
// f32; down: rows r0 .. r0 + R - 1 of W0, out[pair][row] in f32. Stepping
// wave w (w < R / RW, RW = 16 NT) computes RW rows (NT N tiles) x the
// unit's one or two 16-pair M tiles (GU: waves w and w + R / (2 RW) the
// same rows of gate and up); the other waves stage records only.
template <int T, bool GU, int MT>
__device__ __forceinline__ void ph_proj(uint8_t *smem, const uint8_t *W0, const uint8_t *W1, uint64_t row_bytes,
                                        int64_t nb, const uint8_t *rec, const uint32_t *roff, const int32_t *pair,
                                        const float *srow, int nv, int64_t r0, float *__restrict__ out,
                                        int64_t ld_out) {
    constexpr int BB = PhFmt<T>::BB, PW = PhFmt<T>::PW, SW = PhFmt<T>::SW, R = PhFmt<T>::R;
    constexpr int NT = PhFmt<T>::NT, RW = 16 * NT, AW = R / RW, HALF = AW / 2;
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)), l = threadIdx.x & 63, n = l & 15,
              g = l >> 4;
    const bool on = w < AW;
    const uint8_t *Wm = (GU && w >= HALF) ? W1 : W0;
    const int64_t grow = r0 + RW * (GU ? w % HALF : w);   // the wave's first global row
    auto a_stage = [&](int b) { return smem + (uint32_t)(b & 1) * PH_ABYTES; };
    auto w_stage = [&](int b) { return smem + 2 * PH_ABYTES + (uint32_t)b % SW * PhLds<T>::W; };
    const uint8_t *tab = smem + PhLds<T>::TAB, *signs = smem + PhLds<T>::SIGNS;
    ph_fill_tables<T>(smem);   // published by the first block's barrier
    PhDma<T, GU> dma;
    dma.init(roff, row_bytes, r0, nv);
    pf_f32x4 acc[NT][2];
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int mt = 0; mt < 2; mt++) acc[t][mt] = pf_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const int nbi = (int)nb;
    dma.issue_a(0, a_stage(0), rec);
    for (int c = 0; c < SW - 1 && c < nbi; c++) dma.issue_w(c, w_stage(c), Wm);
    constexpr int APB = 16 * PH_AP;   // bytes of a staged record
    constexpr int KW = PhDma<T, GU>::KW;
    for (int b = 0; b < nbi; b++) {
        // everything up to A_b and W_b; the weights of blocks b + 1 .. b + SW - 2 may fly
        const int ahead = (nbi - 1 - b) < (SW - 2) ? (nbi - 1 - b) : (SW - 2);
        pq_wait_vm<KW * (SW - 2)>((on ? KW : 0) * ahead);
        // the blocks at offset o of their staged rows (rows of 4-byte multiples)
        const uint8_t *blk[NT];
#pragma unroll
        for (int t = 0; t < NT; t++)
            blk[t] = w_stage(b) + (uint32_t)(RW * w + 16 * t + n) * (PW * 16) + (((uint32_t)b * BB) & 3u);
        asm volatile("" ::: "memory");
        __syncthreads();   // every wave's record pieces of A_b, the tables
        asm volatile("" ::: "memory");
        if (b + 1 < nbi) dma.issue_a(b + 1, a_stage(b + 1), rec);
        if (b + SW - 1 < nbi) dma.issue_w(b + SW - 1, w_stage(b + SW - 1), Wm);
        if (!on) continue;
        const uint8_t *As = a_stage(b);
        pf_f32x4 cb[NT][2], cb2[NT][2];
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int mt = 0; mt < 2; mt++) {
                cb[t][mt] = pf_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                cb2[t][mt] = pf_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            }
        // Software-pipelined by one K step: step s + 1's codes (LDS
        // gathers and their VALU) and activation planes are read before
        // step s's matrix ops are issued (the scheduling barrier keeps that
        // order), so the gathers' latency runs under the MFMAs.
        PhB B[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) B[t] = ph_decode<T>(blk[t], tab, signs, 0, g);
        ph_h8 ah[MT], al[MT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const uint8_t *ap = As + (16 * mt + n) * APB + 16 * g;
            ah[mt] = *(const __attribute__((address_space(3))) ph_h8 *)(size_t)pf_lds(ap);
            al[mt] = *(const __attribute__((address_space(3))) ph_h8 *)(size_t)pf_lds(ap + 512);
        }
#pragma unroll
        for (int s = 0; s < 8; s++) {
            PhB Bn[NT];
            ph_h8 ahn[MT], aln[MT];
            if (s + 1 < 8) {
#pragma unroll
                for (int t = 0; t < NT; t++) Bn[t] = ph_decode<T>(blk[t], tab, signs, s + 1, g);
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
                    const uint8_t *ap = As + (16 * mt + n) * APB + 64 * (s + 1) + 16 * g;
                    ahn[mt] = *(const __attribute__((address_space(3))) ph_h8 *)(size_t)pf_lds(ap);
                    aln[mt] = *(const __attribute__((address_space(3))) ph_h8 *)(size_t)pf_lds(ap + 512);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    if constexpr (PhFmt<T>::STEP) {
                        pf_f32x4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[mt], B[t].b, pf_f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[mt], B[t].b, c, 0, 0, 0);
#pragma unroll
                        for (int i = 0; i < 4; i++) acc[t][mt][i] = __builtin_fmaf(B[t].sc, c[i], acc[t][mt][i]);
                    } else {
                        cb[t][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[mt], B[t].b, cb[t][mt], 0, 0, 0);
                        cb[t][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[mt], B[t].b, cb[t][mt], 0, 0, 0);
                        if constexpr (T == ST_Q6_K) {
                            cb2[t][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[mt], B[t].b2, cb2[t][mt], 0, 0, 0);
                            cb2[t][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[mt], B[t].b2, cb2[t][mt], 0, 0, 0);
                        }
                    }
                }
            }
            if (s + 1 < 8) {
#pragma unroll
                for (int t = 0; t < NT; t++) B[t] = Bn[t];
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
                    ah[mt] = ahn[mt];
                    al[mt] = aln[mt];
                }
            }
        }
#pragma unroll
        for (int t = 0; t < NT; t++) {
            if constexpr (T == ST_IQ2_XS || T == ST_IQ3_XXS) {
                const float d = ph_h2f(blk[t]) * (T == ST_IQ2_XS ? 2048.0f : 4096.0f);   // 2^14 / 8, 2^14 / 4
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[t][mt][i] = __builtin_fmaf(d, cb[t][mt][i], acc[t][mt][i]);
            } else if constexpr (T == ST_Q6_K) {
                const float d = ph_h2f(blk[t] + 208);
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        acc[t][mt][i] =
                            __builtin_fmaf(d, __builtin_fmaf(16.0f, cb2[t][mt][i], cb[t][mt][i]), acc[t][mt][i]);
            } else if constexpr (T == ST_Q5_K) {   // d C - dmin sum_j m_j S_j, the min terms on the f32 matrix cores
                const float d = ph_h2f(blk[t]), dmin = ph_h2f(blk[t] + 2);
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
                    pf_f32x4 cm = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int h = 0; h < 2; h++) {
                        // A[pair][k] = S_(4 h + k) of pair 16 mt + n; B[k][row n] = m_(4 h + k)
                        const float sa = *(const __attribute__((address_space(3))) float *)(size_t)pf_lds(
                            As + (16 * mt + n) * APB + 1024 + 4 * (4 * h + g));
                        const float mb = (float)k_min_6(blk[t] + 4, 4 * h + g);
                        cm = __builtin_amdgcn_mfma_f32_16x16x4f32(sa, mb, cm, 0, 0, 0);
                    }
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        acc[t][mt][i] = __builtin_fmaf(-dmin, cm[i], __builtin_fmaf(d, cb[t][mt][i], acc[t][mt][i]));
                }
            }
        }
    }
    // y = s_pair * acc; lane: pairs 16 mt + 4 g + i, rows grow + 16 t + n
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float sp = srow[16 * mt + 4 * g + i];
#pragma unroll
            for (int t = 0; t < NT; t++) acc[t][mt][i] *= sp;
        }
    if constexpr (GU) {
        __syncthreads();   // every wave is done with the stages
        float *xch = (float *)smem + ((w % HALF) * 64 + l) * (8 * NT);
        if (on && w >= HALF) {
#pragma unroll
            for (int t = 0; t < NT; t++)
#pragma unroll
                for (int mt = 0; mt < 2; mt++) *(pf_f32x4 *)(xch + 8 * t + 4 * mt) = acc[t][mt];
        }
        __syncthreads();
        if (!on || w >= HALF) return;
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const pf_f32x4 u = *(const pf_f32x4 *)(xch + 8 * t + 4 * mt);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int m = 16 * mt + 4 * g + i;
                    if (m < nv) out[(int64_t)pair[m] * ld_out + grow + 16 * t + n] = silu_f32(acc[t][mt][i]) * u[i];
                }
            }
    } else {
        if (!on) return;
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int m = 16 * mt + 4 * g + i;
                    if (m < nv) out[(int64_t)pair[m] * ld_out + grow + 16 * t + n] = acc[t][mt][i];
                }
    }
}

// The launch has one workgroup per row slice (gate/up: 64 rows of each
// matrix; down: 128 rows); a format with R = 256 rows covers two slices (see
// ph_slice).
#define PH_DISPATCH(TYPE, GU, R0, ...)                                                               \
    do {                                                                                             \
        switch (TYPE) {                                                                              \
        case ST_IQ2_XS: PH_CALL(ST_IQ2_XS, GU, R0, __VA_ARGS__); break;                              \
        case ST_IQ3_XXS: PH_CALL(ST_IQ3_XXS, GU, R0, __VA_ARGS__); break;                            \
        case ST_IQ4_XS: PH_CALL(ST_IQ4_XS, GU, R0, __VA_ARGS__); break;                              \
        case ST_Q5_K: PH_CALL(ST_Q5_K, GU, R0, __VA_ARGS__); break;                                  \
        case ST_Q6_K: PH_CALL(ST_Q6_K, GU, R0, __VA_ARGS__); break;                                  \
        case ST_Q8_0: PH_CALL(ST_Q8_0, GU, R0, __VA_ARGS__); break;                                  \
        default: break;                                                                              \
        }                                                                                            \
    } while (0)
#define PH_CALL(T, GU, R0, smem, W0, W1, row_bytes, nb, rec, roff, pair, srow, nv, out, ld_out)      \
    do {                                                                                             \
        if (nv > 16) ph_proj<T, GU, 2>(smem, W0, W1, row_bytes, nb, rec, roff, pair, srow, nv, R0, out, ld_out); \
        else ph_proj<T, GU, 1>(smem, W0, W1, row_bytes, nb, rec, roff, pair, srow, nv, R0, out, ld_out);        \
    } while (0)
// Formats staged 128 rows at a time (the others 256).
__device__ __forceinline__ bool ph_rows128(int32_t t) { return t == ST_Q6_K || t == ST_Q8_0; }
// The first row slice of slot x, or -1 for none: formats staged 256
// rows at a time take slices 2 x, 2 x + 1 in the slots x < gridDim.x / 2.
// Keeping the active slots at consecutive x spreads them over all 8 XCDs
// (the hardware deals consecutive workgroup ids to the XCDs in turn: with
// rows of 48 workgroups, active even x alone would land on 4 of them).
__device__ __forceinline__ int64_t ph_slice(int32_t t, int32_t x) {
    if (ph_rows128(t)) return x;
    return x < (int32_t)gridDim.x / 2 ? 2 * (int64_t)x : -1;
}
// 256-column blocks of a row (a projection's n_blocks counts Q8_0's
// 32-column blocks; its 256-column block is eight of them, 272 bytes).
__device__ __forceinline__ int64_t ph_nb(int32_t t, int64_t n_blocks) { return t == ST_Q8_0 ? n_blocks / 8 : n_blocks; }

// Gate/up: workgroup (64-row slice bx of I, unit by); hf[p][row] = silu(gate
// . x_t) * (up . x_t) in f32 for the unit's pairs p (token t = p / n_sel).
// The host launches it only when every projection of the layer has one of
// the formats above, with 4-byte-aligned rows, and H and I are multiples of
// 256.
extern "C" __global__ __launch_bounds__(64 * PH_WAVES) void sepia_ph_gateup(
    PfProj gate, PfProj up, PfProj s_gate, PfProj s_up, int32_t n_routed, int32_t n_sel, int64_t I, int64_t H,
    const uint8_t *__restrict__ phx, const float *__restrict__ phxs, const int32_t *__restrict__ list,
    const int32_t *__restrict__ units, const int32_t *__restrict__ n_units, float *__restrict__ hf) {
    const PfSlot slot = pf_slot();
    if (slot.y >= n_units[0]) return;
    extern __shared__ __attribute__((aligned(16))) uint8_t pf_smem[];
    uint8_t *smem = pf_smem;
    const int32_t *un = units + 3 * slot.y;
    const int32_t e = un[0], nv = un[2];
    const bool routed = e < n_routed;
    const PfProj &G = routed ? gate : s_gate, &U = routed ? up : s_up;
    const int64_t ei = routed ? e : e - n_routed;
    const uint8_t *wg = G.base + ei * G.stride, *wu = U.base + ei * U.stride;
    const int64_t sl = ph_slice(G.type, slot.x);
    if (sl < 0) return;
    uint32_t *roff;
    int32_t *pair;
    float *srow;
    pq_unit_rows(list + un[1], nv, true, n_sel, (H / 256) * PH_REC, phxs, smem, roff, pair, srow);
    PH_DISPATCH(G.type, true, sl * 64, smem, wg, wu, G.row_bytes, ph_nb(G.type, G.n_blocks), phx, roff,
                pair, srow, nv, hf, I);
}

// Down: workgroup (128-row slice bx of H, unit by); yp[p][row] = down_e .
// h_p in f32 (h_p the PH row p). Same launch conditions.
extern "C" __global__ __launch_bounds__(64 * PH_WAVES) void sepia_ph_down(
    PfProj down, PfProj s_down, int32_t n_routed, int64_t I, int64_t H, const uint8_t *__restrict__ phh,
    const float *__restrict__ phhs, const int32_t *__restrict__ list, const int32_t *__restrict__ units,
    const int32_t *__restrict__ n_units, float *__restrict__ yp) {
    const PfSlot slot = pf_slot();
    if (slot.y >= n_units[0]) return;
    extern __shared__ __attribute__((aligned(16))) uint8_t pf_smem[];
    uint8_t *smem = pf_smem;
    const int32_t *un = units + 3 * slot.y;
    const int32_t e = un[0], nv = un[2];
    const bool routed = e < n_routed;
    const PfProj &D = routed ? down : s_down;
    const int64_t ei = routed ? e : e - n_routed;
    const uint8_t *wd = D.base + ei * D.stride;
    const int64_t sl = ph_slice(D.type, slot.x);
    if (sl < 0) return;
    uint32_t *roff;
    int32_t *pair;
    float *srow;
    pq_unit_rows(list + un[1], nv, false, 1, (I / 256) * PH_REC, phhs, smem, roff, pair, srow);
    PH_DISPATCH(D.type, false, sl * 128, smem, wd, wd, D.row_bytes, ph_nb(D.type, D.n_blocks), phh,
                roff, pair, srow, nv, yp, H);
}
