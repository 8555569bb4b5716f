/* oracle/sepia_oracle.c -- CPU restatement of the reference's quantized-weight
 * path. TEST INFRASTRUCTURE ONLY (see sepia_oracle.h): the product never links
 * it; tests, smoke() and bench.py's CPU baseline use it as the checker.
 *
 * Build with -ffp-contract=off: the dequantizers must round every product and
 * difference separately, exactly like the reference (src/quants.c:1-6).
 *
 * What pins each function (tests/test_oracle.py):
 *   f16_to_f32, dequant F16/Q8_0/Q4_K/Q5_K/Q6_K/IQ2_XS/IQ3_XXS/IQ4_XS:
 *       the reference's 8 SQFX golden fixtures (bitwise) and a differential
 *       run against the reference's own src/quants.c compiled into oracle/_ref
 *       on fresh random blocks (bitwise), plus exhaustive f16.
 *   dequant Q2_K/Q3_K: not in the reference (no decoder to match): pinned by an
 *       independent vectorised numpy restatement of the public ggml layout and
 *       by single-field probe blocks (closed-form values). Parity against the
 *       reference itself is unpinned.
 *   dequant IQ2_XXS: the codebook is absent offline, so the type is
 *       unsupported unless a table is installed; with a stand-in table the
 *       decode structure is pinned against the numpy restatement only.
 *   qlinear: the reference's SQLX fixture (bitwise) and a numpy sequential
 *       float64 accumulation (np.cumsum) over reference-decoded rows.
 *   sigmoid/silu/logsigmoid: closed forms in float64 (tolerance).
 *   route_select: the transformers InklingTopkRouter golden vectors
 *       (tests/golden), and invariants (weights sum to route_scale*global_scale,
 *       bias moves selection only, ties go to the lowest index).
 *   expert_ffn / moe_layer: composition of the above; the transformers
 *       InklingMoE golden vectors pin the composition order.
 */
#include "sepia_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#include "../sepia_amd/csrc/iq_tables.h"

static const uint64_t k_iq2xs_grid[512] = SEPIA_IQ2XS_GRID_INIT;
static const uint32_t k_iq3xxs_grid[256] = SEPIA_IQ3XXS_GRID_INIT;
static const int8_t k_iq4nl[16] = SEPIA_IQ4NL_VALUES_INIT;
static uint64_t g_iq2xxs_grid[256];
static int g_have_iq2xxs;

void orc_set_iq2xxs_grid(const uint64_t *grid256) {
    if (!grid256) { g_have_iq2xxs = 0; return; }
    memcpy(g_iq2xxs_grid, grid256, sizeof g_iq2xxs_grid);
    g_have_iq2xxs = 1;
}

/* ------------------------------------------------------------ sizes ---- */
/* Block geometry: src/quants.c:28-56 for the reference's types,
 * tools/gguf_inspect.py:109-117 for Q2_K (84 B), Q3_K (110 B), IQ2_XXS (66 B). */
static int geom(int t, int64_t *elems, size_t *bytes) {
    int64_t e; size_t b;
    switch (t) {
    case ORC_T_F32: e = 1; b = 4; break;
    case ORC_T_F16: e = 1; b = 2; break;
    case ORC_T_Q8_0: e = 32; b = 34; break;
    case ORC_T_Q2_K: e = 256; b = 84; break;
    case ORC_T_Q3_K: e = 256; b = 110; break;
    case ORC_T_Q4_K: e = 256; b = 144; break;
    case ORC_T_Q5_K: e = 256; b = 176; break;
    case ORC_T_Q6_K: e = 256; b = 210; break;
    case ORC_T_IQ2_XXS: if (!g_have_iq2xxs) return 0; e = 256; b = 66; break;
    case ORC_T_IQ2_XS: e = 256; b = 74; break;
    case ORC_T_IQ3_XXS: e = 256; b = 98; break;
    case ORC_T_IQ4_XS: e = 256; b = 136; break;
    default: return 0;
    }
    if (elems) *elems = e;
    if (bytes) *bytes = b;
    return 1;
}

int orc_supported(int t) { return geom(t, NULL, NULL); }
int64_t orc_block_elems(int t) { int64_t e = 0; return geom(t, &e, NULL) ? e : 0; }
size_t orc_block_bytes(int t) { size_t b = 0; return geom(t, NULL, &b) ? b : 0; }
size_t orc_row_bytes(int t, int64_t n) {
    int64_t e; size_t b;
    if (!geom(t, &e, &b) || n < 0 || n % e) return 0;
    return (size_t)(n / e) * b;
}

/* ------------------------------------------------------------ f16 ------ */
/* src/quants.c:58-77: exact IEEE binary16 -> binary32, subnormals normalised,
 * inf/nan keep their payload. */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    int32_t e = (h >> 10) & 31;
    uint32_t m = h & 0x3FFu, out;
    if (e == 31) {
        out = sign | 0x7F800000u | (m << 13);
    } else if (e != 0) {
        out = sign | ((uint32_t)(e + 112) << 23) | (m << 13);
    } else if (m == 0) {
        out = sign;
    } else {
        int32_t ee = 113;                 /* exponent of 2^-14, the f16 subnormal scale */
        while (!(m & 0x400u)) { m <<= 1; ee--; }
        out = sign | ((uint32_t)ee << 23) | ((m & 0x3FFu) << 13);
    }
    float f;
    memcpy(&f, &out, 4);
    return f;
}

static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline uint32_t rd32(const uint8_t *p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
static inline float h2f(const uint8_t *p) { return orc_f16_to_f32(rd16(p)); }

/* ---------------------------------------------------------- decoders ---- */
/* Each decodes ONE block into out[]. Rounding order per the reference line
 * cited; every `a * b - c` is two separately rounded operations. */

/* src/quants.c:85-94: y = d * q, q int8. */
static void blk_q8_0(const uint8_t *b, float *out) {
    const float d = h2f(b);
    for (int i = 0; i < 32; i++) out[i] = d * (float)(int8_t)b[2 + i];
}

/* 6-bit (scale, min) pair number j of the 12 packed K-quant scale bytes
 * (src/quants.c:96-102): j < 4 keeps the low 6 bits of bytes j and j+4;
 * j >= 4 joins a nibble of byte j+4 with the top 2 bits of byte j-4 / j. */
static void k4_scale_min(const uint8_t *s, int j, int *sc, int *mn) {
    if (j < 4) {
        *sc = s[j] & 63;
        *mn = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
        *mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

/* src/quants.c:104-125. Layout {f16 d@0, f16 dmin@2, scales[12]@4, qs[128]@16}.
 * 64-weight chunk c: low nibbles of qs[32c..32c+31] are sub-block 2c, high
 * nibbles sub-block 2c+1; y = (d*sc)*q - (dmin*m). */
static void blk_q4_k(const uint8_t *b, float *out) {
    const float d = h2f(b), dmin = h2f(b + 2);
    const uint8_t *qs = b + 16;
    for (int c = 0; c < 4; c++) {
        for (int half = 0; half < 2; half++) {
            int sc, mn;
            k4_scale_min(b + 4, 2 * c + half, &sc, &mn);
            const float ds = d * (float)sc, dm = dmin * (float)mn;
            for (int l = 0; l < 32; l++) {
                int q = half ? (qs[32 * c + l] >> 4) : (qs[32 * c + l] & 15);
                out[64 * c + 32 * half + l] = ds * (float)q - dm;
            }
        }
    }
}

/* src/quants.c:127-151. Layout {d@0, dmin@2, scales[12]@4, qh[32]@16, ql[128]@48}.
 * As Q4_K plus a fifth bit: qh[l] bit (2c + half) adds 16. */
static void blk_q5_k(const uint8_t *b, float *out) {
    const float d = h2f(b), dmin = h2f(b + 2);
    const uint8_t *qh = b + 16, *ql = b + 48;
    for (int c = 0; c < 4; c++) {
        for (int half = 0; half < 2; half++) {
            int sc, mn;
            k4_scale_min(b + 4, 2 * c + half, &sc, &mn);
            const float ds = d * (float)sc, dm = dmin * (float)mn;
            for (int l = 0; l < 32; l++) {
                int q = half ? (ql[32 * c + l] >> 4) : (ql[32 * c + l] & 15);
                if (qh[l] & (1u << (2 * c + half))) q += 16;
                out[64 * c + 32 * half + l] = ds * (float)q - dm;
            }
        }
    }
}

/* src/quants.c:153-177. Layout {ql[128]@0, qh[64]@128, int8 sc[16]@192, f16 d@208}.
 * Half h (128 weights) uses ql[64h..], qh[32h..], sc[8h..]. Weight 32r + l of
 * the half (r = 0..3, l = 0..31): low 4 bits from ql[l + 32*(r&1)] (nibble r>>1),
 * 2 high bits from qh[l] >> 2r, minus 32; y = (d * sc[r*2 + l/16]) * q. */
static void blk_q6_k(const uint8_t *b, float *out) {
    const float d = h2f(b + 208);
    for (int h = 0; h < 2; h++) {
        const uint8_t *ql = b + 64 * h, *qh = b + 128 + 32 * h;
        const int8_t *sc = (const int8_t *)(b + 192 + 8 * h);
        for (int r = 0; r < 4; r++) {
            for (int l = 0; l < 32; l++) {
                int lo = ql[l + 32 * (r & 1)];
                lo = (r >> 1) ? (lo >> 4) : (lo & 15);
                int q = (lo | (((qh[l] >> (2 * r)) & 3) << 4)) - 32;
                out[128 * h + 32 * r + l] = d * (float)sc[2 * r + l / 16] * (float)q;
            }
        }
    }
}

/* ggml Q2_K (public format; not in the reference). Layout
 * {scales[16]@0 (low nibble scale, high nibble min), qs[64]@16, f16 d@80, f16 dmin@82}.
 * Half h: qs[32h..32h+31]; bit pair s (shift 2s) of qs[32h + l] is weight
 * 128h + 32s + l, in 16-weight group 8h + 2s + (l >= 16);
 * y = (d*sc)*q - (dmin*m). */
static void blk_q2_k(const uint8_t *b, float *out) {
    const float d = h2f(b + 80), dmin = h2f(b + 82);
    for (int h = 0; h < 2; h++) {
        const uint8_t *qs = b + 16 + 32 * h;
        for (int s = 0; s < 4; s++) {
            for (int g = 0; g < 2; g++) {
                const uint8_t scb = b[8 * h + 2 * s + g];
                const float dl = d * (float)(scb & 15), ml = dmin * (float)(scb >> 4);
                for (int l = 0; l < 16; l++) {
                    int q = (qs[16 * g + l] >> (2 * s)) & 3;
                    out[128 * h + 32 * s + 16 * g + l] = dl * (float)q - ml;
                }
            }
        }
    }
}

/* 16 six-bit Q3_K scales from the 12 packed bytes at b+96: scale j takes the
 * low (j < 8) or high (j >= 8) nibble of byte j % 8, and bits 2*(j/4)..+1 of
 * byte 8 + j % 4 as its top two bits; the stored value is biased by +32. */
static int q3_scale(const uint8_t *s, int j) {
    int lo = (j < 8) ? (s[j] & 15) : (s[j - 8] >> 4);
    int hi = (s[8 + (j & 3)] >> (2 * (j >> 2))) & 3;
    return (lo | (hi << 4)) - 32;
}

/* ggml Q3_K (public format; not in the reference). Layout
 * {hmask[32]@0, qs[64]@32, scales[12]@96, f16 d@108}. Weight 128h + 32s + 16g + l
 * (as Q2_K) has low bits (qs[32h + 16g + l] >> 2s) & 3 and is lowered by 4
 * unless hmask[16g + l] has bit 4h + s set; y = (d * scale) * q. */
static void blk_q3_k(const uint8_t *b, float *out) {
    const float d = h2f(b + 108);
    const uint8_t *hm = b, *qsb = b + 32, *scb = b + 96;
    for (int h = 0; h < 2; h++) {
        const uint8_t *qs = qsb + 32 * h;
        for (int s = 0; s < 4; s++) {
            for (int g = 0; g < 2; g++) {
                const float dl = d * (float)q3_scale(scb, 8 * h + 2 * s + g);
                for (int l = 0; l < 16; l++) {
                    int q = (qs[16 * g + l] >> (2 * s)) & 3;
                    if (!(hm[16 * g + l] & (1u << (4 * h + s)))) q -= 4;
                    out[128 * h + 32 * s + 16 * g + l] = dl * (float)q;
                }
            }
        }
    }
}

static inline uint8_t sign_bits(int idx7) {
    return (uint8_t)(idx7 | ((__builtin_popcount((unsigned)idx7) & 1) << 7));
}

/* src/quants.c:179-201. Layout {d@0, u16 qs[32]@2, scales[8]@66}. Group of
 * 32 (ib): db = (d * (0.5 + nibble)) * 0.25, low nibble for its first 16
 * weights, high for the last 16; each u16 = 9-bit grid index | 7-bit signs. */
static void blk_iq2_xs(const uint8_t *b, float *out) {
    const float d = h2f(b);
    for (int ib = 0; ib < 8; ib++) {
        const uint8_t sb = b[66 + ib];
        for (int l = 0; l < 4; l++) {
            const float db = d * (0.5f + (float)((l < 2) ? (sb & 15) : (sb >> 4))) * 0.25f;
            const uint16_t v = rd16(b + 2 + 2 * (4 * ib + l));
            const uint64_t g = k_iq2xs_grid[v & 511];
            const uint8_t sg = sign_bits(v >> 9);
            for (int j = 0; j < 8; j++) {
                const float m = (float)((g >> (8 * j)) & 0xFF);
                out[32 * ib + 8 * l + j] = db * m * ((sg >> j) & 1 ? -1.0f : 1.0f);
            }
        }
    }
}

/* ggml IQ2_XXS (public format; not in the reference). Layout {d@0, qs[64]@2}.
 * Group ib: u32 a = bytes 8ib..8ib+3 (4 grid indices), u32 s = next 4 bytes
 * (4 x 7-bit sign indices, 4-bit scale in the top nibble);
 * db = (d * (0.5 + (s >> 28))) * 0.25. */
static void blk_iq2_xxs(const uint8_t *b, float *out) {
    const float d = h2f(b);
    for (int ib = 0; ib < 8; ib++) {
        const uint8_t *q = b + 2 + 8 * ib;
        const uint32_t s = rd32(q + 4);
        const float db = d * (0.5f + (float)(s >> 28)) * 0.25f;
        for (int l = 0; l < 4; l++) {
            const uint64_t g = g_iq2xxs_grid[q[l]];
            const uint8_t sg = sign_bits((s >> (7 * l)) & 127);
            for (int j = 0; j < 8; j++) {
                const float m = (float)((g >> (8 * j)) & 0xFF);
                out[32 * ib + 8 * l + j] = db * m * ((sg >> j) & 1 ? -1.0f : 1.0f);
            }
        }
    }
}

/* src/quants.c:203-226. Layout {d@0, qs[64]@2, scales_and_signs[32]@66}.
 * Group ib: u32 a at 66 + 4ib; db = (d * (0.5 + (a >> 28))) * 0.5; eight
 * weights per step l take grid entries qs[8ib + 2l], qs[8ib + 2l + 1] and
 * signs (a >> 7l) & 127. */
static void blk_iq3_xxs(const uint8_t *b, float *out) {
    const float d = h2f(b);
    for (int ib = 0; ib < 8; ib++) {
        const uint32_t a = rd32(b + 66 + 4 * ib);
        const float db = d * (0.5f + (float)(a >> 28)) * 0.5f;
        for (int l = 0; l < 4; l++) {
            const uint8_t sg = sign_bits((a >> (7 * l)) & 127);
            for (int half = 0; half < 2; half++) {
                const uint32_t g = k_iq3xxs_grid[b[2 + 8 * ib + 2 * l + half]];
                for (int j = 0; j < 4; j++) {
                    const float m = (float)((g >> (8 * j)) & 0xFF);
                    const int bit = 4 * half + j;
                    out[32 * ib + 8 * l + bit] = db * m * ((sg >> bit) & 1 ? -1.0f : 1.0f);
                }
            }
        }
    }
}

/* src/quants.c:228-248. Layout {d@0, u16 scales_h@2, scales_l[4]@4, qs[128]@8}.
 * Group ib: 6-bit ls = nibble ib of scales_l | 2 bits of scales_h << 4;
 * dl = d * (ls - 32); y = dl * kvalues[nibble]. */
static void blk_iq4_xs(const uint8_t *b, float *out) {
    const float d = h2f(b);
    const uint16_t sh = rd16(b + 2);
    for (int ib = 0; ib < 8; ib++) {
        const int ls = ((b[4 + ib / 2] >> (4 * (ib & 1))) & 15) | (((sh >> (2 * ib)) & 3) << 4);
        const float dl = d * (float)(ls - 32);
        const uint8_t *qs = b + 8 + 16 * ib;
        for (int j = 0; j < 16; j++) {
            out[32 * ib + j] = dl * (float)k_iq4nl[qs[j] & 15];
            out[32 * ib + 16 + j] = dl * (float)k_iq4nl[qs[j] >> 4];
        }
    }
}

/* src/quants.c:250-265: per-type dispatch over whole blocks. */
int orc_dequantize_row(int t, const void *src, float *dst, int64_t n) {
    int64_t e; size_t bb;
    if (!geom(t, &e, &bb) || n < 0 || n % e) return 0;
    const uint8_t *p = (const uint8_t *)src;
    if (t == ORC_T_F32) { memcpy(dst, src, (size_t)n * 4); return 1; }
    if (t == ORC_T_F16) {
        for (int64_t i = 0; i < n; i++) dst[i] = h2f(p + 2 * i);
        return 1;
    }
    void (*fn)(const uint8_t *, float *) = NULL;
    switch (t) {
    case ORC_T_Q8_0: fn = blk_q8_0; break;
    case ORC_T_Q2_K: fn = blk_q2_k; break;
    case ORC_T_Q3_K: fn = blk_q3_k; break;
    case ORC_T_Q4_K: fn = blk_q4_k; break;
    case ORC_T_Q5_K: fn = blk_q5_k; break;
    case ORC_T_Q6_K: fn = blk_q6_k; break;
    case ORC_T_IQ2_XXS: fn = blk_iq2_xxs; break;
    case ORC_T_IQ2_XS: fn = blk_iq2_xs; break;
    case ORC_T_IQ3_XXS: fn = blk_iq3_xxs; break;
    case ORC_T_IQ4_XS: fn = blk_iq4_xs; break;
    default: return 0;
    }
    for (int64_t k = 0; k < n / e; k++) fn(p + (size_t)k * bb, dst + k * e);
    return 1;
}

/* ----------------------------------------------------------- qlinear ---- */
/* src/sepia.c:731-735 (dotf) and :748-753 (qlinear); tools/test_quants.c:30-39:
 * dequantize the row, then a sequential double-precision dot, rounded to f32. */
typedef struct {
    int t;
    const uint8_t *w;
    size_t row_bytes;
    int64_t in_dim, r0, r1;
    const float *x;
    float *y;
    int ok;
} QlinJob;

static void *qlin_worker(void *arg) {
    QlinJob *j = (QlinJob *)arg;
    float *row = (float *)malloc((size_t)j->in_dim * sizeof(float));
    if (!row) { j->ok = 0; return NULL; }
    for (int64_t o = j->r0; o < j->r1; o++) {
        orc_dequantize_row(j->t, j->w + (size_t)o * j->row_bytes, row, j->in_dim);
        double acc = 0.0;
        for (int64_t i = 0; i < j->in_dim; i++) acc += (double)row[i] * (double)j->x[i];
        j->y[o] = (float)acc;
    }
    free(row);
    j->ok = 1;
    return NULL;
}

int orc_qlinear(int t, const void *w, int64_t out_dim, int64_t in_dim, const float *x, float *y, int threads) {
    size_t rb = orc_row_bytes(t, in_dim);
    if (!rb || out_dim < 0 || !w || !x || !y) return 0;
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    if ((int64_t)threads > out_dim) threads = out_dim > 0 ? (int)out_dim : 1;
    QlinJob jobs[256];
    pthread_t tid[256];
    for (int k = 0; k < threads; k++) {
        jobs[k] = (QlinJob){ t, (const uint8_t *)w, rb, in_dim,
                             out_dim * k / threads, out_dim * (k + 1) / threads, x, y, 0 };
    }
    if (threads == 1) { qlin_worker(&jobs[0]); return jobs[0].ok; }
    int started = 0;
    for (int k = 0; k < threads; k++) {
        if (pthread_create(&tid[k], NULL, qlin_worker, &jobs[k]) != 0) break;
        started++;
    }
    for (int k = started; k < threads; k++) qlin_worker(&jobs[k]);
    for (int k = 0; k < started; k++) pthread_join(tid[k], NULL);
    int ok = 1;
    for (int k = 0; k < threads; k++) ok &= jobs[k].ok;
    return ok;
}

/* src/sepia.c:737-740 (linear over f32 rows via dotf). */
void orc_linear_f32(const float *w, int64_t out_dim, int64_t in_dim, const float *x, float *y) {
    for (int64_t o = 0; o < out_dim; o++) {
        const float *r = w + (size_t)o * (size_t)in_dim;
        double acc = 0.0;
        for (int64_t i = 0; i < in_dim; i++) acc += (double)r[i] * (double)x[i];
        y[o] = (float)acc;
    }
}

/* ------------------------------------------------------ activations ---- */
/* src/sepia.c:755-762. */
float orc_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }
float orc_silu(float x) { return x * orc_sigmoid(x); }
float orc_logsigmoid(float x) {
    if (x >= 0.0f) return -log1pf(expf(-x));
    return x - log1pf(expf(x));
}
/* src/sepia.c:3015 / metal/ops.metal:128-136: z = silu(g) * u. */
void orc_silu_mul(const float *g, const float *u, float *z, int64_t n) {
    for (int64_t i = 0; i < n; i++) z[i] = orc_silu(g[i]) * u[i];
}

/* ------------------------------------------------------------ router ---- */
/* src/sepia.c:1329-1353 (moe_route_select, selection half); spec
 * docs/architecture-notes.md:342-394. score = sigmoid(logit) + bias; top-k by
 * repeated argmax with a strict '>' so ties resolve to the lowest index. */
void orc_route_topk(const float *logits, const float *bias, int n_routed, int topk, int *idx) {
    float *score = (float *)malloc(sizeof(float) * (size_t)n_routed);
    unsigned char *taken = (unsigned char *)calloc((size_t)n_routed, 1);
    for (int i = 0; i < n_routed; i++) score[i] = orc_sigmoid(logits[i]) + bias[i];
    for (int k = 0; k < topk; k++) {
        int best = -1;
        for (int i = 0; i < n_routed; i++) {
            if (taken[i]) continue;
            if (best < 0 || score[i] > score[best]) best = i;
        }
        idx[k] = best;
        taken[best] = 1;
    }
    free(score);
    free(taken);
}

/* src/sepia.c:1355-1372 (moe_route_select, weight half): over the selected
 * RAW logits plus the shared-sink logits, logsigmoid in float, a float max,
 * exp of the float difference summed in double, lse = max + log(sum), then
 * w = exp(lp - lse) * route_scale * global_scale in double, rounded to float. */
void orc_route_weights(const float *logits, int n_routed, int n_shared, const int *idx, int topk,
                       double route_scale, double global_scale, float *weights) {
    const int n_sel = topk + n_shared;
    float lp[64] = { 0 };
    if (n_sel < 1 || n_sel > 64) return;
    for (int k = 0; k < n_sel; k++) {
        const float raw = (k < topk) ? logits[idx[k]] : logits[n_routed + (k - topk)];
        lp[k] = orc_logsigmoid(raw);
    }
    float lmax = lp[0];
    for (int k = 1; k < n_sel; k++) if (lp[k] > lmax) lmax = lp[k];
    double se = 0.0;
    for (int k = 0; k < n_sel; k++) se += exp((double)(lp[k] - lmax));
    const double lse = (double)lmax + log(se);
    for (int k = 0; k < n_sel; k++) {
        double w = exp((double)lp[k] - lse);
        w *= route_scale * global_scale;
        weights[k] = (float)w;
    }
}

void orc_route_select(const float *logits, const float *bias, int n_routed, int n_shared, int topk,
                      double route_scale, double global_scale, int *idx, float *weights) {
    orc_route_topk(logits, bias, n_routed, topk, idx);
    orc_route_weights(logits, n_routed, n_shared, idx, topk, route_scale, global_scale, weights);
}

/* ------------------------------------------------------------ experts --- */
/* src/sepia.c:2993-3017 (real_expert_ffn): qlinear gate, qlinear up,
 * h = silu(g) * u, qlinear down. */
int orc_expert_ffn(int tg, const void *gate, int tu, const void *up, int td, const void *down,
                   int64_t hidden, int64_t inter, const float *x, float *y, int threads) {
    float *g = (float *)malloc(sizeof(float) * (size_t)inter);
    float *u = (float *)malloc(sizeof(float) * (size_t)inter);
    int ok = g && u;
    ok = ok && orc_qlinear(tg, gate, inter, hidden, x, g, threads);
    ok = ok && orc_qlinear(tu, up, inter, hidden, x, u, threads);
    if (ok) {
        orc_silu_mul(g, u, g, inter);
        ok = orc_qlinear(td, down, hidden, inter, g, y, threads);
    }
    free(g);
    free(u);
    return ok;
}

/* src/sepia.c:1377-1470 (mlp_moe_forward) with the routed experts computed
 * by real_expert_ffn (:1402-1405): router logits by dotf; routed outputs
 * weighted AFTER down and accumulated in selection order (:1425); each
 * shared expert scales its activation by gamma BEFORE down
 * (h = silu(g) * u * gamma, :1441) and adds its down output (:1448-1451). */
int orc_moe_layer(const OrcMoeLayer *L, const float *x, float *y, const int *force_idx,
                  float *logits_out, int *idx_out, float *w_out, int threads) {
    if (!L || L->topk > 32 || L->n_shared > 32 || L->topk < 1) return 0;
    const int n_total = L->n_routed + L->n_shared;
    const int64_t H = L->hidden, I = L->inter;
    float *logits = (float *)malloc(sizeof(float) * (size_t)n_total);
    float *eo = (float *)malloc(sizeof(float) * (size_t)H);
    float *g = (float *)malloc(sizeof(float) * (size_t)I);
    float *u = (float *)malloc(sizeof(float) * (size_t)I);
    int ok = logits && eo && g && u;
    int idx[32];
    float w[64];
    if (ok) {
        orc_linear_f32(L->router_w, n_total, H, x, logits);
        orc_route_select(logits, L->router_bias, L->n_routed, L->n_shared, L->topk,
                         L->route_scale, L->global_scale, idx, w);
        if (force_idx) {
            for (int k = 0; k < L->topk; k++) {
                if (force_idx[k] < 0 || force_idx[k] >= L->n_routed) ok = 0;
                idx[k] = force_idx[k];
            }
            orc_route_weights(logits, L->n_routed, L->n_shared, idx, L->topk,
                              L->route_scale, L->global_scale, w);
        }
    }
    if (ok) {
        for (int64_t d = 0; d < H; d++) y[d] = 0.0f;
        for (int k = 0; ok && k < L->topk; k++) {
            const int e = idx[k];
            ok = orc_expert_ffn(L->t_gate, L->gate[e], L->t_up, L->up[e], L->t_down, L->down[e],
                                H, I, x, eo, threads);
            for (int64_t d = 0; ok && d < H; d++) y[d] += eo[d] * w[k];
        }
        for (int s = 0; ok && s < L->n_shared; s++) {
            const float gamma = w[L->topk + s];
            ok = orc_qlinear(L->ts_gate, L->s_gate[s], I, H, x, g, threads)
              && orc_qlinear(L->ts_up, L->s_up[s], I, H, x, u, threads);
            for (int64_t i = 0; ok && i < I; i++) g[i] = orc_silu(g[i]) * u[i] * gamma;
            ok = ok && orc_qlinear(L->ts_down, L->s_down[s], H, I, g, eo, threads);
            for (int64_t d = 0; ok && d < H; d++) y[d] += eo[d];
        }
    }
    if (ok) {
        if (logits_out) memcpy(logits_out, logits, sizeof(float) * (size_t)n_total);
        if (idx_out) memcpy(idx_out, idx, sizeof(int) * (size_t)L->topk);
        if (w_out) memcpy(w_out, w, sizeof(float) * (size_t)(L->topk + L->n_shared));
    }
    free(logits);
    free(eo);
    free(g);
    free(u);
    return ok;
}

/* ---------------------------------------------------------- attention ---- */
/* rel_logits[t,h,r] = sum_d r_vec[t,h,d] * rel_proj[d,r]: the dense
 * relative-position projection of attn_forward_chunk (src/sepia.c:1203-1209,
 * inside its per-(t,h) body from :1077), accumulated in double and rounded
 * to float as there. */
void orc_rel_project(const float *r_vec, const float *rel_proj, float *rel_logits, int64_t T, int64_t H,
                     int64_t d_rel, int64_t rel_extent) {
    for (int64_t th = 0; th < T * H; th++) {
        const float *rv = r_vec + (size_t)th * (size_t)d_rel;
        for (int64_t r = 0; r < rel_extent; r++) {
            double acc = 0.0;
            for (int64_t d = 0; d < d_rel; d++) acc += (double)rv[d] * (double)rel_proj[(size_t)d * (size_t)rel_extent + r];
            rel_logits[(size_t)th * (size_t)rel_extent + r] = (float)acc;
        }
    }
}

/* The per-(t,h) banded attention of attn_forward_chunk (src/sepia.c:1211-1247) in the
 * split the GPU ABI takes (src/sepia_gpu.h, sepia_gpu_banded_attn): q is
 * already tau-scaled by the caller, tau scales the band bias only. For query
 * token t at q_pos = q_pos_base + t and kv in [kv_lo[t], kv_hi[t]]:
 * content = (double)dot_f32(q, k) * inv_head_dim (the reference's dotf, a
 * double sum rounded to float), bias = dist < rel_extent ?
 * (double)rel_logits[dist] * tau : 0 (dist = q_pos - kv), score =
 * (float)(content + bias); softmax with exp in double over (score - max)
 * and a double sum; out = sum of (double)p / sum * v in double, rounded to
 * float. GQA: head h reads kv head h / (H / Hkv). Returns 0 on a bound
 * that leaves [0, q_pos]. */
int orc_banded_attn(const float *q, const float *k, const float *v, const float *rel_logits, float *out,
                    const int64_t *kv_lo, const int64_t *kv_hi, const float *tau, int64_t T, int64_t H, int64_t Hkv,
                    int64_t Dh, int64_t rel_extent, int64_t q_pos_base, int64_t kv_dim, float inv_head_dim) {
    if (T < 1 || H < 1 || Hkv < 1 || H % Hkv || Dh < 1) return 0;
    const int64_t group = H / Hkv;
    for (int64_t t = 0; t < T; t++) {
        const int64_t q_pos = q_pos_base + t, lo = kv_lo[t], hi = kv_hi[t];
        if (lo < 0 || hi < lo || hi > q_pos) return 0;
        const int64_t n = hi - lo + 1;
        float *sc = (float *)malloc((size_t)n * sizeof(float));
        double *acc = (double *)malloc((size_t)Dh * sizeof(double));
        if (!sc || !acc) { free(sc); free(acc); return 0; }
        for (int64_t h = 0; h < H; h++) {
            const int64_t hk = h / group;
            const float *qv = q + (size_t)(t * H + h) * (size_t)Dh;
            const float *rl = rel_logits + (size_t)(t * H + h) * (size_t)rel_extent;
            float mx = -INFINITY;
            for (int64_t kv = lo; kv <= hi; kv++) {
                const float *kr = k + (size_t)kv * (size_t)kv_dim + (size_t)hk * (size_t)Dh;
                double dot = 0.0;
                for (int64_t d = 0; d < Dh; d++) dot += (double)qv[d] * (double)kr[d];
                const double content = (double)(float)dot * (double)inv_head_dim;
                const int64_t dist = q_pos - kv;
                const double bias = dist < rel_extent ? (double)rl[dist] * (double)tau[t] : 0.0;
                const float s = (float)(content + bias);
                sc[kv - lo] = s;
                if (s > mx) mx = s;
            }
            double sum = 0.0;
            for (int64_t i = 0; i < n; i++) {
                const double e = exp((double)(sc[i] - mx));
                sc[i] = (float)e;
                sum += e;
            }
            for (int64_t d = 0; d < Dh; d++) acc[d] = 0.0;
            for (int64_t i = 0; i < n; i++) {
                const double wgt = (double)sc[i] / sum;
                const float *vr = v + (size_t)(lo + i) * (size_t)kv_dim + (size_t)hk * (size_t)Dh;
                for (int64_t d = 0; d < Dh; d++) acc[d] += wgt * (double)vr[d];
            }
            float *o = out + (size_t)(t * H + h) * (size_t)Dh;
            for (int64_t d = 0; d < Dh; d++) o[d] = (float)acc[d];
        }
        free(sc);
        free(acc);
    }
    return 1;
}
