/* sepia_hip.c -- HIP host backend for SEPIA's GPU ABI on AMD Instinct MI355X.
 *
 * The counterpart of the reference's src/sepia_metal.m: it implements every
 * function of include/sepia_gpu.h (reference src/sepia_gpu.h) plus the
 * additive entries of include/sepia_hip_ext.h, over the HIP runtime C API.
 * Kernels are prebuilt for gfx950 into sepia_kernels.hsaco and loaded with
 * hipModuleLoad from the directory given to sepia_gpu_init (the reference
 * compiles metal_dir's *.metal at the same point, src/sepia_metal.m:103-149);
 * when that directory holds no code object (sepia.c passes "metal",
 * src/sepia.c:6181) the one next to this library is used.
 *
 * Single host thread, no locking, one in-order HIP stream at default
 * priority. Every function logs one "sepia: hip: ..." line and returns 0/NULL
 * on failure; nothing exits (src/sepia_gpu.h:1-3, src/sepia_metal.m:15-18).
 */
#define _GNU_SOURCE 1
#define __HIP_PLATFORM_AMD__ 1
#include <hip/hip_runtime_api.h>

#include "../../include/sepia_gpu.h"
#include "../../include/sepia_hip_ext.h"
#include "internal.h"
#include "noalloc.h"

#include <dlfcn.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

static void logf_(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    fprintf(stderr, "sepia: hip: ");
    vfprintf(stderr, fmt, ap);
    fprintf(stderr, "\n");
    va_end(ap);
}
#define LOG(...) logf_(__VA_ARGS__)

/* ------------------------------------------------------------ kernels --- */
enum {
    K_DQ_Q8_0, K_DQ_Q2_K, K_DQ_Q3_K, K_DQ_Q4_K, K_DQ_Q5_K, K_DQ_Q6_K,
    K_DQ_IQ2_XXS, K_DQ_IQ2_XS, K_DQ_IQ3_XXS, K_DQ_IQ4_XS, K_DQ_F16,
    K_MV_Q8_0, K_MV_Q2_K, K_MV_Q3_K, K_MV_Q4_K, K_MV_Q5_K, K_MV_Q6_K,
    K_MV_IQ2_XXS, K_MV_IQ2_XS, K_MV_IQ3_XXS, K_MV_IQ4_XS,
    K_MATVEC_F32, K_SILU_MUL, K_ADD, K_SCALE, K_COPY, K_TOUCH, K_RMSNORM, K_SOFTMAX,
    K_SCONV, K_SCONV_HIST, K_MOE_ROUTE, K_MOE_GATEUP, K_MOE_DOWN, K_SYNTH_FILL, K_SYNTH_F16,
    K_TILE_Q2_K, K_TILE_Q3_K, K_TILE_Q4_K,
    /* expert-FFN tile kernels: 9 (routed, shared) format pairs over
     * {Q2_K, Q3_K, Q4_K}, each gate/up (x f32), gate/up (x planes), down */
    K_FFN_BASE,
    /* matrix-core matvecs (kernels/mq.h), by mq_code: Q2_K, Q3_K, Q4_K, IQ2_XS, IQ3_XXS, Q5_K, Q6_K, IQ4_XS, Q8_0 */
    K_MQ_MV = K_FFN_BASE + 27,
    /* matrix-core expert FFN: gate/up, down */
    K_MQ_GU = K_MQ_MV + 9,
    K_MQ_DN = K_MQ_GU + 1,
    /* batched prefill MoE layer (kernels/prefill.h) */
    K_PF_ROUTE = K_MQ_DN + 1, K_PF_SELECT, K_PF_GROUP, K_PF_GATEUP, K_PF_DOWN, K_PF_COMBINE, K_PF_SPLIT,
    /* prefill router logits on the f32 matrix cores (kernels/prefill.h) */
    K_PF_ROUTE_M,
    /* u32 fill (counter words of caller-provided scratch) */
    K_FILL_U32,
    /* attention (kernels/attn.h): relative-position projection, banded attention partials and fold */
    K_REL_PROJECT, K_ATTN_PARTIAL, K_ATTN_COMBINE,
    /* prefill projections of Q2_K / Q3_K / Q4_K on the int8 matrix cores (kernels/prefill_q.h) */
    K_PF_QUANT, K_PF_GATEUP_Q, K_PF_DOWN_Q,
    /* prefill projections of the real checkpoint's formats on the f16 matrix cores (kernels/prefill_h.h) */
    K_PH_QUANT, K_PH_GATEUP, K_PH_DOWN,
    /* HBM read ceiling probe (measurement) */
    K_READ_PROBE, K_READ_PROBE_DMA,
    K_COUNT
};
#define FFN_NAMES(p) "sepia_ffn_gateup_" p, "sepia_ffn_gateup_" p "_xp", "sepia_ffn_down_" p
static const char *const k_names[K_COUNT] = {
    "sepia_dequant_rows_q8_0", "sepia_dequant_rows_q2_k", "sepia_dequant_rows_q3_k",
    "sepia_dequant_rows_q4_k", "sepia_dequant_rows_q5_k", "sepia_dequant_rows_q6_k",
    "sepia_dequant_rows_iq2_xxs", "sepia_dequant_rows_iq2_xs", "sepia_dequant_rows_iq3_xxs",
    "sepia_dequant_rows_iq4_xs", "sepia_dequant_rows_f16",
    "sepia_matvec_generic_q8_0", "sepia_matvec_generic_q2_k", "sepia_matvec_generic_q3_k",
    "sepia_matvec_generic_q4_k", "sepia_matvec_generic_q5_k", "sepia_matvec_generic_q6_k",
    "sepia_matvec_generic_iq2_xxs", "sepia_matvec_generic_iq2_xs", "sepia_matvec_generic_iq3_xxs",
    "sepia_matvec_generic_iq4_xs",
    "sepia_matvec_f32", "sepia_silu_mul_f32", "sepia_add_f32", "sepia_scale_f32", "sepia_copy_f32",
    "sepia_touch_f32", "sepia_rmsnorm_f32", "sepia_softmax_f32", "sepia_sconv_f32",
    "sepia_sconv_hist_roll_f32", "sepia_moe_route", "sepia_moe_gateup_generic", "sepia_moe_down_generic",
    "sepia_synth_fill", "sepia_synth_patch_f16",
    "sepia_mv_q2_k", "sepia_mv_q3_k", "sepia_mv_q4_k",
    FFN_NAMES("22"), FFN_NAMES("23"), FFN_NAMES("24"), FFN_NAMES("32"), FFN_NAMES("33"), FFN_NAMES("34"),
    FFN_NAMES("42"), FFN_NAMES("43"), FFN_NAMES("44"),
    "sepia_mq_mv_q2_k", "sepia_mq_mv_q3_k", "sepia_mq_mv_q4_k", "sepia_mq_mv_iq2_xs", "sepia_mq_mv_iq3_xxs",
    "sepia_mq_mv_q5_k", "sepia_mq_mv_q6_k", "sepia_mq_mv_iq4_xs", "sepia_mq_mv_q8_0",
    "sepia_mq_gateup", "sepia_mq_down",
    "sepia_pf_route", "sepia_pf_select", "sepia_pf_group", "sepia_pf_gateup", "sepia_pf_down", "sepia_pf_combine",
    "sepia_pf_split", "sepia_pf_route_m", "sepia_fill_u32",
    "sepia_rel_project_f32", "sepia_attn_partial", "sepia_attn_combine",
    "sepia_pf_quant", "sepia_pf_gateup_q", "sepia_pf_down_q",
    "sepia_ph_quant", "sepia_ph_gateup", "sepia_ph_down",
    "sepia_read_probe", "sepia_read_probe_dma",
};
#undef FFN_NAMES

/* GGUF block geometry (reference src/quants.c:28-56; tools/gguf_inspect.py:109-117). */
typedef struct {
    int type;
    int64_t elems;
    size_t bytes;
    int parts;      /* 32-weight parts per block (dequant threads per block) */
    int k_dq, k_mv; /* kernel ids, -1 if none */
    int f16_off[2]; /* byte offsets of f16 scale fields, -1 = none */
    int k_tile;     /* tile matvec kernel (kernels/mv.h), -1 if none */
    int align;      /* byte alignment the tile kernels need for a matrix base */
} TypeInfo;
static const TypeInfo k_types[] = {
    { 1, 1, 2, 1, K_DQ_F16, -1, { -1, -1 }, -1, 1 },
    { 8, 32, 34, 1, K_DQ_Q8_0, K_MV_Q8_0, { 0, -1 }, -1, 1 },
    { 10, 256, 84, 8, K_DQ_Q2_K, K_MV_Q2_K, { 80, 82 }, K_TILE_Q2_K, 4 },
    { 11, 256, 110, 8, K_DQ_Q3_K, K_MV_Q3_K, { 108, -1 }, K_TILE_Q3_K, 2 },
    { 12, 256, 144, 8, K_DQ_Q4_K, K_MV_Q4_K, { 0, 2 }, K_TILE_Q4_K, 4 },
    { 13, 256, 176, 8, K_DQ_Q5_K, K_MV_Q5_K, { 0, 2 }, -1, 1 },
    { 14, 256, 210, 8, K_DQ_Q6_K, K_MV_Q6_K, { 208, -1 }, -1, 1 },
    { 16, 256, 66, 8, K_DQ_IQ2_XXS, K_MV_IQ2_XXS, { 0, -1 }, -1, 1 },
    { 17, 256, 74, 8, K_DQ_IQ2_XS, K_MV_IQ2_XS, { 0, -1 }, -1, 1 },
    { 18, 256, 98, 8, K_DQ_IQ3_XXS, K_MV_IQ3_XXS, { 0, -1 }, -1, 1 },
    { 23, 256, 136, 8, K_DQ_IQ4_XS, K_MV_IQ4_XS, { 0, -1 }, -1, 1 },
};

/* Tile geometry (kernels/mv.h, struct TileGeo): 384-thread workgroups; a
 * row of U = in_dim / 64 units takes U lanes (U a multiple of 16 dividing
 * 384), S = 384 / U rows run side by side and a workgroup walks T <= 3 such
 * steps. x is converted per workgroup, at most two 16-column segments per
 * thread. */
#define TILE_NT 384
#define TILE_TMAX 3
#define TILE_MAX_COLS (2 * 16 * TILE_NT)
#define TILE_CUS 256    /* MI355X compute units: the grid aims at one workgroup per CU */
typedef struct {
    int32_t U, S, T, tiles;
} TileGeo;

static int g_opt_tile = 1;   /* sepia_hip_set_option("tile", 0) forces the generic kernels */
static int g_opt_mq = 1;     /* sepia_hip_set_option("mq", 0) disables the matrix-core kernels */
/* sepia_hip_set_option("mq_p" | "mq_c" | "mq_s", v) force the matrix-core
 * workgroup geometry (parts per item, item lanes, ring stages of the largest
 * format; 0 = planned) */
static int g_opt_mq_p = 0, g_opt_mq_c = 0, g_opt_mq_s = 0;
static int g_opt_mq_rdelay = 80;  /* "mq_rdelay": KB of weights a routed gate/up workgroup of the MoE layer is
                                   * charged for its late start (the selection) when workgroups are split
                                   * between routed and shared experts; 80 measured best at C3 (57.8 vs
                                   * 59.8 us per token with 0; the plateau spans 50-100) */
static int g_opt_mq_gufac = 100, g_opt_mq_dnfac = 100;   /* "mq_gufac", "mq_dnfac": percent scale on the routed
                                                         * formats' relative cost (k_mq_cost) in the gate/up
                                                         * and down splits */
static int g_opt_mq_scope = 0;     /* "mq_scope": the mq_p/mq_c/mq_s/mq_x overrides apply to every matrix-core
                                    * launch (0) or only to the matvec (1), gate/up (2) or down (3) launches */
static int g_mq_sconv = 0;         /* mq_geo may plan vector mode 3 (by default only the expert FFN's gate/up,
                                    * where it measured faster: C2 16.5 -> 15.5 us; the MoE layer's launches,
                                    * the matvecs and the FFN down measured slower or no faster with it) */
static int g_mq_kind = 0;          /* the launch kind mq_geo is planning: 1 matvec, 2 gate/up, 3 down */
static int g_opt_mq_x = 0;   /* "mq_x": 0 = planner's choice, 1 = vector from global, 2 = vector by LDS DMA,
                              * 3 = converter waves */
static int g_opt_pf_route_m = 1;   /* "pf_route_m": 1 = prefill router logits on the f32 matrix cores
                                    * (sepia_pf_route_m) when x and the router rows are 16-byte aligned
                                    * and hidden is a multiple of 512,
                                    * 0 = sepia_pf_route */
static int g_opt_pf_h = 1;   /* "pf_h": 1 = a prefill layer whose six projections all have formats of the
                              * real checkpoint (IQ2_XS, IQ3_XXS, IQ4_XS, Q5_K, Q6_K, Q8_0) runs them on the
                              * f16 matrix cores (sepia_ph_quant, sepia_ph_gateup, sepia_ph_down); 0 = the
                              * bf16 kernels */
static int g_opt_pf_q = 1;   /* "pf_q": 1 = a prefill layer whose six projections are all Q2_K, Q3_K or Q4_K
                              * runs them on the int8 matrix cores (sepia_pf_quant, sepia_pf_gateup_q,
                              * sepia_pf_down_q); 0 = the bf16 kernels sepia_pf_gateup / _down, which
                              * every other layer always takes */
static int g_opt_tile_t = 0; /* sepia_hip_set_option("tile_t", T) forces T steps per workgroup */

/* Geometry for `mats` stacked copies of a [rows, 256 * n_blocks] matrix; 0
 * when the row length does not fit the tile kernels. T is the smallest step
 * count that keeps the whole launch within about one workgroup per CU. */
static int tile_geo(int64_t n_blocks, int64_t rows, int64_t mats, TileGeo *g) {
    const int64_t U = 4 * n_blocks;
    if (U <= 0 || U % 16 || TILE_NT % U || 256 * n_blocks > TILE_MAX_COLS || rows <= 0) return 0;
    g->U = (int32_t)U;
    g->S = (int32_t)(TILE_NT / U);
    const int64_t steps = (rows + g->S - 1) / g->S;
    int64_t T = (mats * steps + TILE_CUS - 1) / TILE_CUS;
    if (g_opt_tile_t) T = g_opt_tile_t;
    g->T = (int32_t)(T < 1 ? 1 : (T > TILE_TMAX ? TILE_TMAX : T));
    g->tiles = (int32_t)((steps + g->T - 1) / g->T);
    return 1;
}

/* Dynamic LDS of a tile workgroup: x planes, scales and sums of n staged
 * columns, then `mats` matrices' row partials. */
static size_t tile_lds(int64_t n_staged, const TileGeo *g, int mats) {
    return (size_t)(3 * n_staged + 2 * (n_staged / 16) * 4) + 4 * (size_t)(mats * g->T * g->S * (g->U / 16));
}

static int g_available;
static size_t g_lds_max = 65536;    /* per-workgroup LDS limit, from the device at init */
static int g_cus = 0;               /* compute units, from the device at init */
static int g_have_iq2xxs;
static int g_noalloc_ok;            /* the allocation-free entry's device array is set up */
static char g_device_name[256];
static hipModule_t g_module;
static hipStream_t g_stream;
static hipFunction_t g_fn[K_COUNT];
static int g_batch_open;

static const TypeInfo *type_info(int t) {
    for (size_t i = 0; i < sizeof k_types / sizeof k_types[0]; i++) {
        if (k_types[i].type != t) continue;
        if (t == SEPIA_T_IQ2_XXS && !g_have_iq2xxs) return NULL;
        return &k_types[i];
    }
    return NULL;
}

/* ------------------------------------------------------------ buffers --- */
enum { BUF_SHARED = 0, BUF_PRIVATE = 1, BUF_WRAPPED = 2 };

/* Device allocations are padded by DEV_PAD bytes so a vectorised kernel may
 * read a full 16-byte line that straddles the logical end of a buffer. */
#define DEV_ALIGN 256u
#define DEV_PAD 256u

/* Shared buffers keep a pinned host copy beside the device allocation. The
 * host may write the copy only through a pointer from sepia_gpu_host_ptr,
 * so that call marks every chunk (SHADOW_CHUNK bytes) of the buffer
 * host-dirty. An op uploads, right before it is queued, the dirty parts of
 * exactly the byte range it reads, and marks clean only the chunks that
 * range covers whole: the host may still be writing the rest of a chunk it
 * covers in part (the reference's loader threads fill one expert slot of a
 * slab while ops read another slot of the same slab, src/sepia.c:3249-3290),
 * so such a chunk stays dirty until an op that reads it whole uploads it. A
 * buffer a kernel writes is downloaded whole at sepia_gpu_end. A slab the
 * host fills once is therefore uploaded once, however many batches read it,
 * and a host write that lands after an earlier op of the batch read other
 * bytes still reaches the op that reads it. */
#define SHADOW_CHUNK ((size_t)1 << 16)
struct SepiaGpuBuf {
    uint8_t *dev;
    void *host;        /* pinned copy (shared), caller's base (wrapped), NULL (private) */
    size_t len;
    int kind;
    size_t ndirty;     /* chunks of the host copy that may be newer than the device copy */
    uint64_t *dirty;   /* per-chunk host-dirty bits (shared buffers) */
    size_t nchunks;
    int dev_newer;     /* download at sepia_gpu_end */
    struct SepiaGpuBuf *prev, *next; /* registry of shared buffers */
};
static SepiaGpuBuf *g_shared;

static size_t dev_bytes(size_t len) { return ((len + DEV_ALIGN - 1) / DEV_ALIGN) * DEV_ALIGN + DEV_PAD; }

static int need_init(const char *op) {
    if (!g_available) {
        LOG("%s: GPU not initialized", op);
        return 0;
    }
    return 1;
}

static int need_batch(const char *op) {
    if (!need_init(op)) return 0;
    if (!g_batch_open) {
        LOG("%s: no active batch (call sepia_gpu_begin first)", op);
        return 0;
    }
    return 1;
}

/* ---- hooks for the other host files (internal.h) ---- */
void sepia_log(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    fprintf(stderr, "sepia: hip: ");
    vfprintf(stderr, fmt, ap);
    fprintf(stderr, "\n");
    va_end(ap);
}
int sepia_ready(const char *op) { return need_init(op); }
hipStream_t sepia_stream(void) { return g_stream; }
uint8_t *sepia_buf_dev(SepiaGpuBuf *b) { return b ? b->dev : NULL; }
size_t sepia_buf_len(const SepiaGpuBuf *b) { return b ? b->len : 0; }
int64_t sepia_row_bytes(int ggml_type, int64_t n) {
    if (n < 0) return -1;
    if (ggml_type == 0) return 4 * n;   /* F32 */
    for (size_t i = 0; i < sizeof k_types / sizeof k_types[0]; i++) {
        if (k_types[i].type != ggml_type) continue;
        if (n % k_types[i].elems) return -1;
        return n / k_types[i].elems * k_types[i].bytes;
    }
    return -1;
}

/* b holds [off, off + n) */
static int chk(const SepiaGpuBuf *b, size_t off, size_t n, const char *op, const char *what) {
    if (!b || !b->dev) {
        LOG("%s: %s buffer is NULL", op, what);
        return 0;
    }
    if (off > b->len || n > b->len - off) {
        LOG("%s: %s range [%zu, +%zu) exceeds its buffer of %zu bytes", op, what, off, n, b->len);
        return 0;
    }
    return 1;
}

/* Bytes uploaded to shared buffers' device copies since init (tests read it
 * through sepia_hip_uploaded_bytes). */
static uint64_t g_uploaded;
/* Device and pinned-host allocations the library has made since it loaded
 * (sepia_hip_alloc_count): the allocation-free entry's tests check that it
 * leaves this unchanged. */
static uint64_t g_allocs;
uint64_t sepia_hip_alloc_count(void) { return g_allocs; }
void sepia_count_alloc(void) { g_allocs++; }

/* Bring [off, off + n) of the device copy up to date before a kernel reads
 * it: upload the parts of that range that lie in host-dirty chunks,
 * coalesced into runs, and mark clean the dirty chunks it covers whole. */
static int dirty_bit(const SepiaGpuBuf *b, size_t c) { return (int)((b->dirty[c >> 6] >> (c & 63)) & 1u); }
static int sync_in_range(SepiaGpuBuf *b, size_t off, size_t n, const char *op) {
    if (b->kind != BUF_SHARED || b->ndirty == 0 || n == 0) return 1;
    if (off >= b->len) return 1;
    if (n > b->len - off) n = b->len - off;
    const size_t end = off + n;
    const size_t c0 = off / SHADOW_CHUNK, c1 = (end - 1) / SHADOW_CHUNK;
    size_t c = c0;
    while (c <= c1) {
        if (!dirty_bit(b, c)) {
            c++;
            continue;
        }
        size_t e = c;
        while (e + 1 <= c1 && dirty_bit(b, e + 1)) e++;
        const size_t lo = c * SHADOW_CHUNK > off ? c * SHADOW_CHUNK : off;
        const size_t hi = (e + 1) * SHADOW_CHUNK < end ? (e + 1) * SHADOW_CHUNK : end;
        hipError_t err = hipMemcpyAsync(b->dev + lo, (uint8_t *)b->host + lo, hi - lo, hipMemcpyHostToDevice, g_stream);
        if (err != hipSuccess) {
            LOG("%s: upload failed: %s", op, hipGetErrorString(err));
            return 0;
        }
        g_uploaded += hi - lo;
        for (size_t k = c; k <= e; k++) {
            const size_t klo = k * SHADOW_CHUNK, khi = klo + SHADOW_CHUNK < b->len ? klo + SHADOW_CHUNK : b->len;
            if (klo < off || khi > end) continue;   /* covered in part: the rest may still change */
            b->dirty[k >> 6] &= ~((uint64_t)1 << (k & 63));
            b->ndirty--;
        }
        c = e + 1;
    }
    return 1;
}
static int sync_in(SepiaGpuBuf *b, const char *op) { return sync_in_range(b, 0, b->len, op); }

/* An input read over [off, off + n) (the whole buffer with prep_in). */
static int prep_in_r(SepiaGpuBuf *b, size_t off, size_t n, const char *op) { return sync_in_range(b, off, n, op); }
static int prep_in(SepiaGpuBuf *b, const char *op) { return sync_in(b, op); }
/* An output: the whole device copy is made current first, since the buffer
 * is downloaded whole at sepia_gpu_end. */
static int prep_out(SepiaGpuBuf *b, const char *op) {
    if (!sync_in(b, op)) return 0;
    if (b->kind == BUF_SHARED) b->dev_newer = 1;
    return 1;
}

/* Library scratch in HBM: a region of arrival counters (zeroed once; every
 * kernel that uses one leaves it at zero again) followed by a data region
 * for partial sums and intermediate vectors, grown on demand. */
#define CNT_BYTES (64u * 1024u)
static void *g_scratch;
static size_t g_scratch_len;

/* Data region of at least `need` bytes (the counters sit in front of it).
 * Growing waits for the stream, since queued kernels may still use the old
 * region; the new allocation is cleared so every counter starts at zero.
 * None of that may enter a stream capture: while the library's stream is
 * being captured a region that is too small is an error (run the same call
 * once before the capture, or reserve with sepia_hip_reserve_scratch). */
static void *scratch(size_t need, const char *op) {
    if (g_scratch && need <= g_scratch_len - CNT_BYTES) return (uint8_t *)g_scratch + CNT_BYTES;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(g_stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) {
        LOG("%s: needs %zu bytes of scratch but has %zu, and the stream is being captured (growing it would "
            "allocate); run the call once before the capture or call sepia_hip_reserve_scratch",
            op, need, g_scratch ? g_scratch_len - CNT_BYTES : (size_t)0);
        return NULL;
    }
    hipStreamSynchronize(g_stream);
    if (g_scratch) hipFree(g_scratch);
    g_scratch = NULL;
    g_scratch_len = 0;
    size_t want = CNT_BYTES + (need < (4u << 20) ? (4u << 20) : need);
    g_allocs++;
    hipError_t e = hipMalloc(&g_scratch, want);
    if (e == hipSuccess) e = hipMemsetAsync(g_scratch, 0, want, g_stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
    if (e != hipSuccess) {
        LOG("%s: scratch allocation of %zu bytes failed: %s", op, want, hipGetErrorString(e));
        if (g_scratch) hipFree(g_scratch);
        g_scratch = NULL;
        return NULL;
    }
    g_scratch_len = want;
    return (uint8_t *)g_scratch + CNT_BYTES;
}

size_t sepia_hip_scratch_bytes(void) { return g_scratch_len; }

int sepia_hip_reserve_scratch(size_t bytes) {
    if (!need_init("reserve_scratch")) return 0;
    return scratch(bytes, "reserve_scratch") != NULL;
}

static SepiaGpuBuf *new_buf(size_t len, int kind) {
    SepiaGpuBuf *b = (SepiaGpuBuf *)calloc(1, sizeof *b);
    if (!b) {
        LOG("alloc: out of host memory");
        return NULL;
    }
    b->len = len;
    b->kind = kind;
    g_allocs++;
    hipError_t e = hipMalloc((void **)&b->dev, dev_bytes(len));
    if (e != hipSuccess) {
        LOG("alloc: hipMalloc(%zu) failed: %s", dev_bytes(len), hipGetErrorString(e));
        free(b);
        return NULL;
    }
    return b;
}

/* Freed buffers kept for reuse. The reference's host path allocates and
 * frees its temporaries around single ops (src/sepia.c real_forward_chunk_gpu:
 * about 36 buffers per token, most of them 0.1-400 KB), and a fresh shared
 * buffer costs a pinned host allocation, a device allocation and a stream
 * synchronisation (about 0.2 ms with its release). A freed shared or
 * private buffer of at most POOL_BUF_MAX bytes therefore goes to this pool,
 * which releases its oldest buffers to stay within POOL_MAX buffers and
 * POOL_BYTES_MAX bytes; an allocation of the same kind and length takes
 * the newest such buffer back, cleared again as a new one is (device copy
 * by a fill queued on the library's stream, host copy by memset) without
 * another synchronisation. sepia_gpu_shutdown releases the pool. */
#define POOL_MAX 256
#define POOL_BUF_MAX ((size_t)64 << 20)
#define POOL_BYTES_MAX ((size_t)512 << 20)
typedef struct {
    uint8_t *dev;
    void *host;
    uint64_t *dirty;
    size_t len;
    int kind;
} PoolEnt;
static PoolEnt g_pool[POOL_MAX];
static int g_pool_n;
static size_t g_pool_bytes;

static size_t pool_cost(const PoolEnt *p) { return dev_bytes(p->len) + (p->host ? p->len : 0); }

static void pool_release(PoolEnt *p) {
    if (p->host) hipHostFree(p->host);
    free(p->dirty);
    hipFree(p->dev);
}

static void pool_release_all(void) {
    for (int i = 0; i < g_pool_n; i++) pool_release(&g_pool[i]);
    g_pool_n = 0;
    g_pool_bytes = 0;
}

/* Entry i out of the pool, the order of the others kept (oldest first). */
static PoolEnt pool_remove(int i) {
    const PoolEnt p = g_pool[i];
    memmove(&g_pool[i], &g_pool[i + 1], (size_t)(g_pool_n - 1 - i) * sizeof g_pool[0]);
    g_pool_n--;
    g_pool_bytes -= pool_cost(&p);
    return p;
}

/* Keep b's memory for reuse, releasing the oldest kept buffers as needed;
 * 0 if the pool does not take it (the caller frees it). The stream has
 * been synchronised: nothing queued uses b or the buffers released. */
static int pool_put(SepiaGpuBuf *b) {
    if (b->kind == BUF_WRAPPED || b->len > POOL_BUF_MAX) return 0;
    const PoolEnt p = { b->dev, b->host, b->dirty, b->len, b->kind };
    while (g_pool_n > 0 && (g_pool_n == POOL_MAX || g_pool_bytes + pool_cost(&p) > POOL_BYTES_MAX)) {
        PoolEnt old = pool_remove(0);
        pool_release(&old);
    }
    g_pool[g_pool_n++] = p;
    g_pool_bytes += pool_cost(&p);
    return 1;
}

/* A cleared buffer of this kind and length from the pool, or NULL. Not
 * while the library's stream is being captured: the clearing fill would
 * become a node of the caller's graph (a fresh allocation fails there, at
 * its stream synchronisation, as before). */
static SepiaGpuBuf *pool_take(size_t len, int kind) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(g_stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return NULL;
    int i = g_pool_n - 1;
    while (i >= 0 && (g_pool[i].kind != kind || g_pool[i].len != len)) i--;
    if (i < 0) return NULL;
    SepiaGpuBuf *b = (SepiaGpuBuf *)calloc(1, sizeof *b);
    if (!b) return NULL;
    PoolEnt p = pool_remove(i);
    if (hipMemsetAsync(p.dev, 0, dev_bytes(len), g_stream) != hipSuccess) {
        pool_release(&p);
        free(b);
        return NULL;
    }
    b->dev = p.dev;
    b->len = len;
    b->kind = kind;
    if (kind == BUF_SHARED) {
        b->host = p.host;
        memset(b->host, 0, len);
        b->nchunks = (len + SHADOW_CHUNK - 1) / SHADOW_CHUNK;
        b->dirty = p.dirty;
        memset(b->dirty, 0, ((b->nchunks + 63) / 64) * sizeof(uint64_t));
        b->next = g_shared;
        if (g_shared) g_shared->prev = b;
        g_shared = b;
    }
    return b;
}

SepiaGpuBuf *sepia_gpu_alloc(size_t len, int gpu_private) {
    if (!need_init("alloc")) return NULL;
    if (len == 0) {
        LOG("alloc: zero length");
        return NULL;
    }
    SepiaGpuBuf *b = pool_take(len, gpu_private ? BUF_PRIVATE : BUF_SHARED);
    if (b) return b;
    b = new_buf(len, gpu_private ? BUF_PRIVATE : BUF_SHARED);
    if (!b) return NULL;
    hipError_t e = hipMemsetAsync(b->dev, 0, dev_bytes(len), g_stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
    if (e != hipSuccess) {
        LOG("alloc: clearing the buffer failed: %s", hipGetErrorString(e));
        hipFree(b->dev);
        free(b);
        return NULL;
    }
    if (b->kind == BUF_SHARED) {
        g_allocs++;
        e = hipHostMalloc(&b->host, len, hipHostMallocDefault);
        if (e != hipSuccess) {
            LOG("alloc: pinned host copy of %zu bytes failed: %s", len, hipGetErrorString(e));
            hipFree(b->dev);
            free(b);
            return NULL;
        }
        memset(b->host, 0, len);
        b->nchunks = (len + SHADOW_CHUNK - 1) / SHADOW_CHUNK;
        b->dirty = (uint64_t *)calloc((b->nchunks + 63) / 64, sizeof(uint64_t));
        if (!b->dirty) {
            LOG("alloc: out of host memory");
            hipHostFree(b->host);
            hipFree(b->dev);
            free(b);
            return NULL;
        }
        b->next = g_shared;
        if (g_shared) g_shared->prev = b;
        g_shared = b;
    }
    return b;
}

SepiaGpuBuf *sepia_gpu_wrap_mmap(void *base, size_t len) {
    if (!need_init("wrap_mmap")) return NULL;
    if (!base || len == 0) {
        LOG("wrap_mmap: invalid base/len");
        return NULL;
    }
    const size_t page = (size_t)sysconf(_SC_PAGESIZE);
    if ((uintptr_t)base % page) {
        LOG("wrap_mmap: base %p is not page-aligned (page=%zu)", base, page);
        return NULL;
    }
    SepiaGpuBuf *b = new_buf(len, BUF_WRAPPED);
    if (!b) return NULL;
    hipError_t e = hipMemsetAsync(b->dev + len, 0, dev_bytes(len) - len, g_stream);
    if (e == hipSuccess) e = hipMemcpyAsync(b->dev, base, len, hipMemcpyHostToDevice, g_stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
    if (e != hipSuccess) {
        LOG("wrap_mmap: copy of %zu bytes into HBM failed: %s", len, hipGetErrorString(e));
        hipFree(b->dev);
        free(b);
        return NULL;
    }
    b->host = base;
    return b;
}

void sepia_gpu_free(SepiaGpuBuf *b) {
    if (!b) return;
    if (g_available) hipStreamSynchronize(g_stream);
    if (b->kind == BUF_SHARED) {
        if (b->prev) b->prev->next = b->next;
        else g_shared = b->next;
        if (b->next) b->next->prev = b->prev;
    }
    if (g_available && pool_put(b)) {
        free(b);
        return;
    }
    if (b->kind == BUF_SHARED) {
        if (b->host) hipHostFree(b->host);
        free(b->dirty);
    }
    if (b->dev) hipFree(b->dev);
    free(b);
}

void *sepia_gpu_host_ptr(SepiaGpuBuf *b) {
    if (!b) return NULL;
    if (b->kind == BUF_PRIVATE) return NULL;
    if (b->kind == BUF_SHARED) {
        /* the caller may write anywhere in the copy from now on */
        memset(b->dirty, 0xFF, ((b->nchunks + 63) / 64) * sizeof(uint64_t));
        if (b->nchunks % 64) b->dirty[b->nchunks / 64] = ((uint64_t)1 << (b->nchunks % 64)) - 1;
        b->ndirty = b->nchunks;
    }
    return b->host;
}

uint64_t sepia_gpu_gpu_addr(SepiaGpuBuf *b) { return b ? (uint64_t)(uintptr_t)b->dev : 0; }

uint64_t sepia_hip_uploaded_bytes(void) { return g_uploaded; }

/* ------------------------------------------------------------ lifecycle - */
int sepia_gpu_available(void) { return g_available; }

/* dir/sepia_kernels.hsaco if that file exists, else the code object beside
 * this shared library. 0 if neither path fits in `path`. */
static int kernel_path(const char *dir, char *path, size_t cap) {
    if (dir && dir[0]) {
        if ((size_t)snprintf(path, cap, "%s/sepia_kernels.hsaco", dir) >= cap) return 0;
        if (access(path, R_OK) == 0) return 1;
    }
    Dl_info info;
    if (dladdr((void *)&sepia_gpu_init, &info) && info.dli_fname) {
        const char *slash = strrchr(info.dli_fname, '/');
        const int len = slash ? (int)(slash - info.dli_fname) : 1;
        const char *base = slash ? info.dli_fname : ".";
        if ((size_t)snprintf(path, cap, "%.*s/sepia_kernels.hsaco", len, base) >= cap) return 0;
        if (access(path, R_OK) == 0) return 1;
    }
    if (dir && dir[0]) snprintf(path, cap, "%s/sepia_kernels.hsaco", dir);  /* report the caller's path */
    return 1;
}

/* The device error word: a word of pinned host memory that kernels can
 * write (a bounded spin wait that expired records its code there), read by
 * the host after each batch. Its device address goes into the code object's
 * sepia_err_word; sepia_wait_ticks takes the spin-wait bound. */
static volatile uint32_t *g_err_host;
static hipDeviceptr_t g_wait_ticks_dev;
#define WAIT_TICKS_DEFAULT 200000000ull   /* 2 s of s_memrealtime (100 MHz) */

static int set_wait_ticks(uint64_t ticks) {
    hipError_t e = hipMemcpyHtoD(g_wait_ticks_dev, &ticks, sizeof ticks);
    if (e != hipSuccess) {
        LOG("setting the kernels' wait bound failed: %s", hipGetErrorString(e));
        return 0;
    }
    return 1;
}

static int err_word_setup(void) {
    hipDeviceptr_t gp;
    size_t gsz = 0;
    hipError_t e = hipModuleGetGlobal(&gp, &gsz, g_module, "sepia_err_word");
    if (e != hipSuccess || gsz != sizeof(void *)) {
        LOG("init: the code object has no device error word: %s", hipGetErrorString(e));
        return 0;
    }
    e = hipModuleGetGlobal(&g_wait_ticks_dev, &gsz, g_module, "sepia_wait_ticks");
    if (e != hipSuccess || gsz != sizeof(uint64_t)) {
        LOG("init: the code object has no wait bound: %s", hipGetErrorString(e));
        return 0;
    }
    if (!g_err_host) {
        void *h = NULL;
        g_allocs++;
        e = hipHostMalloc(&h, 256, hipHostMallocMapped | hipHostMallocCoherent);
        if (e != hipSuccess) {
            LOG("init: pinned memory for the device error word failed: %s", hipGetErrorString(e));
            return 0;
        }
        g_err_host = (volatile uint32_t *)h;
    }
    *g_err_host = 0;
    void *dp = NULL;
    e = hipHostGetDevicePointer(&dp, (void *)g_err_host, 0);
    if (e == hipSuccess) e = hipMemcpyHtoD(gp, &dp, sizeof dp);
    if (e != hipSuccess) {
        LOG("init: publishing the device error word failed: %s", hipGetErrorString(e));
        return 0;
    }
    return set_wait_ticks(WAIT_TICKS_DEFAULT);
}

/* The first error code a kernel recorded since the last call (0: none), and
 * clear it. */
unsigned sepia_hip_take_device_error(void) {
    if (!g_err_host) return 0;
    const unsigned code = *g_err_host;
    if (code) *g_err_host = 0;
    return code;
}

int sepia_gpu_init(const char *kernel_dir) {
    if (g_available) return 1;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n < 1) {
        LOG("no HIP device available (%s)", e == hipSuccess ? "0 devices" : hipGetErrorString(e));
        return 0;
    }
    if ((e = hipSetDevice(0)) != hipSuccess) {
        LOG("hipSetDevice(0) failed: %s", hipGetErrorString(e));
        return 0;
    }
    hipDeviceProp_t prop;
    if ((e = hipGetDeviceProperties(&prop, 0)) != hipSuccess) {
        LOG("hipGetDeviceProperties failed: %s", hipGetErrorString(e));
        return 0;
    }
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        LOG("device 0 is %s (%s); this library is built for gfx950 only", prop.name, prop.gcnArchName);
        return 0;
    }
    g_lds_max = prop.sharedMemPerBlock ? prop.sharedMemPerBlock : 65536;
    g_cus = prop.multiProcessorCount;
    char path[4096];
    if (!kernel_path(kernel_dir, path, sizeof path)) {
        LOG("init: kernel directory path too long");
        return 0;
    }
    if ((e = hipStreamCreate(&g_stream)) != hipSuccess) {
        LOG("failed to create a stream: %s", hipGetErrorString(e));
        return 0;
    }
    if ((e = hipModuleLoad(&g_module, path)) != hipSuccess) {
        LOG("cannot load %s: %s", path, hipGetErrorString(e));
        hipStreamDestroy(g_stream);
        return 0;
    }
    for (int k = 0; k < K_COUNT; k++) {
        if ((e = hipModuleGetFunction(&g_fn[k], g_module, k_names[k])) != hipSuccess) {
            LOG("kernel \"%s\" not found in %s: %s", k_names[k], path, hipGetErrorString(e));
            hipModuleUnload(g_module);
            hipStreamDestroy(g_stream);
            return 0;
        }
    }
    if (!err_word_setup()) {
        hipModuleUnload(g_module);
        hipStreamDestroy(g_stream);
        return 0;
    }
    /* the allocation-free decode entry's array: its device address, once,
     * with this device current */
    g_noalloc_ok = sepia_noalloc_setup();
    if (!g_noalloc_ok) LOG("init: the device array of sepia_hip_moe_decode_noalloc is unavailable");
    if (prop.name[0])
        snprintf(g_device_name, sizeof g_device_name, "%s", prop.name);
    else
        snprintf(g_device_name, sizeof g_device_name, "AMD %.200s", prop.gcnArchName);
    g_available = 1;
    g_batch_open = 0;
    g_have_iq2xxs = 0;
    return 1;
}

void sepia_gpu_shutdown(void) {
    if (!g_available) return;
    hipStreamSynchronize(g_stream);
    sepia_store_shutdown();
    pool_release_all();
    if (g_scratch) hipFree(g_scratch);
    g_scratch = NULL;
    g_scratch_len = 0;
    hipModuleUnload(g_module);
    hipStreamDestroy(g_stream);
    g_available = 0;
    g_batch_open = 0;
    g_have_iq2xxs = 0;
    g_device_name[0] = '\0';
}

const char *sepia_gpu_device_name(void) { return g_available ? g_device_name : NULL; }

void *sepia_hip_stream(void) { return g_available ? (void *)g_stream : NULL; }

/* ------------------------------------------------------------ batching -- */
int sepia_gpu_begin(void) {
    if (!need_init("begin")) return 0;
    if (g_batch_open) {
        LOG("begin: a batch is already active");
        return 0;
    }
    g_batch_open = 1;
    return 1;
}

/* Ops are launched as they are issued, so the queued work is already in
 * the GPU's hands; flush keeps the batch open (src/sepia_gpu.h:72-79). */
int sepia_gpu_flush(void) {
    if (!need_init("flush")) return 0;
    if (!g_batch_open) {
        LOG("flush: no active batch");
        return 0;
    }
    return 1;
}

int sepia_gpu_end(void) {
    if (!need_init("end")) return 0;
    if (!g_batch_open) {
        LOG("end: no active batch");
        return 0;
    }
    g_batch_open = 0;
    hipError_t e = hipSuccess;
    for (SepiaGpuBuf *b = g_shared; b && e == hipSuccess; b = b->next) {
        if (!b->dev_newer) continue;
        e = hipMemcpyAsync(b->host, b->dev, b->len, hipMemcpyDeviceToHost, g_stream);
        b->dev_newer = 0;
    }
    hipError_t s = hipStreamSynchronize(g_stream);
    if (e == hipSuccess) e = s;
    if (e != hipSuccess) {
        LOG("end: batch failed: %s", hipGetErrorString(e));
        return 0;
    }
    const unsigned code = sepia_hip_take_device_error();
    if (code) {
        LOG("end: a kernel's bounded wait expired (device error %u); the batch's outputs are invalid", code);
        return 0;
    }
    return 1;
}

/* Launch profiling (sepia_hip_profile_*): while on, every launch is
 * bracketed by a pair of HIP events recorded on the launch stream. */
#define PROF_MAX 16384
static int g_prof_on;
static int g_prof_n;
static int g_prof_overflow;
static hipEvent_t g_prof_ev[PROF_MAX][2];
static int g_prof_kid[PROF_MAX];
static int g_prof_ev_made;
static double g_prof_ms[K_COUNT];
static int64_t g_prof_cnt[K_COUNT];

/* AMD's launch extension (declared in the C++-only hip/hip_ext.h): the
 * start/stop events are attached to the dispatch itself, so their interval
 * is the kernel's execution, not the surrounding queue traffic. */
extern hipError_t hipExtModuleLaunchKernel(hipFunction_t f, uint32_t globalWorkSizeX, uint32_t globalWorkSizeY,
                                           uint32_t globalWorkSizeZ, uint32_t localWorkSizeX,
                                           uint32_t localWorkSizeY, uint32_t localWorkSizeZ, size_t sharedMemBytes,
                                           hipStream_t hStream, void **kernelParams, void **extra,
                                           hipEvent_t startEvent, hipEvent_t stopEvent, uint32_t flags);

/* Launch of kernel k on a gx x gy x gz grid of `block`-thread workgroups
 * with `lds` bytes of dynamic LDS (timed when the profiler is on). */
static int launch3(int k, unsigned gx, unsigned gy, unsigned gz, unsigned block, size_t lds, void **args,
                   const char *op) {
    if (gx == 0 || gy == 0 || gz == 0) return 1;
    hipError_t e;
    if (g_prof_on && g_prof_n < g_prof_ev_made) {
        const int slot = g_prof_n++;
        g_prof_kid[slot] = k;
        e = hipExtModuleLaunchKernel(g_fn[k], gx * block, gy, gz, block, 1, 1, lds, g_stream, args, NULL,
                                     g_prof_ev[slot][0], g_prof_ev[slot][1], 0);
    } else {
        if (g_prof_on) g_prof_overflow = 1;
        e = hipModuleLaunchKernel(g_fn[k], gx, gy, gz, block, 1, 1, (unsigned)lds, g_stream, args, NULL);
    }
    if (e != hipSuccess) {
        LOG("%s: launch of %s failed: %s", op, k_names[k], hipGetErrorString(e));
        return 0;
    }
    return 1;
}

static int launch2(int k, unsigned gx, unsigned gy, unsigned block, size_t lds, void **args, const char *op) {
    return launch3(k, gx, gy, 1, block, lds, args, op);
}

static int launch_lds(int k, unsigned grid, unsigned block, size_t lds, void **args, const char *op) {
    return launch2(k, grid, 1, block, lds, args, op);
}

static int launch(int k, unsigned grid, unsigned block, void **args, const char *op) {
    return launch_lds(k, grid, block, 0, args, op);
}

int sepia_hip_profile_start(void) {
    if (!need_init("profile_start")) return 0;
    if (g_prof_on) {
        LOG("profile_start: profiling is already on");
        return 0;
    }
    while (g_prof_ev_made < PROF_MAX) {
        if (hipEventCreate(&g_prof_ev[g_prof_ev_made][0]) != hipSuccess) break;
        if (hipEventCreate(&g_prof_ev[g_prof_ev_made][1]) != hipSuccess) {
            hipEventDestroy(g_prof_ev[g_prof_ev_made][0]);
            break;
        }
        g_prof_ev_made++;
    }
    if (g_prof_ev_made == 0) {
        LOG("profile_start: cannot create events");
        return 0;
    }
    g_prof_on = 1;
    g_prof_n = 0;
    return 1;
}

int sepia_hip_profile_stop(void) {
    if (!need_init("profile_stop")) return 0;
    if (!g_prof_on) {
        LOG("profile_stop: profiling is off");
        return 0;
    }
    g_prof_on = 0;
    hipError_t e = hipStreamSynchronize(g_stream);
    for (int i = 0; i < g_prof_n && e == hipSuccess; i++) {
        float ms = 0.0f;
        e = hipEventElapsedTime(&ms, g_prof_ev[i][0], g_prof_ev[i][1]);
        g_prof_ms[g_prof_kid[i]] += ms;
        g_prof_cnt[g_prof_kid[i]]++;
    }
    g_prof_n = 0;
    if (e != hipSuccess) {
        LOG("profile_stop: %s", hipGetErrorString(e));
        return 0;
    }
    if (g_prof_overflow) LOG("profile_stop: more than %d launches; the rest were not timed", g_prof_ev_made);
    g_prof_overflow = 0;
    return 1;
}

int sepia_hip_profile_query(const char *kernel, int64_t *launches, double *total_ms) {
    for (int k = 0; k < K_COUNT; k++) {
        if (!kernel || strcmp(kernel, k_names[k]) != 0) continue;
        if (launches) *launches = g_prof_cnt[k];
        if (total_ms) *total_ms = g_prof_ms[k];
        return 1;
    }
    LOG("profile_query: unknown kernel \"%s\"", kernel ? kernel : "(null)");
    return 0;
}

void sepia_hip_profile_reset(void) {
    memset(g_prof_ms, 0, sizeof g_prof_ms);
    memset(g_prof_cnt, 0, sizeof g_prof_cnt);
}

static unsigned blocks_for(int64_t n, int64_t per) { return (unsigned)((n + per - 1) / per); }

#define MAX_GRID ((int64_t)0x7FFFFFFF)

/* ------------------------------------------------------------ f32 ops --- */
static int f32_off_ok(size_t off, const char *op, const char *what) {
    if (off % 4) {
        LOG("%s: %s offset %zu is not 4-byte aligned", op, what, off);
        return 0;
    }
    return 1;
}

static int do_matvec_f32(const char *op, SepiaGpuBuf *w, size_t w_off, SepiaGpuBuf *x, SepiaGpuBuf *y,
                         int64_t out_dim, int64_t in_dim) {
    if (!w || !x || !y || out_dim <= 0 || in_dim <= 0 || (out_dim + 3) / 4 > MAX_GRID) {
        LOG("%s: invalid arguments", op);
        return 0;
    }
    if (!f32_off_ok(w_off, op, "w") ||
        !chk(w, w_off, (size_t)out_dim * (size_t)in_dim * 4, op, "w") ||
        !chk(x, 0, (size_t)in_dim * 4, op, "x") || !chk(y, 0, (size_t)out_dim * 4, op, "y"))
        return 0;
    if (!need_batch(op) || !prep_in_r(w, w_off, (size_t)out_dim * (size_t)in_dim * 4, op) || !prep_in(x, op) ||
        !prep_out(y, op))
        return 0;
    const float *wp = (const float *)(w->dev + w_off);
    int64_t ld = in_dim;
    void *args[] = { &wp, &ld, &x->dev, &y->dev, &out_dim, &in_dim };
    return launch(K_MATVEC_F32, blocks_for(out_dim, 4), 256, args, op);
}

int sepia_gpu_matvec(SepiaGpuBuf *w, SepiaGpuBuf *x, SepiaGpuBuf *y, int64_t out_dim, int64_t in_dim) {
    return do_matvec_f32("matvec", w, 0, x, y, out_dim, in_dim);
}

int sepia_gpu_matvec_off(SepiaGpuBuf *w, size_t w_off, SepiaGpuBuf *x, SepiaGpuBuf *y, int64_t out_dim,
                         int64_t in_dim) {
    return do_matvec_f32("matvec_off", w, w_off, x, y, out_dim, in_dim);
}

static int do_rmsnorm(const char *op, SepiaGpuBuf *w, size_t w_off, SepiaGpuBuf *x, SepiaGpuBuf *y,
                      int64_t rows, int64_t n, float eps) {
    if (!w || !x || !y || rows <= 0 || n <= 0 || rows > MAX_GRID) {
        LOG("%s: invalid arguments", op);
        return 0;
    }
    if (!f32_off_ok(w_off, op, "w") || !chk(w, w_off, (size_t)n * 4, op, "w") ||
        !chk(x, 0, (size_t)rows * (size_t)n * 4, op, "x") || !chk(y, 0, (size_t)rows * (size_t)n * 4, op, "y"))
        return 0;
    if (!need_batch(op) || !prep_in_r(w, w_off, (size_t)n * 4, op) || !prep_in(x, op) || !prep_out(y, op)) return 0;
    const float *wp = (const float *)(w->dev + w_off);
    void *args[] = { &wp, &x->dev, &y->dev, &n, &eps };
    return launch(K_RMSNORM, (unsigned)rows, 256, args, op);
}

int sepia_gpu_rmsnorm(SepiaGpuBuf *w, SepiaGpuBuf *x, SepiaGpuBuf *y, int64_t rows, int64_t n, float eps) {
    return do_rmsnorm("rmsnorm", w, 0, x, y, rows, n, eps);
}

int sepia_gpu_rmsnorm_off(SepiaGpuBuf *w, size_t w_off, SepiaGpuBuf *x, SepiaGpuBuf *y, int64_t rows, int64_t n,
                          float eps) {
    return do_rmsnorm("rmsnorm_off", w, w_off, x, y, rows, n, eps);
}

static int elementwise_ok(const char *op, int64_t n) {
    if (n <= 0 || (n + 255) / 256 > MAX_GRID) {
        LOG("%s: invalid arguments", op);
        return 0;
    }
    return 1;
}

int sepia_gpu_silu_mul(SepiaGpuBuf *g, SepiaGpuBuf *u, SepiaGpuBuf *z, int64_t n) {
    const char *op = "silu_mul";
    if (!g || !u || !z || !elementwise_ok(op, n)) {
        if (!g || !u || !z) LOG("%s: invalid arguments", op);
        return 0;
    }
    size_t nb = (size_t)n * 4;
    if (!chk(g, 0, nb, op, "g") || !chk(u, 0, nb, op, "u") || !chk(z, 0, nb, op, "z")) return 0;
    if (!need_batch(op) || !prep_in(g, op) || !prep_in(u, op) || !prep_out(z, op)) return 0;
    void *args[] = { &g->dev, &u->dev, &z->dev, &n };
    return launch(K_SILU_MUL, blocks_for(n, 256), 256, args, op);
}

int sepia_gpu_add(SepiaGpuBuf *a, SepiaGpuBuf *b, SepiaGpuBuf *out, int64_t n) {
    const char *op = "add";
    if (!a || !b || !out || !elementwise_ok(op, n)) {
        if (!a || !b || !out) LOG("%s: invalid arguments", op);
        return 0;
    }
    size_t nb = (size_t)n * 4;
    if (!chk(a, 0, nb, op, "a") || !chk(b, 0, nb, op, "b") || !chk(out, 0, nb, op, "out")) return 0;
    if (!need_batch(op) || !prep_in(a, op) || !prep_in(b, op) || !prep_out(out, op)) return 0;
    void *args[] = { &a->dev, &b->dev, &out->dev, &n };
    return launch(K_ADD, blocks_for(n, 256), 256, args, op);
}

int sepia_gpu_scale(float scale, SepiaGpuBuf *x, SepiaGpuBuf *y, int64_t n) {
    const char *op = "scale";
    if (!x || !y || !elementwise_ok(op, n)) {
        if (!x || !y) LOG("%s: invalid arguments", op);
        return 0;
    }
    size_t nb = (size_t)n * 4;
    if (!chk(x, 0, nb, op, "x") || !chk(y, 0, nb, op, "y")) return 0;
    if (!need_batch(op) || !prep_in(x, op) || !prep_out(y, op)) return 0;
    void *args[] = { &x->dev, &y->dev, &n, &scale };
    return launch(K_SCALE, blocks_for(n, 256), 256, args, op);
}

int sepia_gpu_copy(SepiaGpuBuf *src, size_t src_off, SepiaGpuBuf *dst, size_t dst_off, int64_t n) {
    const char *op = "copy";
    if (!src || !dst || !elementwise_ok(op, n)) {
        if (!src || !dst) LOG("%s: invalid arguments", op);
        return 0;
    }
    size_t nb = (size_t)n * 4;
    if (!f32_off_ok(src_off, op, "src") || !f32_off_ok(dst_off, op, "dst") ||
        !chk(src, src_off, nb, op, "src") || !chk(dst, dst_off, nb, op, "dst"))
        return 0;
    if (!need_batch(op) || !prep_in(src, op) || !prep_out(dst, op)) return 0;
    const uint8_t *s = src->dev + src_off;
    uint8_t *d = dst->dev + dst_off;
    void *args[] = { &s, &d, &n };
    return launch(K_COPY, blocks_for(n, 256), 256, args, op);
}

int sepia_hip_read_probe(SepiaGpuBuf *buf, size_t off, size_t bytes, unsigned grid) {
    const char *op = "read_probe";
    if (!buf || bytes == 0 || bytes % 16 || off % 16 || grid == 0 || grid > MAX_GRID) {
        LOG("%s: invalid arguments (16-byte aligned offset and size, 1 <= grid <= %d)", op, MAX_GRID);
        return 0;
    }
    if (!chk(buf, off, bytes, op, "buf") || !need_batch(op) || !prep_in_r(buf, off, bytes, op)) return 0;
    uint32_t *sink = (uint32_t *)scratch((size_t)grid * 4, op);
    if (!sink) return 0;
    const uint8_t *p = buf->dev + off;
    int64_t n16 = (int64_t)(bytes / 16);
    void *args[] = { &p, &n16, &sink };
    return launch(K_READ_PROBE, grid, 256, args, op);
}

int sepia_hip_read_probe_dma(SepiaGpuBuf *buf, size_t off, size_t bytes, unsigned grid, unsigned threads, int kb,
                             int stages) {
    const char *op = "read_probe_dma";
    const int shape = kb * 8 + stages;
    const size_t lds = (size_t)(threads / 64) * (size_t)stages * (size_t)kb * 1024;
    if (!buf || bytes == 0 || bytes % 16 || off % 16 || grid == 0 || grid > MAX_GRID || threads < 64 ||
        threads > 1024 || threads % 64 ||
        !(shape == 7 * 8 + 1 || shape == 7 * 8 + 2 || shape == 4 * 8 + 1 || shape == 4 * 8 + 2 ||
          shape == 4 * 8 + 4 || shape == 2 * 8 + 4 || shape == 1 * 8 + 4) ||
        lds > g_lds_max || (bytes / grid + 16) >= (1ull << 32)) {
        LOG("%s: invalid arguments (16-byte aligned offset and size, 1 <= grid <= %d, 64..1024 threads in whole "
            "waves, (kb, stages) one of (7,1) (7,2) (4,1) (4,2) (4,4) (2,4) (1,4) within the LDS)", op, MAX_GRID);
        return 0;
    }
    if (!chk(buf, off, bytes, op, "buf") || !need_batch(op) || !prep_in_r(buf, off, bytes, op)) return 0;
    uint32_t *sink = (uint32_t *)scratch((size_t)grid * 4, op);
    if (!sink) return 0;
    const uint8_t *p = buf->dev + off;
    int64_t n16 = (int64_t)(bytes / 16);
    int32_t kb32 = kb, s32 = stages;
    void *args[] = { &p, &n16, &sink, &kb32, &s32 };
    return launch_lds(K_READ_PROBE_DMA, grid, threads, lds, args, op);
}

int sepia_gpu_softmax(SepiaGpuBuf *x, SepiaGpuBuf *y, int64_t rows, int64_t n) {
    const char *op = "softmax";
    if (!x || !y || rows <= 0 || n <= 0 || rows > MAX_GRID) {
        LOG("%s: invalid arguments", op);
        return 0;
    }
    size_t nb = (size_t)rows * (size_t)n * 4;
    if (!chk(x, 0, nb, op, "x") || !chk(y, 0, nb, op, "y")) return 0;
    if (!need_batch(op) || !prep_in(x, op) || !prep_out(y, op)) return 0;
    void *args[] = { &x->dev, &y->dev, &n };
    return launch(K_SOFTMAX, (unsigned)rows, 256, args, op);
}

static int do_sconv(const char *op, SepiaGpuBuf *w, size_t w_off, SepiaGpuBuf *hist, SepiaGpuBuf *in,
                    SepiaGpuBuf *out, int64_t C, int64_t K, int64_t T) {
    if (!w || !hist || !in || !out || C <= 0 || K <= 0 || T <= 0 || C > 0x7FFFFFFF || K > 0x7FFFFFFF ||
        T > 0x7FFFFFFF || (C * T + 255) / 256 > MAX_GRID) {
        LOG("%s: invalid arguments", op);
        return 0;
    }
    size_t cs = (size_t)C * 4;
    if (!f32_off_ok(w_off, op, "w") || !chk(w, w_off, cs * (size_t)K, op, "w") ||
        !chk(hist, 0, cs * (size_t)(K - 1), op, "hist") || !chk(in, 0, cs * (size_t)T, op, "in") ||
        !chk(out, 0, cs * (size_t)T, op, "out"))
        return 0;
    if (!need_batch(op) || !prep_in_r(w, w_off, cs * (size_t)K, op) || !prep_in(hist, op) || !prep_in(in, op) ||
        !prep_out(out, op))
        return 0;
    const float *wp = (const float *)(w->dev + w_off);
    int32_t c = (int32_t)C, k = (int32_t)K, t = (int32_t)T;
    void *args[] = { &wp, &hist->dev, &in->dev, &out->dev, &c, &k, &t };
    return launch(K_SCONV, blocks_for(C * T, 256), 256, args, op);
}

int sepia_gpu_sconv(SepiaGpuBuf *w, SepiaGpuBuf *hist, SepiaGpuBuf *in, SepiaGpuBuf *out, int64_t C, int64_t K,
                    int64_t T) {
    return do_sconv("sconv", w, 0, hist, in, out, C, K, T);
}

int sepia_gpu_sconv_off(SepiaGpuBuf *w, size_t w_off, SepiaGpuBuf *hist, SepiaGpuBuf *in, SepiaGpuBuf *out,
                        int64_t C, int64_t K, int64_t T) {
    return do_sconv("sconv_off", w, w_off, hist, in, out, C, K, T);
}

int sepia_gpu_sconv_hist_roll(SepiaGpuBuf *hist, SepiaGpuBuf *in, int64_t C, int64_t K, int64_t T) {
    const char *op = "sconv_hist_roll";
    if (!hist || !in || C <= 0 || K <= 0 || T <= 0 || C > 0x7FFFFFFF || T > 0x7FFFFFFF) {
        LOG("%s: invalid arguments", op);
        return 0;
    }
    int64_t km1 = K - 1;
    if (km1 > 15) {
        LOG("%s: K-1=%lld exceeds the supported maximum (15)", op, (long long)km1);
        return 0;
    }
    if (km1 == 0) return 1;
    if (!chk(hist, 0, (size_t)km1 * (size_t)C * 4, op, "hist") || !chk(in, 0, (size_t)T * (size_t)C * 4, op, "in"))
        return 0;
    if (!need_batch(op) || !prep_in(in, op) || !prep_out(hist, op)) return 0;
    int32_t c = (int32_t)C, k = (int32_t)km1, t = (int32_t)T;
    void *args[] = { &hist->dev, &in->dev, &c, &k, &t };
    return launch(K_SCONV_HIST, blocks_for(C, 256), 256, args, op);
}

/* ---------------------------------------------------------- attention --- */
/* Relative-position projection (reference src/sepia_gpu.h:209, :253):
 * rel_logits [T, H, rel_extent] = r_vec [T, H, d_rel] x rel_proj [d_rel,
 * rel_extent], f32 (kernels/attn.h). */
static int do_rel_project(const char *op, SepiaGpuBuf *r_vec, SepiaGpuBuf *rel_proj, size_t rp_off,
                          SepiaGpuBuf *rel_logits, int64_t T, int64_t H, int64_t d_rel, int64_t rel_extent) {
    if (!r_vec || !rel_proj || !rel_logits || T < 1 || H < 1 || d_rel < 1 || rel_extent < 1 ||
        d_rel > 0x7FFFFFFF || rel_extent > 0x7FFFFFFF || (rel_extent + 255) / 256 > MAX_GRID ||
        (T * H + 7) / 8 > 65535) {
        LOG("%s: invalid arguments", op);
        return 0;
    }
    const size_t th = (size_t)T * (size_t)H;
    if (!f32_off_ok(rp_off, op, "rel_proj") || !chk(r_vec, 0, th * (size_t)d_rel * 4, op, "r_vec") ||
        !chk(rel_proj, rp_off, (size_t)d_rel * (size_t)rel_extent * 4, op, "rel_proj") ||
        !chk(rel_logits, 0, th * (size_t)rel_extent * 4, op, "rel_logits"))
        return 0;
    if (!need_batch(op) || !prep_in_r(r_vec, 0, th * (size_t)d_rel * 4, op) ||
        !prep_in_r(rel_proj, rp_off, (size_t)d_rel * (size_t)rel_extent * 4, op) || !prep_out(rel_logits, op))
        return 0;
    const float *rp = (const float *)(rel_proj->dev + rp_off);
    int64_t TH = (int64_t)th;
    int32_t dr = (int32_t)d_rel, R = (int32_t)rel_extent;
    void *args[] = { &r_vec->dev, &rp, &rel_logits->dev, &TH, &dr, &R };
    return launch2(K_REL_PROJECT, (unsigned)((rel_extent + 255) / 256), (unsigned)((TH + 7) / 8), 256, 0, args, op);
}

int sepia_gpu_rel_project(SepiaGpuBuf *r_vec, SepiaGpuBuf *rel_proj, SepiaGpuBuf *rel_logits, int64_t T, int64_t H,
                          int64_t d_rel, int64_t rel_extent) {
    return do_rel_project("rel_project", r_vec, rel_proj, 0, rel_logits, T, H, d_rel, rel_extent);
}

int sepia_gpu_rel_project_off(SepiaGpuBuf *r_vec, SepiaGpuBuf *rel_proj, size_t rel_proj_off,
                              SepiaGpuBuf *rel_logits, int64_t T, int64_t H, int64_t d_rel, int64_t rel_extent) {
    return do_rel_project("rel_project_off", r_vec, rel_proj, rel_proj_off, rel_logits, T, H, d_rel, rel_extent);
}

/* Banded attention (reference src/sepia_gpu.h:226; CPU semantics
 * src/sepia.c:1211-1247): per token a launch of span workgroups per kv head
 * writes per-head partials to scratch, a second launch folds them. Tokens go
 * ATT_TB a launch pair, their kv bounds and tau in the kernel arguments (the
 * caller's host arrays are read here and need not outlive the call). Mirrors
 * struct AttnTok in kernels/attn.h. */
#define ATT_TB 64
#define ATT_CH 128
typedef struct {
    int32_t lo[ATT_TB], hi[ATT_TB];
    float tau[ATT_TB];
} AttnTok;

int sepia_gpu_banded_attn(SepiaGpuBuf *q, SepiaGpuBuf *k, SepiaGpuBuf *v, SepiaGpuBuf *rel_logits,
                          SepiaGpuBuf *attn_out, const int64_t *kv_lo, const int64_t *kv_hi, const float *tau,
                          int64_t T, int64_t H, int64_t Hkv, int64_t Dh, int64_t rel_extent, int64_t q_pos_base,
                          int64_t kv_dim, float inv_head_dim) {
    const char *op = "banded_attn";
    if (!q || !k || !v || !rel_logits || !attn_out || !kv_lo || !kv_hi || !tau || T < 1 || H < 1 || Hkv < 1 ||
        H % Hkv || H / Hkv > 16 || rel_extent < 1 || rel_extent > 0x7FFFFFFF || q_pos_base < 0 ||
        kv_dim < Hkv * Dh || H > 65535 || Hkv > 65535) {
        LOG("%s: invalid arguments", op);
        return 0;
    }
    if (Dh < 4 || Dh > 128 || Dh % 4) {
        LOG("%s: head dim %lld not supported (a multiple of 4 up to 128)", op, (long long)Dh);
        return 0;
    }
    int64_t max_hi = 0, max_n = 0;
    for (int64_t t = 0; t < T; t++) {
        if (kv_lo[t] < 0 || kv_hi[t] < kv_lo[t] || kv_hi[t] > q_pos_base + t || kv_hi[t] > 0x7FFFFFFF) {
            LOG("%s: token %lld: kv range [%lld, %lld] outside [0, q_pos %lld]", op, (long long)t,
                (long long)kv_lo[t], (long long)kv_hi[t], (long long)(q_pos_base + t));
            return 0;
        }
        if (kv_hi[t] > max_hi) max_hi = kv_hi[t];
        if (kv_hi[t] - kv_lo[t] + 1 > max_n) max_n = kv_hi[t] - kv_lo[t] + 1;
    }
    if (kv_dim % 4) {
        LOG("%s: kv_dim %lld is not a multiple of 4 (k and v rows are read 16 bytes at a time)", op,
            (long long)kv_dim);
        return 0;
    }
    const size_t qb = (size_t)T * (size_t)H * (size_t)Dh * 4;
    const size_t kvb = ((size_t)max_hi * (size_t)kv_dim + (size_t)Hkv * (size_t)Dh) * 4;
    const size_t rlb = (size_t)T * (size_t)H * (size_t)rel_extent * 4;
    if (!chk(q, 0, qb, op, "q") || !chk(k, 0, kvb, op, "k") || !chk(v, 0, kvb, op, "v") ||
        !chk(rel_logits, 0, rlb, op, "rel_logits") || !chk(attn_out, 0, qb, op, "attn_out"))
        return 0;
    /* spans: enough workgroups to cover the CUs, each span whole steps */
    const int64_t tb = T < ATT_TB ? T : ATT_TB;
    int64_t nsplit = (1024 + Hkv * tb - 1) / (Hkv * tb);
    const int64_t steps = (max_n + ATT_CH - 1) / ATT_CH;
    if (nsplit > steps) nsplit = steps;
    if (nsplit < 1) nsplit = 1;
    int64_t span = ((steps + nsplit - 1) / nsplit) * ATT_CH;
    nsplit = (max_n + span - 1) / span;
    if (nsplit > 65535 || span > 0x7FFFFFFF) {
        LOG("%s: kv range too long", op);
        return 0;
    }
    if (!need_batch(op)) return 0;
    const size_t part_bytes = (size_t)tb * (size_t)H * (size_t)nsplit * (size_t)(Dh + 2) * 8;
    double *part = (double *)scratch(part_bytes, op);
    if (!part) return 0;
    if (!prep_in_r(q, 0, qb, op) || !prep_in_r(k, 0, kvb, op) || !prep_in_r(v, 0, kvb, op) ||
        !prep_in_r(rel_logits, 0, rlb, op) || !prep_out(attn_out, op))
        return 0;
    int32_t H32 = (int32_t)H, Hkv32 = (int32_t)Hkv, Dh32 = (int32_t)Dh, R32 = (int32_t)rel_extent;
    int32_t ns32 = (int32_t)nsplit, span32 = (int32_t)span;
    int64_t qpb = q_pos_base, kvd = kv_dim;
    float ihd = inv_head_dim;
    for (int64_t t0 = 0; t0 < T; t0 += ATT_TB) {
        const int64_t nt = T - t0 < ATT_TB ? T - t0 : ATT_TB;
        AttnTok tok;
        memset(&tok, 0, sizeof tok);
        for (int64_t i = 0; i < nt; i++) {
            tok.lo[i] = (int32_t)kv_lo[t0 + i];
            tok.hi[i] = (int32_t)kv_hi[t0 + i];
            tok.tau[i] = tau[t0 + i];
        }
        int32_t t032 = (int32_t)t0;
        void *a_p[] = { &q->dev, &k->dev, &v->dev, &rel_logits->dev, &tok, &t032, &H32, &Hkv32, &Dh32, &R32, &qpb,
                        &kvd, &ihd, &ns32, &span32, &part };
        if (!launch3(K_ATTN_PARTIAL, (unsigned)nsplit, (unsigned)Hkv, (unsigned)nt, 256, 0, a_p, op)) return 0;
        void *a_c[] = { &part, &tok, &t032, &H32, &Dh32, &ns32, &span32, &attn_out->dev };
        if (!launch2(K_ATTN_COMBINE, (unsigned)H, (unsigned)nt, 128, 0, a_c, op)) return 0;
    }
    return 1;
}

int sepia_gpu_selftest_touch(SepiaGpuBuf *buf, size_t n_floats) {
    const char *op = "selftest_touch";
    if (!need_init(op)) return 0;
    if (!buf || n_floats == 0 || n_floats > (size_t)MAX_GRID * 256) {
        LOG("%s: invalid buf/n_floats", op);
        return 0;
    }
    if (!chk(buf, 0, n_floats * 4, op, "buf") || !sync_in(buf, op)) return 0;
    int64_t n = (int64_t)n_floats;
    void *args[] = { &buf->dev, &n };
    if (!launch(K_TOUCH, blocks_for(n, 256), 256, args, op)) return 0;
    hipError_t e = hipSuccess;
    if (buf->kind == BUF_SHARED) e = hipMemcpyAsync(buf->host, buf->dev, buf->len, hipMemcpyDeviceToHost, g_stream);
    hipError_t s = hipStreamSynchronize(g_stream);
    if (e == hipSuccess) e = s;
    if (e != hipSuccess) {
        LOG("%s: failed: %s", op, hipGetErrorString(e));
        return 0;
    }
    return 1;
}

/* --------------------------------------------------------- quantized ---- */
/* Tuning switches (sepia_hip_set_option): "tile" 0 forces the generic
 * one-wave-per-row kernels; "tile_t" 1..3 forces the row steps per
 * workgroup of the tile kernels (0 = automatic). */
int sepia_hip_set_option(const char *name, int value) {
    if (!name) {
        LOG("set_option: NULL name");
        return 0;
    }
    if (strcmp(name, "tile") == 0 && (value == 0 || value == 1)) {
        g_opt_tile = value;
        return 1;
    }
    if (strcmp(name, "mq") == 0 && (value == 0 || value == 1)) {
        g_opt_mq = value;
        return 1;
    }
    if (strcmp(name, "wait_ticks") == 0 && value >= 0) {
        /* the kernels' spin-wait bound in s_memrealtime ticks (100 MHz); 0
         * restores the default of 2 s. Tests use a tiny bound to make the
         * waits expire and check that the batch reports it. */
        if (!need_init("set_option")) return 0;
        hipStreamSynchronize(g_stream);
        return set_wait_ticks(value ? (uint64_t)value : WAIT_TICKS_DEFAULT);
    }
    if (strcmp(name, "mq_x") == 0 && value >= 0 && value <= 4) {
        g_opt_mq_x = value;
        return 1;
    }
    if (strcmp(name, "pf_h") == 0 && (value == 0 || value == 1)) {
        g_opt_pf_h = value;
        return 1;
    }
    if (strcmp(name, "pf_q") == 0 && (value == 0 || value == 1)) {
        g_opt_pf_q = value;
        return 1;
    }
    if (strcmp(name, "pf_route_m") == 0 && (value == 0 || value == 1)) {
        g_opt_pf_route_m = value;
        return 1;
    }
    if (strcmp(name, "mq_gufac") == 0 && value >= 25 && value <= 400) {
        g_opt_mq_gufac = value;
        return 1;
    }
    if (strcmp(name, "mq_dnfac") == 0 && value >= 25 && value <= 400) {
        g_opt_mq_dnfac = value;
        return 1;
    }
    if (strcmp(name, "mq_rdelay") == 0 && value >= 0 && value <= 4096) {
        g_opt_mq_rdelay = value;
        return 1;
    }
    if (strcmp(name, "mq_scope") == 0 && value >= 0 && value <= 3) {
        g_opt_mq_scope = value;
        return 1;
    }
    if (strcmp(name, "mq_p") == 0 && value >= 0 && value <= 16) {
        g_opt_mq_p = value;
        return 1;
    }
    if (strcmp(name, "mq_c") == 0 && value >= 0 && value <= 16) {
        g_opt_mq_c = value;
        return 1;
    }
    if (strcmp(name, "mq_s") == 0 && value >= 0 && value <= 4) {
        g_opt_mq_s = value;
        return 1;
    }
    if (strcmp(name, "tile_t") == 0 && value >= 0 && value <= TILE_TMAX) {
        g_opt_tile_t = value;
        return 1;
    }
    LOG("set_option: unknown option %s=%d", name, value);
    return 0;
}

/* Matrix-core kernels (kernels/mq.h). x (or h) is staged once per
 * workgroup as XQ digit planes in LDS (4 bytes per column) behind a
 * 768-byte zero area; then come the items' partial row sums and one LDS
 * ring per wave. An item is 16 rows of one matrix; a wave step is 16 rows x
 * 4 blocks ("quad"), fetched by LDS DMA as Wp 16-byte words per lane (Q2_K
 * and Q3_K 7, Q4_K 9). nw = C * P waves: P parts split each item's quads, C
 * items run side by side; every wave's ring holds S = min(4, ring / Wp KB)
 * steps in flight. */
#define MQ_CUS 256                  /* MI355X compute units */
#define MQ_ZERO 768
typedef struct {
    int32_t P, ring, xraw, orings, conv, nw;   /* as struct MqGeo in kernels/mq.h */
    int32_t C, S, step;                        /* items side by side, ring stages, workgroup stride of the items */
    uint32_t mP, mC, mstep;                    /* mq_recip of P, C and step */
} MqGeo;
/* m with floor(n / d) = (n * m) >> 31 for every n < 2^31 / d (mq_div in
 * kernels/mq.h): the kernels divide by the launch's P, C and stride this
 * way instead of running a division sequence in every wave. */
static uint32_t mq_recip(int64_t d) { return (uint32_t)(((1ull << 31) + (uint64_t)d - 1) / (uint64_t)d); }
static void mq_geo_step(MqGeo *g, int64_t step) {
    g->step = (int32_t)step;
    g->mstep = mq_recip(step);
}
/* In-kernel selection by the gate/up launch (struct MqRoute in
 * kernels/mq.h); logits NULL: the experts come from sel_idx. */
typedef struct {
    const float *logits;
    const float *bias;
    int32_t n_routed, n_shared;
    float route_scale, global_scale;
    int32_t *idx_out;
    float *w_out;
} MqRoute;
#define MQ_SEL_BYTES 528            /* the gate/up kernel's selection area in LDS (MQ_SEL_BYTES in kernels/mq.h) */
#define MQ_XDMA_GAIN 40             /* mq_geo: cost units the vector's LDS DMA saves (measured ~2 us a launch) */
#define MQ_CONV_GAIN 60             /* mq_geo: cost units converter waves save (XQ off the weights' path); by
                                     * default only for the IQ formats, where they measured faster (C4 IQ3_XXS
                                     * 12.2 -> 11.2 us); the K-quants' stepping waves need all 16 */
#define MQ_XQ_SEGS_PER_WAVE 128     /* segments a converter wave turns into XQ at most (MQ_XQP passes of 16) */
#define MQ_SCONV_GAIN 60            /* mq_geo: cost units the first stepping waves save by converting the vector
                                     * before their own weight prologue (vector mode 3) */
static size_t mq_xq_bytes(int64_t n) { return (size_t)(n / 256) * 832 + 3 * (size_t)(n / 16) * 4; }
/* matrix-core format codes (kernels/mq.h decoders, matvec and expert FFN):
 * 0..2 Q2_K, Q3_K, Q4_K; 3..4 IQ2_XS, IQ3_XXS; 5..8 Q5_K, Q6_K, IQ4_XS, Q8_0 */
static int mq_code(int t) {
    switch (t) {
    case SEPIA_T_Q2_K: return 0;
    case SEPIA_T_Q3_K: return 1;
    case 12: return 2;
    case 17: return 3;
    case 18: return 4;
    case 13: return 5;
    case 14: return 6;
    case 23: return 7;
    case 8: return 8;
    default: return -1;
    }
}
#define MQ_FORMATS 9
static const int k_mq_words[MQ_FORMATS] = { 7, 7, 9, 5, 7, 11, 15, 9, 17 };   /* padded words per lane (MQ<T>::Wp) */
static const size_t k_mq_table[MQ_FORMATS] = { 0, 0, 0, 5120, 3072, 0, 0, 0, 0 };   /* LDS codebook and sign selectors (MQ<T>::table_bytes) */
/* Converter waves are planned in the matvecs of every format but Q2_K.
 * Interleaved on one box, kernel us at 4096^2 / 6144^2, planner without
 * them -> with them: Q3_K 6.22 -> 5.53 / 9.96 -> 8.26, Q4_K 6.55 -> 5.61 /
 * 9.84 -> 8.50, Q5_K 6.93 -> 6.37 / 11.30 -> 9.40, Q6_K 7.21 -> 7.00 /
 * 12.40 -> 11.83, Q8_0 7.34 -> 6.63 / 12.16 -> 10.90, IQ4_XS 7.06 -> 6.30 /
 * 11.62 -> 9.50 (IQ2_XS and IQ3_XXS already had them); Q2_K 4.63 -> 5.08
 * / 7.95 -> 7.08, its light decode needing all 16 waves stepping at the
 * smaller size. */
static const int k_mq_conv[MQ_FORMATS] = { 0, 1, 1, 1, 1, 1, 1, 1, 1 };
/* Relative time per weight byte of the matrix-core decoders (percent; the
 * K-quants Q4_K, Q5_K, Q6_K = 100), used to split an FFN launch's
 * workgroups between routed and shared experts. Measured on the MoE decode
 * layer: byte-balanced Q2_K against Q4_K is best, Q3_K against Q4_K at 115,
 * IQ2_XS against Q5_K at 160 (with the sign masks from LDS the layer is
 * within 0.5 us from 130 to 230, slower below) and IQ3_XXS against Q6_K at
 * 145 (100-190 swept). IQ4_XS and Q8_0 are estimates. */
static const int k_mq_cost[MQ_FORMATS] = { 100, 115, 100, 160, 145, 100, 100, 120, 80 };
/* A row of n_blocks format blocks in the matrix-core kernels' 256-column
 * blocks (Q8_0: super-blocks of 8 of its 32-column blocks); -1 if it does
 * not divide. */
static int64_t mq_nb(int type, int64_t n_blocks) {
    if (type == 8) return n_blocks % 8 ? -1 : n_blocks / 8;
    return n_blocks;
}
static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

/* Geometry for workgroups of n_items items of nq quads; mc is the format
 * most items use, wmax the most words of any format the workgroup may run.
 * LDS = o_raw = align256(fixed + 64 * n_items * P), then (if the vector of
 * raw_bytes goes by LDS DMA) the raw vector, or (with converter waves) 16
 * bytes of control words, then nw rings at orings; the rings take the rest
 * of the LDS (each at least one step of wmax words). Converter waves come
 * on top of the nw stepping waves: enough for the vector (at most
 * MQ_XQ_SEGS_PER_WAVE segments each), up to 4 where the 16 allow.
 * Chooses the fewest steps per wave of format mc, counting a one-stage ring
 * with several steps as 1.6 steps each (its loads do not overlap its
 * compute) and crediting the vector's DMA or converter waves, then the most
 * steps in flight, then the most waves. Returns 0 when nothing fits. */
static int mq_geo(int mc, int wmax, int64_t n_items, int64_t nq, size_t fixed, size_t raw_bytes, int allow_conv,
                  unsigned *threads, MqGeo *geo, size_t *lds) {
    const size_t w1 = (size_t)k_mq_words[mc] * 1024, wm = (size_t)wmax * 1024;
    int64_t best_cost = 0, best_fl = 0;
    int best_nw = 0, found = 0;
    /* vector modes: 0 from global memory, 1 by LDS DMA into a raw copy, 2 by
     * converter waves (DMA into the XQ place, converted there), 3 the same
     * by the first stepping waves before they issue their weights; 1..3
     * need the vector's size (raw_bytes) */
    const int64_t segs = (int64_t)raw_bytes / 64, cv_need = (segs + MQ_XQ_SEGS_PER_WAVE - 1) / MQ_XQ_SEGS_PER_WAVE;
    /* a forced mode the launch cannot take (converter waves for the FFN
     * launches) leaves the choice to the planner */
    const int ovr = !g_opt_mq_scope || g_opt_mq_scope == g_mq_kind;
    const int opt_p = ovr ? g_opt_mq_p : 0, opt_c = ovr ? g_opt_mq_c : 0, opt_s = ovr ? g_opt_mq_s : 0;
    /* mode 3 exists only in the FFN gate/up kernel */
    const int forced = !ovr || (g_opt_mq_x >= 3 && !allow_conv) || (g_opt_mq_x == 4 && g_mq_kind != 2) ? 0 : g_opt_mq_x;
    for (int mode = 0; mode <= (raw_bytes > 0 ? (allow_conv ? 3 : 1) : 0); mode++) {
        /* converter waves by default only in the matvecs of the formats that
         * gain from them; the FFN launches measured slower with them (the
         * IQ3_XXS down of a real-format layer 34.9 vs 31.1 us) */
        if (raw_bytes > 0 && (forced ? forced != mode + 1 : ((mode == 2 && !(k_mq_conv[mc] && g_mq_kind == 1)) ||
                                                            (mode == 3 && !g_mq_sconv))))
            continue;
        if (mode == 3 && g_mq_kind != 2) continue;
        for (int P = 1; P <= 16 && P <= nq; P++) {
            if (opt_p && P != opt_p) continue;
            for (int C = 1; C * P <= 16 && C <= n_items; C++) {
                if (opt_c && C != opt_c) continue;
                const int nw = C * P;
                int cv = 0;
                if (mode == 2) {
                    if (nw + cv_need > 16) continue;
                    cv = 16 - nw < 4 ? 16 - nw : 4;
                    if (cv < cv_need) cv = (int)cv_need;
                }
                if (mode == 3 && nw < cv_need) continue;
                const int64_t spw = ((n_items + C - 1) / C) * ((nq + P - 1) / P);
                const size_t o_raw = align256(fixed + (size_t)n_items * P * 64);
                const size_t base = mode == 1 ? align256(o_raw + raw_bytes) : mode >= 2 ? align256(o_raw + 16) : o_raw;
                if (base + (size_t)nw * wm > g_lds_max) continue;
                size_t ring = ((g_lds_max - base) / (size_t)nw) & ~(size_t)1023;
                if (ring > 4 * wm) ring = 4 * wm;
                if (opt_s) {
                    ring = (size_t)opt_s * wm;
                    if (base + (size_t)nw * ring > g_lds_max) continue;
                }
                int64_t S = (int64_t)(ring / w1);
                if (S > 4) S = 4;
                if (S > spw) S = spw;
                /* the vector by DMA ahead of the weights saves about as
                 * much as MQ_XDMA_GAIN cost units, converter waves more */
                const int64_t cost = spw * ((S >= 2 || spw == 1) ? 10 : 16) -
                                     (mode == 1 ? MQ_XDMA_GAIN : mode == 2 ? MQ_CONV_GAIN : mode == 3 ? MQ_SCONV_GAIN : 0);
                const int64_t fl = (int64_t)nw * S;
                if (!found || cost < best_cost ||
                    (cost == best_cost && (fl > best_fl || (fl == best_fl && nw > best_nw)))) {
                    found = 1;
                    best_cost = cost;
                    best_fl = fl;
                    best_nw = nw;
                    geo->P = P;
                    geo->ring = (int32_t)ring;
                    geo->xraw = mode ? (int32_t)o_raw : 0;
                    geo->orings = (int32_t)base;
                    geo->conv = mode == 3 ? -(int32_t)cv_need : cv;
                    geo->nw = nw;
                    geo->C = C;
                    geo->S = (int32_t)(ring / w1 < 4 ? ring / w1 : 4);
                    geo->mP = mq_recip(P);
                    geo->mC = mq_recip(C);
                    mq_geo_step(geo, 1);
                    *threads = 64u * (unsigned)(nw + cv);
                    *lds = base + (size_t)nw * ring;
                }
            }
        }
    }
    return found;
}

/* Shapes the matrix-core kernels take: a format with a decoder, 4-byte
 * aligned rows of a multiple of 4 256-column blocks (nb, mq_nb), row
 * offsets within 32 bits. */
static int mq_shape_ok(int type, int64_t nb, int64_t rows, uintptr_t base, uint64_t row_bytes) {
    return g_opt_mq && mq_code(type) >= 0 && nb >= 4 && nb % 4 == 0 && base % 4 == 0 && row_bytes % 4 == 0 &&
           (uint64_t)rows * row_bytes < (1ull << 32);
}

/* n_blocks: the row's blocks of the format; the kernel takes mq_nb of it. */
static int mq_plan(int type, int64_t n_blocks, int64_t rows, uintptr_t base, uint64_t row_bytes, unsigned *threads,
                   size_t *lds, unsigned *grid, MqGeo *geo) {
    n_blocks = mq_nb(type, n_blocks);
    if (!mq_shape_ok(type, n_blocks, rows, base, row_bytes)) return -1;
    const int mc = mq_code(type);
    const int64_t tiles = (rows + 15) / 16;
    const int64_t per = (tiles + MQ_CUS - 1) / MQ_CUS;     /* row groups per workgroup */
    *grid = (unsigned)((tiles + per - 1) / per);
    g_mq_kind = 1;
    if (!mq_geo(mc, k_mq_words[mc], per, n_blocks / 4, MQ_ZERO + mq_xq_bytes(256 * n_blocks) + k_mq_table[mc],
                (size_t)1024 * n_blocks, 1, threads, geo, lds))
        return -1;
    mq_geo_step(geo, *grid);
    return K_MQ_MV + mc;
}

/* 1 if the tile matvec runs this matrix: the format has a tile decoder, the
 * base is aligned as the decoder loads it and the row length fits. */
static int tile_plan(const TypeInfo *ti, int64_t n_blocks, uintptr_t base, int64_t rows, TileGeo *g) {
    return g_opt_tile && ti->k_tile >= 0 && base % (uintptr_t)ti->align == 0 && tile_geo(n_blocks, rows, 1, g);
}

int sepia_gpu_matvec_q(int ggml_type, SepiaGpuBuf *w, size_t w_off, SepiaGpuBuf *x, SepiaGpuBuf *y,
                       int64_t out_dim, int64_t in_dim) {
    const char *op = "matvec_q";
    if (!w || !x || !y || out_dim <= 0 || in_dim <= 0 || (out_dim + 3) / 4 > MAX_GRID) {
        LOG("%s: invalid arguments", op);
        return 0;
    }
    const TypeInfo *ti = type_info(ggml_type);
    if (!ti || ti->k_mv < 0) {
        LOG("%s: no GPU kernel for ggml type %d", op, ggml_type);
        return 0;
    }
    if (in_dim % ti->elems) {
        LOG("%s: in_dim %lld not a multiple of block size %lld (type %d)", op, (long long)in_dim,
            (long long)ti->elems, ggml_type);
        return 0;
    }
    int64_t n_blocks = in_dim / ti->elems;
    uint64_t row_bytes = (uint64_t)n_blocks * ti->bytes;
    if (!chk(w, w_off, (size_t)out_dim * row_bytes, op, "w") || !chk(x, 0, (size_t)in_dim * 4, op, "x") ||
        !chk(y, 0, (size_t)out_dim * 4, op, "y"))
        return 0;
    if (!need_batch(op) || !prep_in_r(w, w_off, (size_t)out_dim * row_bytes, op) || !prep_in(x, op) ||
        !prep_out(y, op))
        return 0;
    const uint8_t *wp = w->dev + w_off;
    unsigned mq_threads, mq_grid;
    size_t mq_lds;
    MqGeo mgeo;
    const int kmq = mq_plan(ggml_type, n_blocks, out_dim, (uintptr_t)wp, row_bytes, &mq_threads, &mq_lds, &mq_grid,
                            &mgeo);
    if (kmq >= 0) {
        int32_t nb32 = (int32_t)mq_nb(ggml_type, n_blocks);
        void *args[] = { &wp, &row_bytes, &out_dim, &nb32, &x->dev, &y->dev, &mgeo };
        return launch_lds(kmq, mq_grid, mq_threads, mq_lds, args, op);
    }
    TileGeo geo;
    if (tile_plan(ti, n_blocks, (uintptr_t)wp, out_dim, &geo)) {
        int64_t n = in_dim;
        void *args[] = { &wp, &row_bytes, &out_dim, &n, &geo, &x->dev, &y->dev };
        return launch_lds(ti->k_tile, (unsigned)geo.tiles, TILE_NT, tile_lds(n, &geo, 1), args, op);
    }
    void *args[] = { &wp, &row_bytes, &n_blocks, &x->dev, &y->dev, &out_dim };
    return launch(ti->k_mv, blocks_for(out_dim, 4), 256, args, op);
}

int sepia_gpu_dequant_rows(int ggml_type, SepiaGpuBuf *raw, size_t raw_off, SepiaGpuBuf *out, int64_t n) {
    const char *op = "dequant_rows";
    if (!raw || !out || n <= 0) {
        LOG("%s: invalid arguments", op);
        return 0;
    }
    const TypeInfo *ti = type_info(ggml_type);
    if (!ti) {
        LOG("%s: no GPU kernel for ggml type %d", op, ggml_type);
        return 0;
    }
    if (n % ti->elems) {
        LOG("%s: n %lld not a multiple of block size %lld (type %d)", op, (long long)n, (long long)ti->elems,
            ggml_type);
        return 0;
    }
    int64_t nb = n / ti->elems;
    int64_t threads = nb * ti->parts;
    if ((threads + 255) / 256 > MAX_GRID) {
        LOG("%s: n too large", op);
        return 0;
    }
    if (!chk(raw, raw_off, (size_t)nb * ti->bytes, op, "raw") || !chk(out, 0, (size_t)n * 4, op, "out")) return 0;
    if (!need_batch(op) || !prep_in_r(raw, raw_off, (size_t)nb * ti->bytes, op) || !prep_out(out, op)) return 0;
    const uint8_t *rp = raw->dev + raw_off;
    void *args[] = { &rp, &out->dev, &threads };
    return launch(ti->k_dq, blocks_for(threads, 256), 256, args, op);
}

int sepia_hip_set_iq2xxs_grid(const uint64_t *grid256) {
    const char *op = "set_iq2xxs_grid";
    if (!need_init(op)) return 0;
    if (!grid256) {
        LOG("%s: NULL table", op);
        return 0;
    }
    hipDeviceptr_t p;
    size_t sz = 0;
    hipError_t e = hipModuleGetGlobal(&p, &sz, g_module, "g_iq2xxs_grid");
    if (e == hipSuccess && sz != 256 * sizeof(uint64_t)) e = hipErrorInvalidValue;
    if (e == hipSuccess) e = hipMemcpyHtoDAsync(p, (void *)grid256, sz, g_stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
    if (e != hipSuccess) {
        LOG("%s: failed: %s", op, hipGetErrorString(e));
        return 0;
    }
    g_have_iq2xxs = 1;
    return 1;
}

/* ------------------------------------------------------------- synth ---- */
int sepia_hip_synth_blocks(int ggml_type, SepiaGpuBuf *buf, size_t off, int64_t n_blocks, uint64_t seed, float lo,
                           float hi) {
    const char *op = "synth_blocks";
    const TypeInfo *ti = NULL;
    for (size_t i = 0; i < sizeof k_types / sizeof k_types[0]; i++)
        if (k_types[i].type == ggml_type) ti = &k_types[i];
    if (!buf || n_blocks <= 0 || !ti || off % 4) {
        LOG("%s: invalid arguments", op);
        return 0;
    }
    size_t nbytes = (size_t)n_blocks * ti->bytes;
    if (!chk(buf, off, nbytes, op, "buf")) return 0;
    if (!need_batch(op) || !prep_out(buf, op)) return 0;
    uint8_t *p = buf->dev + off;
    uint64_t n = nbytes;
    void *a1[] = { &p, &n, &seed };
    unsigned grid = blocks_for((int64_t)(nbytes / 4) + 1, 256);
    if (grid > 16384) grid = 16384;
    if (!launch(K_SYNTH_FILL, grid, 256, a1, op)) return 0;
    for (int f = 0; f < 2; f++) {
        if (ti->f16_off[f] < 0) continue;
        uint64_t nbk = (uint64_t)n_blocks;
        uint32_t bb = (uint32_t)ti->bytes, fo = (uint32_t)ti->f16_off[f];
        uint64_t s = seed * 31u + (uint64_t)f + 1u;
        void *a2[] = { &p, &nbk, &bb, &fo, &s, &lo, &hi };
        unsigned g2 = blocks_for(n_blocks, 256);
        if (g2 > 16384) g2 = 16384;
        if (!launch(K_SYNTH_F16, g2, 256, a2, op)) return 0;
    }
    return 1;
}

/* --------------------------------------------------------------- MoE ---- */
#define RT_THREADS 512   /* threads per router workgroup (RT_NT in kernels/moe.h) */
#define PH_WAVES 16      /* waves of an f16 projection workgroup (kernels/prefill_h.h) */
/* Mirrors struct MoeProj in kernels/moe.h field for field. */
typedef struct {
    const uint8_t *base;
    uint64_t stride;
    uint64_t row_bytes;
    int64_t n_blocks;
    int32_t type;
    int32_t pad;
} MoeProj;

static int moe_proj(const char *op, const char *what, const SepiaExpertTensor *t, int n_experts, int64_t rows,
                    int64_t cols, MoeProj *out) {
    const TypeInfo *ti = type_info(t->ggml_type);
    if (!ti || ti->k_mv < 0) {
        LOG("%s: %s: no GPU kernel for ggml type %d", op, what, t->ggml_type);
        return 0;
    }
    if (cols % ti->elems) {
        LOG("%s: %s: row length %lld not a multiple of block size %lld", op, what, (long long)cols,
            (long long)ti->elems);
        return 0;
    }
    uint64_t rb = (uint64_t)(cols / ti->elems) * ti->bytes;
    size_t mat = (size_t)rows * rb;
    if (n_experts > 1 && t->stride < mat) {
        LOG("%s: %s: expert stride %zu is smaller than one matrix (%zu bytes)", op, what, t->stride, mat);
        return 0;
    }
    size_t span = (size_t)(n_experts - 1) * t->stride + mat;
    if (!chk(t->buf, t->off, span, op, what)) return 0;
    out->base = t->buf->dev + t->off;
    out->stride = t->stride;
    out->row_bytes = rb;
    out->n_blocks = cols / ti->elems;
    out->type = t->ggml_type;
    out->pad = 0;
    return 1;
}

/* Uploads what a layer's launches may read of its shared buffers: the router
 * rows and bias, x, and the spans of every expert stack (the selection
 * happens on the device, so any expert may be read). */
static int prep_layer(const SepiaMoeLayerDesc *L, const MoeProj *g, const MoeProj *u, const MoeProj *d,
                      const MoeProj *sg, const MoeProj *su, const MoeProj *sd, SepiaGpuBuf *x, size_t x_bytes,
                      const char *op) {
    const int64_t n_tot = L->n_routed + L->n_shared;
    if (!prep_in_r(L->router_w, L->router_w_off, (size_t)n_tot * (size_t)L->hidden * 4, op) ||
        !prep_in_r(L->router_bias, L->router_bias_off, (size_t)L->n_routed * 4, op) ||
        !prep_in_r(x, 0, x_bytes, op))
        return 0;
    const SepiaExpertTensor *ts[6] = { &L->gate, &L->up, &L->down, &L->s_gate, &L->s_up, &L->s_down };
    const MoeProj *ps[6] = { g, u, d, sg, su, sd };
    const int64_t rows[6] = { L->inter, L->inter, L->hidden, L->inter, L->inter, L->hidden };
    for (int i = 0; i < (L->n_shared > 0 ? 6 : 3); i++) {
        const int ne = i < 3 ? L->n_routed : L->n_shared;
        const size_t span = (size_t)(ne - 1) * ts[i]->stride + (size_t)rows[i] * ps[i]->row_bytes;
        if (!prep_in_r(ts[i]->buf, ts[i]->off, span, op)) return 0;
    }
    return 1;
}

/* Mirrors struct XpArgs in kernels/mv.h: x in digit-plane form. */
typedef struct {
    const int8_t *planes;
    const float *xs;
    const float *gs;
} XpArgs;

/* Scratch bytes for n_slots f32 activation vectors of length I. */
/* FFN scratch: h [n_slots][I] f32, then the down partial rows [n_slots][H]
 * f32 (matrix-core path with several slots). */
static size_t ffn_scratch_bytes(int n_slots, int64_t I, int64_t H) {
    return (size_t)n_slots * (size_t)I * 4 + (size_t)n_slots * (size_t)H * 4;
}

/* Index of a format among the tile kernels' {Q2_K, Q3_K, Q4_K}, -1 if none. */
static int tile_code(int t) { return t == SEPIA_T_Q2_K ? 0 : (t == SEPIA_T_Q3_K ? 1 : (t == 12 ? 2 : -1)); }

static int proj_aligned(const MoeProj *p) {
    const TypeInfo *ti = type_info(p->type);
    const uintptr_t a = ti ? (uintptr_t)ti->align : 1;
    return ((uintptr_t)p->base % a) == 0 && p->stride % a == 0 && p->row_bytes % a == 0;
}

/* Matrix-core FFN plan (kernels/mq.h): every projection in {Q2_K, Q3_K,
 * Q4_K} with a shape the kernels take, gate and up of one format per slot
 * kind, H and I multiples of 1024 (rows of whole quads), LDS within the
 * device limit. Both launches give each slot its own workgroups, wps_r per
 * routed slot and wps_s per shared one, in proportion to the slot's bytes
 * (about one workgroup per CU in all); a workgroup walks row groups j0,
 * j0 + wps, ... of its slot. Down workgroups combine the slots' partial rows
 * through per-row-group arrival counters (in the counter region, after the
 * router's). */
typedef struct {
    unsigned gu_threads, dn_threads, gu_grid, dn_grid;
    int32_t gu_wps_r, gu_wps_s, dn_wps_r, dn_wps_s;
    size_t gu_lds, dn_lds;
    MqGeo gu_geo_r, gu_geo_s, dn_geo_r, dn_geo_s;   /* routed and shared workgroups, each for its format */
} MqFfnPlan;
#define MQ_DN_CNT_OFF 64            /* first down arrival counter (u32 index in the counter region) */
/* p: n_blocks already in 256-column blocks (mq_nb). */
static int mq_proj_ok(const MoeProj *p, int64_t rows) {
    return mq_shape_ok(p->type, p->n_blocks, rows, (uintptr_t)p->base, p->row_bytes) && p->stride % 4 == 0;
}
/* Workgroups per slot for slots of byte weights br (routed) and bs (shared):
 * at most MQ_CUS in all (unless one per slot is already more), at most
 * `tiles` per slot, the bytes per workgroup as even as whole counts allow
 * (proportional shares rounded down, then one more workgroup at a time to
 * the kind with the most bytes per workgroup while it fits). */
static void mq_split(int32_t topk, int32_t n_shared, double br, double bs, int64_t tiles, double delay, double rfac,
                     int32_t *wr, int32_t *ws) {
    /* workgroups per routed slot (r) and per shared slot (sh) within MQ_CUS
     * that minimise the larger per-workgroup cost: a routed workgroup's
     * share of a row's bytes plus `delay` (its late start, in the same
     * units), a shared one's share */
    if (n_shared == 0) {
        int64_t r = MQ_CUS / (topk > 0 ? topk : 1);
        *wr = (int32_t)(r < 1 ? 1 : r > tiles ? tiles : r);
        *ws = 1;
        return;
    }
    double best = -1.0;
    int64_t br_best = 1, bs_best = 1;
    for (int64_t r = 1; r <= tiles && topk * r + n_shared <= MQ_CUS; r++) {
        int64_t sh = (MQ_CUS - topk * r) / n_shared;
        if (sh > tiles) sh = tiles;
        const double cr = rfac * br / (double)r + delay, cs = bs / (double)sh;
        const double c = cr > cs ? cr : cs;
        if (best < 0.0 || c < best) {
            best = c;
            br_best = r;
            bs_best = sh;
        }
    }
    *wr = (int32_t)br_best;
    *ws = (int32_t)bs_best;
}
/* One launch's two geometries (routed and shared workgroups) and the
 * launch's thread count and LDS (the larger of the two). */
static int mq_geo2(int mc_r, int mc_s, int has_s, int64_t items_r, int64_t items_s, int64_t nq, size_t fixed_r,
                   size_t fixed_s, size_t raw_r, size_t raw_s, unsigned *threads, MqGeo *geo_r, MqGeo *geo_s,
                   size_t *lds) {
    unsigned tr, ts = 0;
    size_t lr, ls = 0;
    if (!mq_geo(mc_r, k_mq_words[mc_r], items_r, nq, fixed_r, raw_r, 1, &tr, geo_r, &lr)) return 0;
    if (has_s) {
        if (!mq_geo(mc_s, k_mq_words[mc_s], items_s, nq, fixed_s, raw_s, 1, &ts, geo_s, &ls)) return 0;
    } else {
        *geo_s = *geo_r;
    }
    *threads = tr > ts ? tr : ts;
    *lds = lr > ls ? lr : ls;
    return 1;
}
/* route: the gate/up launch selects the experts itself; its routed
 * workgroups then convert x into its XQ place during the selection and
 * need no raw copy of it. */
static int mq_ffn_plan(const MoeProj *g, const MoeProj *u, const MoeProj *d, const MoeProj *sg, const MoeProj *su,
                       const MoeProj *sd, int32_t topk, int32_t n_shared, int64_t H, int64_t I, int route,
                       MqFfnPlan *pl) {
    if (!g_opt_mq || H % 1024 || I % 1024) return 0;
    const MoeProj *ps[6] = { g, u, d, sg, su, sd };
    const int64_t rows[6] = { I, I, H, I, I, H };
    for (int i = 0; i < (n_shared > 0 ? 6 : 3); i++)
        if (!mq_proj_ok(ps[i], rows[i])) return 0;
    if (g->type != u->type || (n_shared > 0 && sg->type != su->type)) return 0;
    const int64_t tiles_i = (I + 15) / 16, tiles_h = (H + 15) / 16;
    if (n_shared + topk > 1 && MQ_DN_CNT_OFF + tiles_h > CNT_BYTES / 4) return 0;
    mq_split(topk, n_shared, (double)g->row_bytes, n_shared > 0 ? (double)sg->row_bytes : 1.0, tiles_i,
             route ? 1024.0 * g_opt_mq_rdelay / (32.0 * (double)tiles_i) : 0.0,   /* 16 gate + 16 up rows a tile */
             0.01 * g_opt_mq_gufac * k_mq_cost[mq_code(g->type)] / k_mq_cost[mq_code(n_shared > 0 ? sg->type : g->type)],
             &pl->gu_wps_r, &pl->gu_wps_s);
    mq_split(topk, n_shared, (double)d->row_bytes, n_shared > 0 ? (double)sd->row_bytes : 1.0, tiles_h, 0.0,
             0.01 * g_opt_mq_dnfac * k_mq_cost[mq_code(d->type)] / k_mq_cost[mq_code(n_shared > 0 ? sd->type : d->type)],
             &pl->dn_wps_r, &pl->dn_wps_s);
    const int has_s = n_shared > 0;
    const int kg = mq_code(g->type), kd = mq_code(d->type);
    const int ksg = has_s ? mq_code(sg->type) : kg, ksd = has_s ? mq_code(sd->type) : kd;
    const int64_t nk_gr = (tiles_i + pl->gu_wps_r - 1) / pl->gu_wps_r, nk_gs = (tiles_i + pl->gu_wps_s - 1) / pl->gu_wps_s;
    const int64_t nk_dr = (tiles_h + pl->dn_wps_r - 1) / pl->dn_wps_r, nk_ds = (tiles_h + pl->dn_wps_s - 1) / pl->dn_wps_s;
    const size_t gu_fixed = MQ_ZERO + mq_xq_bytes(H) + MQ_SEL_BYTES;
    g_mq_kind = 2;
    g_mq_sconv = !route && n_shared == 0;
    const int gu_ok = mq_geo2(kg, ksg, has_s, 2 * nk_gr, 2 * nk_gs, H / 1024, gu_fixed + k_mq_table[kg],
                              gu_fixed + k_mq_table[ksg], route ? 0 : (size_t)H * 4, (size_t)H * 4, &pl->gu_threads,
                              &pl->gu_geo_r, &pl->gu_geo_s, &pl->gu_lds);
    g_mq_sconv = 0;
    if (!gu_ok) return 0;
    /* the routed workgroups' in-place conversion needs 3 waves besides the
     * selecting one (MQ_XQP passes of a quarter of their lanes) */
    if (route && (int64_t)pl->gu_threads - 64 < (H / 16 + MQ_XQ_SEGS_PER_WAVE - 1) / MQ_XQ_SEGS_PER_WAVE * 64)
        pl->gu_threads = (unsigned)(((H / 16 + MQ_XQ_SEGS_PER_WAVE - 1) / MQ_XQ_SEGS_PER_WAVE + 1) * 64);
    const size_t dn_fixed = MQ_ZERO + mq_xq_bytes(I) + 256;
    g_mq_kind = 3;
    if (!mq_geo2(kd, ksd, has_s, nk_dr, nk_ds, I / 1024, dn_fixed + k_mq_table[kd] + (size_t)nk_dr * 4,
                 dn_fixed + k_mq_table[ksd] + (size_t)nk_ds * 4, (size_t)I * 4, (size_t)I * 4, &pl->dn_threads,
                 &pl->dn_geo_r, &pl->dn_geo_s, &pl->dn_lds))
        return 0;
    mq_geo_step(&pl->gu_geo_r, pl->gu_wps_r);
    mq_geo_step(&pl->gu_geo_s, pl->gu_wps_s);
    mq_geo_step(&pl->dn_geo_r, pl->dn_wps_r);
    mq_geo_step(&pl->dn_geo_s, pl->dn_wps_s);
    pl->gu_grid = (unsigned)(topk * pl->gu_wps_r + n_shared * pl->gu_wps_s);
    pl->dn_grid = (unsigned)(topk * pl->dn_wps_r + n_shared * pl->dn_wps_s);
    return 1;
}

/* mq_ffn_plan on copies of the six projections (mp) whose n_blocks count
 * the matrix-core kernels' 256-column blocks. */
static int mq_ffn_prep(const MoeProj *g, const MoeProj *u, const MoeProj *d, const MoeProj *sg, const MoeProj *su,
                       const MoeProj *sd, int32_t topk, int32_t n_shared, int64_t H, int64_t I, int route, MoeProj mp[6],
                       MqFfnPlan *pl) {
    const MoeProj *ps[6] = { g, u, d, sg, su, sd };
    for (int i = 0; i < 6; i++) {
        mp[i] = *ps[i];
        mp[i].n_blocks = mq_nb(mp[i].type, mp[i].n_blocks);
    }
    return mq_ffn_plan(&mp[0], &mp[1], &mp[2], &mp[3], &mp[4], &mp[5], topk, n_shared, H, I, route, pl);
}

/* LDS of the prefill projection kernels (PF_LDS_BYTES in kernels/prefill.h):
 * the whole 160 KB (tiles, raw-block stages, row tables at the top). */
#define PF_LDS_BYTES 163840
/* Formats the prefill projections decode (kernels/prefill.h). */
static int pf_type_ok(int t) {
    return t == SEPIA_T_Q2_K || t == SEPIA_T_Q3_K || t == 12 || t == 13 || t == 14 || t == 17 || t == 18 || t == 23;
}
/* Formats of the int8 prefill projections (kernels/prefill_q.h): Q2_K, Q3_K, Q4_K. */
static int pf_type_int(int t) { return t == SEPIA_T_Q2_K || t == SEPIA_T_Q3_K || t == 12; }
/* Formats of the f16 prefill projections (kernels/prefill_h.h): the real
 * checkpoint's IQ2_XS, IQ3_XXS, IQ4_XS, Q5_K, Q6_K and Q8_0. */
static int pf_type_h(int t) { return t == 17 || t == 18 || t == 23 || t == 13 || t == 14 || t == 8; }
#define PH_REC 1056   /* bytes of a 256-column PH record (kernels/prefill_h.h) */

int sepia_gpu_moe_prefill(const SepiaMoeLayerDesc *L, int64_t n_tokens, SepiaGpuBuf *x, SepiaGpuBuf *y,
                          SepiaGpuBuf *route_out) {
    const char *op = "moe_prefill";
    if (!L || !x || !y || n_tokens < 1 || n_tokens > (1 << 20) || L->hidden <= 0 || L->inter <= 0 ||
        L->n_routed < 1 || L->n_routed > 1024 || L->n_shared < 0 || L->topk < 1 || L->topk > L->n_routed ||
        L->topk + L->n_shared > 64 || !L->router_w || !L->router_bias) {
        LOG("%s: invalid layer description", op);
        return 0;
    }
    if (L->n_shared > 0 && (!L->s_gate.buf || !L->s_up.buf || !L->s_down.buf)) {
        LOG("%s: shared expert tensors missing", op);
        return 0;
    }
    const int64_t H = L->hidden, I = L->inter, T = n_tokens;
    const int32_t nr = L->n_routed, ns = L->n_shared, tk = L->topk, n_sel = tk + ns;
    const int64_t n_tot = nr + ns;
    MoeProj g, u, d, sg, su, sd;
    memset(&sg, 0, sizeof sg);
    memset(&su, 0, sizeof su);
    memset(&sd, 0, sizeof sd);
    if (!moe_proj(op, "gate", &L->gate, nr, I, H, &g) || !moe_proj(op, "up", &L->up, nr, I, H, &u) ||
        !moe_proj(op, "down", &L->down, nr, H, I, &d))
        return 0;
    if (ns > 0 && (!moe_proj(op, "shared gate", &L->s_gate, ns, I, H, &sg) ||
                   !moe_proj(op, "shared up", &L->s_up, ns, I, H, &su) ||
                   !moe_proj(op, "shared down", &L->s_down, ns, H, I, &sd)))
        return 0;
    const MoeProj *ps[6] = { &g, &u, &d, &sg, &su, &sd };
    /* 4-byte-aligned rows everywhere (the int8 and f16 paths stage blocks
     * from 4-byte boundaries) */
    int q_aligned = 1;
    for (int i = 0; i < (ns > 0 ? 6 : 3); i++)
        if (((uintptr_t)ps[i]->base | ps[i]->stride | ps[i]->row_bytes) & 3) q_aligned = 0;
    /* f16 path: every projection in the real checkpoint's formats, 4-byte
     * aligned rows (activations as PH rows: kernels/prefill_h.h, 1056 bytes
     * per 256 columns); Q8_0 has no other prefill kernels */
    const int use_h_all = g_opt_pf_h && q_aligned && pf_type_h(g.type) && pf_type_h(d.type) &&
                          (ns == 0 || (pf_type_h(sg.type) && pf_type_h(sd.type)));
    for (int i = 0; i < (ns > 0 ? 6 : 3); i++)
        if (!(pf_type_ok(ps[i]->type) || (use_h_all && pf_type_h(ps[i]->type))) ||
            ((uintptr_t)ps[i]->base | ps[i]->stride | ps[i]->row_bytes) & 1) {
            LOG("%s: projection %d: ggml type %d or its layout is not supported by the prefill kernels", op, i,
                ps[i]->type);
            return 0;
        }
    if (g.type != u.type || (ns > 0 && sg.type != su.type)) {
        LOG("%s: gate and up must share a format", op);
        return 0;
    }
    if (!f32_off_ok(L->router_w_off, op, "router_w") || !f32_off_ok(L->router_bias_off, op, "router_bias") ||
        !chk(L->router_w, L->router_w_off, (size_t)n_tot * (size_t)H * 4, op, "router_w") ||
        !chk(L->router_bias, L->router_bias_off, (size_t)nr * 4, op, "router_bias") ||
        !chk(x, 0, (size_t)T * H * 4, op, "x") || !chk(y, 0, (size_t)T * H * 4, op, "y"))
        return 0;
    const size_t route_bytes = (size_t)T * (size_t)(tk + n_sel) * 4;
    if (route_out && !chk(route_out, 0, route_bytes, op, "route_out")) return 0;
    /* units of <= 32 pairs: routed pairs split over at most n_routed experts,
     * each shared expert takes every token */
    const int64_t umax = (T * tk + 31) / 32 + nr + (int64_t)ns * ((T + 31) / 32) + 1;
    /* grid rows of the f16 unit kernels: a multiple of 8, so they deal the
     * units to the 8 XCDs in turn (kernels/prefill.h pf_slot) */
    const int64_t ugrid = (umax + 7) & ~(int64_t)7;
    const int64_t P = T * n_sel;
    if (H % 256 || I % 256) {
        LOG("%s: hidden and inter must be multiples of 256", op);
        return 0;
    }
    /* int8 path: every projection Q2_K, Q3_K or Q4_K with 4-byte-aligned
     * rows (its DMA stages Q2_K and Q4_K blocks from their own starts);
     * activations as PQ rows (kernels/prefill_q.h: 832 bytes per 256
     * columns) */
    const int use_q = g_opt_pf_q && q_aligned && pf_type_int(g.type) && pf_type_int(d.type) &&
                      (ns == 0 || (pf_type_int(sg.type) && pf_type_int(sd.type)));
    const int use_h = !use_q && use_h_all;
    const int64_t ldqx = H / 256 * (use_h ? PH_REC : 832), ldqh = I / 256 * (use_h ? PH_REC : 832);
    const int use_qh = use_q || use_h;
    /* the pipelines address activation rows with 32-bit byte offsets */
    if (ugrid > 65535 || (H + 255) / 256 > MAX_GRID || (uint64_t)T * H * 2 >= (1ull << 32) ||
        (uint64_t)P * I * 2 >= (1ull << 32) || (T * H + 255) / 256 > MAX_GRID || P > MAX_GRID ||
        (use_qh && ((uint64_t)T * ldqx >= (1ull << 32) || (uint64_t)P * ldqh >= (1ull << 32)))) {
        LOG("%s: batch too large", op);
        return 0;
    }
    if (!need_batch(op)) return 0;

    size_t o = 0;
#define PF_REGION(name, bytes) const size_t name = o; o += ((size_t)(bytes) + 255) & ~(size_t)255
    PF_REGION(o_logits, T * n_tot * 4);
    PF_REGION(o_idx, T * tk * 4);
    PF_REGION(o_w, P * 4);
    PF_REGION(o_list, P * 4);
    PF_REGION(o_units, umax * 12);
    PF_REGION(o_nu, 4);   /* n_units */
    PF_REGION(o_xh, use_qh ? 0 : T * H * 2);
    PF_REGION(o_xl, use_qh ? 0 : T * H * 2);
    PF_REGION(o_hh, use_qh ? 0 : P * I * 2);
    PF_REGION(o_hl, use_qh ? 0 : P * I * 2);
    PF_REGION(o_pqx, use_qh ? T * ldqx : 0);
    PF_REGION(o_pqxs, use_qh ? T * 4 : 0);
    PF_REGION(o_hf, use_qh ? P * I * 4 : 0);
    PF_REGION(o_pqh, use_qh ? P * ldqh : 0);
    PF_REGION(o_pqhs, use_qh ? P * 4 : 0);
    PF_REGION(o_yp, P * H * 4);
#undef PF_REGION
    uint8_t *s = (uint8_t *)scratch(o, op);
    if (!s) return 0;
    float *logits = (float *)(s + o_logits), *sel_w = (float *)(s + o_w), *yp = (float *)(s + o_yp);
    void *xh = s + o_xh, *xl = s + o_xl, *hh = s + o_hh, *hl = s + o_hl;
    int32_t *sel_idx = (int32_t *)(s + o_idx), *list = (int32_t *)(s + o_list), *units = (int32_t *)(s + o_units),
            *n_units = (int32_t *)(s + o_nu);

    if (!prep_layer(L, &g, &u, &d, &sg, &su, &sd, x, (size_t)T * H * 4, op)) return 0;
    if (!prep_out(y, op) || (route_out && !prep_out(route_out, op))) return 0;

    const float *rw = (const float *)(L->router_w->dev + L->router_w_off);
    const float *rb = (const float *)(L->router_bias->dev + L->router_bias_off);
    int64_t ld = H, hid = H, inter = I, tt = T, ntot = n_tot;
    float rs = L->route_scale, gsc = L->global_scale;
    int32_t nr32 = nr, ns32 = ns, tk32 = tk, nsel32 = n_sel;
    void *a_rt[] = { &x->dev, &tt, &rw, &ld, &ntot, &hid, &logits };
    const int rt_m = g_opt_pf_route_m && ((((uintptr_t)x->dev | (uintptr_t)rw) & 15) == 0) && (ld % 4) == 0 && H % 512 == 0;
    if (rt_m ? !launch2(K_PF_ROUTE_M, (unsigned)((T + 15) / 16), (unsigned)((n_tot + 15) / 16), 256, 0, a_rt, op)
             : !launch2(K_PF_ROUTE, (unsigned)((T + 31) / 32), (unsigned)((n_tot + 31) / 32), 256, 0, a_rt, op))
        return 0;
    void *a_sel[] = { &logits, &rb, &nr32, &ns32, &tk32, &rs, &gsc, &sel_idx, &sel_w };
    if (!launch(K_PF_SELECT, (unsigned)T, 64, a_sel, op)) return 0;
    void *a_grp[] = { &sel_idx, &tt, &nr32, &ns32, &tk32, &list, &units, &n_units };
    if (!launch(K_PF_GROUP, 1, 1024, a_grp, op)) return 0;
    if (use_qh) {
        /* int8 (PQ rows) or f16 (PH rows): quantize x, gate/up to f32 h,
         * quantize h, down to the per-pair partial rows. The f16 gate/up
         * runs over 64-row slices of I, its down over 128-row slices of H
         * (a 256-row format takes two slices, in the first half of the
         * workgroups). */
        void *pqx = s + o_pqx, *pqxs = s + o_pqxs, *hf = s + o_hf, *pqh = s + o_pqh, *pqhs = s + o_pqhs;
        int64_t ldq_x = ldqx, ldq_h = ldqh;
        const int kq = use_q ? K_PF_QUANT : K_PH_QUANT;
        const unsigned th_p = use_q ? 512 : 64 * PH_WAVES;   /* threads of a projection workgroup */
        const unsigned gy = (unsigned)(use_q ? umax : ugrid);   /* its units */
        void *a_qx[] = { &x->dev, &hid, &hid, &pqx, &ldq_x, &pqxs };
        if (!launch(kq, (unsigned)T, 256, a_qx, op)) return 0;
        void *a_gq[] = { (void *)&g, (void *)&u, (void *)&sg, (void *)&su, &nr32, &nsel32, &inter, &hid,
                         &pqx, &pqxs, &list, &units, &n_units, &hf };
        if (!launch2(use_q ? K_PF_GATEUP_Q : K_PH_GATEUP, (unsigned)(use_q ? I / 128 : I / 64), gy, th_p,
                     PF_LDS_BYTES, a_gq, op))
            return 0;
        void *a_qh[] = { &hf, &inter, &inter, &pqh, &ldq_h, &pqhs };
        if (!launch(kq, (unsigned)P, 256, a_qh, op)) return 0;
        void *a_dq[] = { (void *)&d, (void *)&sd, &nr32, &inter, &hid, &pqh, &pqhs, &list, &units, &n_units, &yp };
        if (!launch2(use_q ? K_PF_DOWN_Q : K_PH_DOWN, (unsigned)(use_q ? H / 256 : H / 128), gy, th_p,
                     PF_LDS_BYTES, a_dq, op))
            return 0;
    } else {
        int64_t nseg = T * H / 16;
        void *a_sp[] = { &x->dev, &nseg, &xh, &xl };
        if (!launch(K_PF_SPLIT, (unsigned)((nseg + 255) / 256), 256, a_sp, op)) return 0;
        void *a_gu[] = { (void *)&g, (void *)&u, (void *)&sg, (void *)&su, &nr32, &nsel32, &inter, &hid, &xh, &xl,
                         &list, &units, &n_units, &hh, &hl };
        if (!launch2(K_PF_GATEUP, (unsigned)((I + 31) / 32), (unsigned)umax, 512, PF_LDS_BYTES, a_gu, op)) return 0;
        void *a_dn[] = { (void *)&d, (void *)&sd, &nr32, &inter, &hid, &hh, &hl, &list, &units, &n_units, &yp };
        if (!launch2(K_PF_DOWN, (unsigned)((H + 63) / 64), (unsigned)umax, 512, PF_LDS_BYTES, a_dn, op)) return 0;
    }
    void *a_cb[] = { &yp, &sel_w, &nsel32, &tt, &hid, &y->dev };
    if (!launch2(K_PF_COMBINE, (unsigned)((H + 255) / 256), (unsigned)T, 256, 0, a_cb, op)) return 0;
    if (route_out) {
        hipError_t e = hipMemcpyAsync(route_out->dev, sel_idx, (size_t)T * tk * 4, hipMemcpyDeviceToDevice, g_stream);
        if (e == hipSuccess)
            e = hipMemcpyAsync(route_out->dev + (size_t)T * tk * 4, sel_w, (size_t)P * 4, hipMemcpyDeviceToDevice,
                               g_stream);
        if (e != hipSuccess) {
            LOG("%s: route_out copy failed: %s", op, hipGetErrorString(e));
            return 0;
        }
    }
    return 1;
}

/* The SwiGLU expert FFN over n_slots = topk + n_shared slots: routed slot s
 * uses expert sel_idx[s] (or fixed + s when sel_idx is NULL), then come the
 * shared experts. One slot without weights stores y; several slots add
 * sel_w[s] * their output into y. Uses the matrix-core kernels when the
 * formats and shapes fit, else the tile kernels, else the generic
 * one-wave-per-row kernels. scr: scratch for the slots' f32 h vectors and
 * partial rows; cnt_region: the counter words (zero on entry, left zero). */
static int ffn_launch(const char *op, const MoeProj *g, const MoeProj *u, const MoeProj *d, const MoeProj *sg,
                      const MoeProj *su, const MoeProj *sd, const int32_t *sel_idx, const float *sel_w, int32_t fixed,
                      int32_t topk, int32_t n_shared, int64_t H, int64_t I, const uint8_t *xdev, float *ydev,
                      uint8_t *scr, uint8_t *cnt_region, const MqRoute *route) {
    int32_t n_slots = topk + n_shared;
    int64_t inter = I, hid = H;
    MqFfnPlan pl;
    MoeProj mp[6];
    if (mq_ffn_prep(g, u, d, sg, su, sd, topk, n_shared, H, I, route != NULL, mp, &pl)) {
        int32_t inter32 = (int32_t)I;
        float *h = (float *)scr;
        float *ypart = (float *)(scr + (size_t)n_slots * (size_t)I * 4);
        uint32_t *cnt = (uint32_t *)cnt_region + MQ_DN_CNT_OFF;
        MqRoute rt;
        memset(&rt, 0, sizeof rt);
        if (route) rt = *route;
        void *a_gu[] = { &mp[0], &mp[1], &mp[3], &mp[4], &sel_idx, &fixed, &topk, &inter32,
                         &pl.gu_wps_r, &pl.gu_wps_s, &xdev, &h, &pl.gu_geo_r, &pl.gu_geo_s, &rt };
        if (!launch_lds(K_MQ_GU, pl.gu_grid, pl.gu_threads, pl.gu_lds, a_gu, op)) return 0;
        void *a_dn[] = { &mp[2], &mp[5], &sel_idx, &sel_w, &fixed, &topk, &n_slots, &n_slots, &inter32, &hid, &h,
                         &ydev, &pl.dn_geo_r, &pl.dn_geo_s, &pl.dn_wps_r, &pl.dn_wps_s, &ypart, &cnt };
        return launch_lds(K_MQ_DN, pl.dn_grid, pl.dn_threads, pl.dn_lds, a_dn, op);
    }
    if (route) {
        LOG("%s: in-kernel selection needs the matrix-core FFN", op);
        return 0;
    }
    const int cr = tile_code(g->type), cdr = tile_code(d->type);
    const int cs = n_shared > 0 ? tile_code(sg->type) : cr, cds = n_shared > 0 ? tile_code(sd->type) : cdr;
    TileGeo gu, dn;
    int tile = g_opt_tile && cr >= 0 && cs >= 0 && cdr >= 0 && cds >= 0 && g->type == u->type && H % 256 == 0 &&
               I % 256 == 0 && proj_aligned(g) && proj_aligned(u) && proj_aligned(d) &&
               tile_geo(H / 256, I, 2 * (int64_t)n_slots, &gu) && tile_geo(I / 256, H, n_slots, &dn);
    if (tile && n_shared > 0)
        tile = sg->type == su->type && proj_aligned(sg) && proj_aligned(su) && proj_aligned(sd);
    float *h = (float *)scr;
    if (tile) {
        XpArgs xa = { NULL, NULL, NULL };
        float *y_zero = n_slots > 1 ? ydev : NULL;
        int64_t y_n = H;
        const int k_gu = K_FFN_BASE + 3 * (3 * cr + cs);
        const int k_dn = K_FFN_BASE + 3 * (3 * cdr + cds) + 2;
        void *a_gu[] = { (void *)g, (void *)u, (void *)sg, (void *)su, &sel_idx, &fixed, &topk, &inter, &hid,
                         &gu, &xdev, &xa, &h, &y_zero, &y_n };
        if (!launch_lds(k_gu, (unsigned)(n_slots * gu.tiles), TILE_NT, tile_lds(H, &gu, 2), a_gu, op))
            return 0;
        void *a_dn[] = { (void *)d, (void *)sd, &sel_idx, &sel_w, &fixed, &topk, &n_slots, &inter, &hid,
                         &dn, &h, &ydev };
        return launch_lds(k_dn, (unsigned)(n_slots * dn.tiles), TILE_NT, tile_lds(I, &dn, 1), a_dn, op);
    }
    void *a_gu[] = { (void *)g, (void *)u, (void *)sg, (void *)su, &sel_idx, &fixed, &topk, &inter, &xdev, &h };
    if (!launch(K_MOE_GATEUP, (unsigned)(n_slots * ((I + 3) / 4)), 256, a_gu, op)) return 0;
    void *a_dn[] = { (void *)d, (void *)sd, &sel_idx, &sel_w, &fixed, &topk, &n_shared, &inter, &hid, &h, &ydev };
    return launch(K_MOE_DOWN, blocks_for(H, 4), 256, a_dn, op);
}

/* The selection and weights into the caller's route_out (if any). */
static int route_copy(const char *op, SepiaGpuBuf *route_out, const int32_t *sel_idx, const float *sel_w, int topk,
                      int n_slots) {
    if (!route_out) return 1;
    hipError_t e = hipMemcpyAsync(route_out->dev, sel_idx, (size_t)topk * 4, hipMemcpyDeviceToDevice, g_stream);
    if (e == hipSuccess)
        e = hipMemcpyAsync(route_out->dev + (size_t)topk * 4, sel_w, (size_t)n_slots * 4, hipMemcpyDeviceToDevice,
                           g_stream);
    if (e != hipSuccess) {
        LOG("%s: route_out copy failed: %s", op, hipGetErrorString(e));
        return 0;
    }
    return 1;
}

/* The MoE decode layer on scratch from the library's growable region
 * (fixed == NULL) or from the allocation-free entry's device array: counter
 * words at fixed, data after CNT_BYTES, at most fixed_bytes in all. */
static int moe_decode_impl(const char *op, const SepiaMoeLayerDesc *L, SepiaGpuBuf *x, SepiaGpuBuf *y,
                           SepiaGpuBuf *route_out, uint8_t *fixed, size_t fixed_bytes) {
    if (!L || !x || !y || L->hidden <= 0 || L->inter <= 0 || L->n_routed < 1 || L->n_routed > 1024 ||
        L->n_shared < 0 || L->topk < 1 || L->topk > L->n_routed || L->topk + L->n_shared > 64 || !L->router_w ||
        !L->router_bias) {
        LOG("%s: invalid layer description", op);
        return 0;
    }
    if (L->n_shared > 0 && (!L->s_gate.buf || !L->s_up.buf || !L->s_down.buf)) {
        LOG("%s: shared expert tensors missing", op);
        return 0;
    }
    const int64_t H = L->hidden, I = L->inter;
    const int n_tot = L->n_routed + L->n_shared, n_slots = L->topk + L->n_shared;
    MoeProj g, u, d, sg, su, sd;
    memset(&sg, 0, sizeof sg);
    memset(&su, 0, sizeof su);
    memset(&sd, 0, sizeof sd);
    if (!moe_proj(op, "gate", &L->gate, L->n_routed, I, H, &g) || !moe_proj(op, "up", &L->up, L->n_routed, I, H, &u) ||
        !moe_proj(op, "down", &L->down, L->n_routed, H, I, &d))
        return 0;
    if (L->n_shared > 0 &&
        (!moe_proj(op, "shared gate", &L->s_gate, L->n_shared, I, H, &sg) ||
         !moe_proj(op, "shared up", &L->s_up, L->n_shared, I, H, &su) ||
         !moe_proj(op, "shared down", &L->s_down, L->n_shared, H, I, &sd)))
        return 0;
    if (!f32_off_ok(L->router_w_off, op, "router_w") || !f32_off_ok(L->router_bias_off, op, "router_bias") ||
        !chk(L->router_w, L->router_w_off, (size_t)n_tot * (size_t)H * 4, op, "router_w") ||
        !chk(L->router_bias, L->router_bias_off, (size_t)L->n_routed * 4, op, "router_bias") ||
        !chk(x, 0, (size_t)H * 4, op, "x") || !chk(y, 0, (size_t)H * 4, op, "y"))
        return 0;
    const size_t route_bytes = (size_t)(2 * L->topk + L->n_shared) * 4;
    if (route_out && !chk(route_out, 0, route_bytes, op, "route_out")) return 0;
    if ((int64_t)n_slots * ((I + 3) / 4) > MAX_GRID || (H + 3) / 4 > MAX_GRID) {
        LOG("%s: layer too large", op);
        return 0;
    }
    if (!need_batch(op)) return 0;

    /* scratch: logits | sel_idx | sel_w | FFN activations, each 256-byte
     * aligned; the router's arrival counter is the first word of the
     * counter region */
    const size_t o_logits = 0;
    const size_t o_idx = o_logits + (((size_t)n_tot * 4 + 255) & ~(size_t)255);
    const size_t o_w = o_idx + 256;
    const size_t o_h = o_w + 256;
    const size_t need = o_h + ffn_scratch_bytes(n_slots, I, H);
    uint8_t *s, *cnt_region;
    if (fixed) {
        if (CNT_BYTES + need > fixed_bytes) {
            LOG("%s: the layer needs %zu bytes of scratch; the allocation-free entry's device array holds %zu",
                op, CNT_BYTES + need, fixed_bytes);
            return 0;
        }
        s = fixed + CNT_BYTES;
        cnt_region = fixed;
    } else {
        s = (uint8_t *)scratch(need, op);
        if (!s) return 0;
        cnt_region = (uint8_t *)g_scratch;
    }
    float *logits = (float *)(s + o_logits), *sel_w = (float *)(s + o_w);
    int32_t *sel_idx = (int32_t *)(s + o_idx);
    uint32_t *counter = (uint32_t *)cnt_region;

    if (!prep_layer(L, &g, &u, &d, &sg, &su, &sd, x, (size_t)H * 4, op)) return 0;
    if (!prep_out(y, op) || (route_out && !prep_out(route_out, op))) return 0;
    if (fixed) {
        /* the array keeps the last call's contents: the router's and the
         * down launch's arrival counters must start at zero */
        uint32_t *cw = (uint32_t *)cnt_region;
        int64_t nw = MQ_DN_CNT_OFF + (H + 15) / 16;
        if (nw > (int64_t)(CNT_BYTES / 4)) nw = CNT_BYTES / 4;
        uint32_t zero = 0;
        void *a_fill[] = { &cw, &nw, &zero };
        if (!launch(K_FILL_U32, blocks_for(nw, 256), 256, a_fill, op)) return 0;
    }

    const float *rw = (const float *)(L->router_w->dev + L->router_w_off);
    const float *rb = (const float *)(L->router_bias->dev + L->router_bias_off);
    int64_t ld = H, hid = H;
    int32_t nr = L->n_routed, ns = L->n_shared, tk = L->topk;
    float rs = L->route_scale, gsc = L->global_scale;
    const MqRoute rt = { logits, rb, nr, ns, rs, gsc, sel_idx, sel_w };
    /* with the matrix-core FFN the gate/up launch selects from the logits;
     * otherwise the router's last workgroup does */
    MqFfnPlan pl;
    MoeProj mp[6];
    const int in_kernel = mq_ffn_prep(&g, &u, &d, &sg, &su, &sd, tk, ns, H, I, 1, mp, &pl);
    int32_t select = !in_kernel;
    void *a_route[] = { &rw, &ld, &rb, &x->dev, &hid, &nr, &ns, &tk, &rs, &gsc, &logits, &sel_idx, &sel_w, &counter,
                        &select };
    if (!launch(K_MOE_ROUTE, (unsigned)n_tot, RT_THREADS, a_route, op)) return 0;

    if (!ffn_launch(op, &g, &u, &d, &sg, &su, &sd, sel_idx, sel_w, 0, tk, ns, H, I, x->dev, (float *)y->dev, s + o_h,
                    cnt_region, in_kernel ? &rt : NULL))
        return 0;
    return route_copy(op, route_out, sel_idx, sel_w, L->topk, n_slots);
}

int sepia_gpu_moe_decode(const SepiaMoeLayerDesc *L, SepiaGpuBuf *x, SepiaGpuBuf *y, SepiaGpuBuf *route_out) {
    return moe_decode_impl("moe_decode", L, x, y, route_out, NULL, 0);
}

/* The same layer with every scratch byte in the library's fixed device
 * array (noalloc.hip): no allocation, so it may run under stream capture or
 * where hipMalloc is forbidden. Calls that overlap on one device race on the
 * array. */
int sepia_hip_moe_decode_noalloc(const SepiaMoeLayerDesc *L, SepiaGpuBuf *x, SepiaGpuBuf *y, SepiaGpuBuf *route_out) {
    const char *op = "moe_decode_noalloc";
    if (!need_init(op)) return 0;
    uint8_t *arr = g_noalloc_ok ? (uint8_t *)sepia_noalloc_ptr() : NULL;
    if (!arr) {
        LOG("%s: the device array is not set up on this device", op);
        return 0;
    }
    return moe_decode_impl(op, L, x, y, route_out, arr, SEPIA_NOALLOC_BYTES);
}

int sepia_gpu_expert_ffn(const SepiaExpertTensor *gate, const SepiaExpertTensor *up, const SepiaExpertTensor *down,
                         int n_experts, int expert, int64_t hidden, int64_t inter, SepiaGpuBuf *x, SepiaGpuBuf *y) {
    const char *op = "expert_ffn";
    if (!gate || !up || !down || !x || !y || hidden <= 0 || inter <= 0 || n_experts < 1 || expert < 0 ||
        expert >= n_experts || (inter + 3) / 4 > MAX_GRID || (hidden + 3) / 4 > MAX_GRID) {
        LOG("%s: invalid arguments", op);
        return 0;
    }
    MoeProj g, u, d, none;
    memset(&none, 0, sizeof none);
    if (!moe_proj(op, "gate", gate, n_experts, inter, hidden, &g) || !moe_proj(op, "up", up, n_experts, inter, hidden, &u) ||
        !moe_proj(op, "down", down, n_experts, hidden, inter, &d))
        return 0;
    if (!chk(x, 0, (size_t)hidden * 4, op, "x") || !chk(y, 0, (size_t)hidden * 4, op, "y")) return 0;
    if (!need_batch(op)) return 0;
    uint8_t *scr = (uint8_t *)scratch(ffn_scratch_bytes(1, inter, hidden), op);
    if (!scr) return 0;
    if (!prep_in_r(gate->buf, gate->off + (size_t)expert * gate->stride, (size_t)inter * g.row_bytes, op) ||
        !prep_in_r(up->buf, up->off + (size_t)expert * up->stride, (size_t)inter * u.row_bytes, op) ||
        !prep_in_r(down->buf, down->off + (size_t)expert * down->stride, (size_t)hidden * d.row_bytes, op) ||
        !prep_in(x, op) || !prep_out(y, op))
        return 0;
    return ffn_launch(op, &g, &u, &d, &none, &none, &none, NULL, NULL, expert, 1, 0, hidden, inter, x->dev,
                      (float *)y->dev, scr, (uint8_t *)g_scratch, NULL);
}
