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
    /* matrix-core matvecs (kernels/mq.h): Q2_K, Q3_K, Q4_K */
    K_MQ_MV = K_FFN_BASE + 27,
    /* matrix-core expert FFN: gate/up, down */
    K_MQ_GU = K_MQ_MV + 5,
    K_MQ_DN = K_MQ_GU + 1,
    /* the whole MoE layer / expert FFN in one launch (kernels/mq_fused.h) */
    K_MQ_MOE = K_MQ_DN + 1,
    /* batched prefill MoE layer (kernels/prefill.h) */
    K_PF_ROUTE = K_MQ_MOE + 1, K_PF_SELECT, K_PF_GROUP, K_PF_GATEUP, K_PF_DOWN, K_PF_COMBINE, K_PF_SPLIT,
    /* one expert's FFN in one launch, gate/up and down waves side by side (kernels/mq_flow.h) */
    K_MQ_FFN,
    /* MoE gate/up with the selection behind shared-expert streaming (kernels/mq_mix.h) */
    K_MQ_GU_MIX,
    /* MoE down with every slot of a row group in one workgroup (kernels/mq_rows.h) */
    K_MQ_DN_ROWS,
    /* prefill gate/up of the integer formats with 16 waves a workgroup (kernels/prefill.h) */
    K_PF_GATEUP_I,
    /* prefill gate/up of the integer formats with the codes in registers (kernels/prefill.h) */
    K_PF_GATEUP_R,
    /* prefill down of the integer formats with the codes in registers (kernels/prefill.h) */
    K_PF_DOWN_R,
    /* prefill router logits on the f32 matrix cores (kernels/prefill.h) */
    K_PF_ROUTE_M,
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
    "sepia_mq_gateup", "sepia_mq_down", "sepia_mq_moe",
    "sepia_pf_route", "sepia_pf_select", "sepia_pf_group", "sepia_pf_gateup", "sepia_pf_down", "sepia_pf_combine",
    "sepia_pf_split", "sepia_mq_ffn", "sepia_mq_gateup_mix", "sepia_mq_down_rows", "sepia_pf_gateup_i",
    "sepia_pf_gateup_r", "sepia_pf_down_r", "sepia_pf_route_m",
};
#undef FFN_NAMES

/* GGUF block geometry (reference src/quants.c:46-51; tools/gguf_inspect.py:109-117). */
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
static int g_opt_mq_x = 0;   /* "mq_x": 0 = planner's choice, 1 = vector from global, 2 = vector by LDS DMA,
                              * 3 = converter waves */
static int g_opt_fuse = 0;   /* sepia_hip_set_option("fuse", 1) runs the MoE layer / expert FFN as one launch */
static int g_opt_mix = 0;    /* "mix": 1 runs the MoE decode's gate/up as sepia_mq_gateup_mix (every workgroup
                              * streams shared units while its wave 0 selects, then routed ones) */
static int g_opt_dnrows = 0; /* "dnrows": 1 runs the MoE decode's down as sepia_mq_down_rows (all slots of
                              * a row group in one workgroup, summed in LDS) */
static int g_opt_hxq = 0;    /* "hxq": 1 = h crosses from gate/up to down in XQ form (measured slower: the XQ epilogue costs gate/up more than it saves down), 0 = f32 */
static int g_opt_dyn = 0;    /* "dyn": 1 deals the MoE down launch's steps at run time (MqDyn) */
static int g_opt_pf_gu = 2;   /* "pf_gu": the gate/up launch of a prefill layer whose gate/up projections are
                               * all Q2_K, Q3_K or Q4_K: 2 = sepia_pf_gateup_r (codes in registers), 1 =
                               * sepia_pf_gateup_i (16 waves), 0 = sepia_pf_gateup (other layers always) */
static int g_opt_pf_route_m = 1;   /* "pf_route_m": 1 = prefill router logits on the f32 matrix cores
                                    * (sepia_pf_route_m) when x and the router rows are 16-byte aligned,
                                    * 0 = sepia_pf_route */
static int g_opt_pf_dn = 1;   /* "pf_dn": 1 = a prefill layer whose down projections are all Q2_K, Q3_K or Q4_K
                               * runs them as sepia_pf_down_r (codes in registers), 0 = sepia_pf_down */
static int g_opt_route_sel = 0;   /* "route_sel": 1 = the router launch's last workgroup selects the
                                   * experts even for the matrix-core FFN (0: its gate/up launch does) */
static int g_opt_flow = 0;   /* "flow": 1 runs the expert FFN as one sepia_mq_ffn launch (gate/up and down waves) */
static int g_opt_flow_delay = 250;   /* "flow_delay": s_memrealtime ticks (10 ns) a flow workgroup without
                                      * gate/up units holds its down weights back */
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
static int g_fused_pending = 0;     /* a fused launch ran in the open batch: check its error flag at end */
static int g_have_iq2xxs;
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

struct SepiaGpuBuf {
    uint8_t *dev;
    void *host;        /* pinned copy (shared), caller's base (wrapped), NULL (private) */
    size_t len;
    int kind;
    int exposed;       /* host_ptr handed out: the host may write it */
    int host_newer;    /* upload before the next device access */
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

/* Bring the device copy up to date before a kernel touches the buffer. */
static int sync_in(SepiaGpuBuf *b, const char *op) {
    if (b->kind == BUF_SHARED && b->host_newer) {
        hipError_t e = hipMemcpyAsync(b->dev, b->host, b->len, hipMemcpyHostToDevice, g_stream);
        if (e != hipSuccess) {
            LOG("%s: upload failed: %s", op, hipGetErrorString(e));
            return 0;
        }
        b->host_newer = 0;
    }
    return 1;
}

static int prep_in(SepiaGpuBuf *b, const char *op) { return sync_in(b, op); }
static int prep_out(SepiaGpuBuf *b, const char *op) {
    if (!sync_in(b, op)) return 0;
    if (b->kind == BUF_SHARED) b->dev_newer = 1;
    return 1;
}

/* Library scratch in HBM: a region of arrival counters (zeroed once; every
 * kernel that uses one leaves it at zero again) followed by a data region
 * for partial sums and intermediate vectors, grown on demand. */
#define CNT_BYTES (64u * 1024u)
#define MQ_BAR_WORD 1               /* fused launches' grid-barrier counter (never reset) */
#define MQ_ERR_WORD 2               /* fused and flow launches' time-out flag */
#define MQ_FLOW_HCNT_WORD 3         /* flow launches: units of h published (back to zero at the end) */
#define MQ_FLOW_FLAG_OFF 8192       /* flow launches: workgroup b's h flag at word OFF + 32 b (lowered again) */
#define MQ_FLOW_FLAG_WORDS (32 * 256)
static void *g_scratch;
static size_t g_scratch_len;

/* Data region of at least `need` bytes (the counters sit in front of it).
 * Growing waits for the stream, since queued kernels may still use the old
 * region; the new allocation is cleared so every counter starts at zero. */
static void *scratch(size_t need, const char *op) {
    if (g_scratch && need <= g_scratch_len - CNT_BYTES) return (uint8_t *)g_scratch + CNT_BYTES;
    hipStreamSynchronize(g_stream);
    if (g_scratch) hipFree(g_scratch);
    g_scratch = NULL;
    g_scratch_len = 0;
    size_t want = CNT_BYTES + (need < (4u << 20) ? (4u << 20) : need);
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

static SepiaGpuBuf *new_buf(size_t len, int kind) {
    SepiaGpuBuf *b = (SepiaGpuBuf *)calloc(1, sizeof *b);
    if (!b) {
        LOG("alloc: out of host memory");
        return NULL;
    }
    b->len = len;
    b->kind = kind;
    hipError_t e = hipMalloc((void **)&b->dev, dev_bytes(len));
    if (e != hipSuccess) {
        LOG("alloc: hipMalloc(%zu) failed: %s", dev_bytes(len), hipGetErrorString(e));
        free(b);
        return NULL;
    }
    return b;
}

SepiaGpuBuf *sepia_gpu_alloc(size_t len, int gpu_private) {
    if (!need_init("alloc")) return NULL;
    if (len == 0) {
        LOG("alloc: zero length");
        return NULL;
    }
    SepiaGpuBuf *b = new_buf(len, gpu_private ? BUF_PRIVATE : BUF_SHARED);
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
        e = hipHostMalloc(&b->host, len, hipHostMallocDefault);
        if (e != hipSuccess) {
            LOG("alloc: pinned host copy of %zu bytes failed: %s", len, hipGetErrorString(e));
            hipFree(b->dev);
            free(b);
            return NULL;
        }
        memset(b->host, 0, len);
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
        if (b->host) hipHostFree(b->host);
    }
    if (b->dev) hipFree(b->dev);
    free(b);
}

void *sepia_gpu_host_ptr(SepiaGpuBuf *b) {
    if (!b) return NULL;
    if (b->kind == BUF_PRIVATE) return NULL;
    if (b->kind == BUF_SHARED) {
        b->exposed = 1;
        b->host_newer = 1;
    }
    return b->host;
}

uint64_t sepia_gpu_gpu_addr(SepiaGpuBuf *b) { return b ? (uint64_t)(uintptr_t)b->dev : 0; }

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
    for (SepiaGpuBuf *b = g_shared; b; b = b->next)
        if (b->exposed) b->host_newer = 1;
    if (e != hipSuccess) {
        LOG("end: batch failed: %s", hipGetErrorString(e));
        return 0;
    }
    if (g_fused_pending) {
        /* a fused launch whose grid barrier timed out leaves its flag (word
         * MQ_ERR_WORD of the counter region) set; its results are invalid */
        g_fused_pending = 0;
        uint32_t flag = 0;
        e = hipMemcpy(&flag, (uint32_t *)g_scratch + MQ_ERR_WORD, 4, hipMemcpyDeviceToHost);
        if (e == hipSuccess && flag) {
            /* clear the flag, realign the barrier counter (a workgroup that
             * gave up left it between multiples of the grid size) and zero
             * the flow counters */
            const uint32_t zero[3] = { 0, 0, 0 };
            hipMemcpy((uint32_t *)g_scratch + MQ_BAR_WORD, zero, 12, hipMemcpyHostToDevice);
            hipMemset((uint32_t *)g_scratch + MQ_FLOW_FLAG_OFF, 0, MQ_FLOW_FLAG_WORDS * 4);
            hipDeviceSynchronize();
            LOG("end: a one-launch FFN timed out waiting (flag %u); the batch's results are invalid", flag);
            return 0;
        }
        if (e != hipSuccess) {
            LOG("end: reading the fused-launch flag failed: %s", hipGetErrorString(e));
            return 0;
        }
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

/* Launch of kernel k on a gx x gy grid of `block`-thread workgroups with
 * `lds` bytes of dynamic LDS (timed when the profiler is on). */
static int launch2(int k, unsigned gx, unsigned gy, unsigned block, size_t lds, void **args, const char *op) {
    if (gx == 0 || gy == 0) return 1;
    hipError_t e;
    if (g_prof_on && g_prof_n < g_prof_ev_made) {
        const int slot = g_prof_n++;
        g_prof_kid[slot] = k;
        e = hipExtModuleLaunchKernel(g_fn[k], gx * block, gy, 1, block, 1, 1, lds, g_stream, args, NULL,
                                     g_prof_ev[slot][0], g_prof_ev[slot][1], 0);
    } else {
        if (g_prof_on) g_prof_overflow = 1;
        e = hipModuleLaunchKernel(g_fn[k], gx, gy, 1, block, 1, 1, (unsigned)lds, g_stream, args, NULL);
    }
    if (e != hipSuccess) {
        LOG("%s: launch of %s failed: %s", op, k_names[k], hipGetErrorString(e));
        return 0;
    }
    return 1;
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
    if (!need_batch(op) || !prep_in(w, op) || !prep_in(x, op) || !prep_out(y, op)) return 0;
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
    if (!need_batch(op) || !prep_in(w, op) || !prep_in(x, op) || !prep_out(y, op)) return 0;
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
    if (!need_batch(op) || !prep_in(w, op) || !prep_in(hist, op) || !prep_in(in, op) || !prep_out(out, op))
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

int sepia_gpu_rel_project(SepiaGpuBuf *r_vec, SepiaGpuBuf *rel_proj, SepiaGpuBuf *rel_logits, int64_t T, int64_t H,
                          int64_t d_rel, int64_t rel_extent) {
    (void)r_vec; (void)rel_proj; (void)rel_logits; (void)T; (void)H; (void)d_rel; (void)rel_extent;
    LOG("rel_project: banded attention is not implemented by this backend");
    return 0;
}

int sepia_gpu_rel_project_off(SepiaGpuBuf *r_vec, SepiaGpuBuf *rel_proj, size_t rel_proj_off,
                              SepiaGpuBuf *rel_logits, int64_t T, int64_t H, int64_t d_rel, int64_t rel_extent) {
    (void)r_vec; (void)rel_proj; (void)rel_proj_off; (void)rel_logits; (void)T; (void)H; (void)d_rel;
    (void)rel_extent;
    LOG("rel_project_off: banded attention is not implemented by this backend");
    return 0;
}

int sepia_gpu_banded_attn(SepiaGpuBuf *q, SepiaGpuBuf *k, SepiaGpuBuf *v, SepiaGpuBuf *rel_logits,
                          SepiaGpuBuf *attn_out, const int64_t *kv_lo, const int64_t *kv_hi, const float *tau,
                          int64_t T, int64_t H, int64_t Hkv, int64_t Dh, int64_t rel_extent, int64_t q_pos_base,
                          int64_t kv_dim, float inv_head_dim) {
    (void)q; (void)k; (void)v; (void)rel_logits; (void)attn_out; (void)kv_lo; (void)kv_hi; (void)tau;
    (void)T; (void)H; (void)Hkv; (void)Dh; (void)rel_extent; (void)q_pos_base; (void)kv_dim; (void)inv_head_dim;
    LOG("banded_attn: banded attention is not implemented by this backend");
    return 0;
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
    if (strcmp(name, "mq_x") == 0 && value >= 0 && value <= 3) {
        g_opt_mq_x = value;
        return 1;
    }
    if (strcmp(name, "fuse") == 0 && (value == 0 || value == 1)) {
        g_opt_fuse = value;
        return 1;
    }
    if (strcmp(name, "mix") == 0 && (value == 0 || value == 1)) {
        g_opt_mix = value;
        return 1;
    }
    if (strcmp(name, "dnrows") == 0 && (value == 0 || value == 1)) {
        g_opt_dnrows = value;
        return 1;
    }
    if (strcmp(name, "hxq") == 0 && (value == 0 || value == 1)) {
        g_opt_hxq = value;
        return 1;
    }
    if (strcmp(name, "dyn") == 0 && (value == 0 || value == 1)) {
        g_opt_dyn = value;
        return 1;
    }
    if (strcmp(name, "pf_gu") == 0 && value >= 0 && value <= 2) {
        g_opt_pf_gu = value;
        return 1;
    }
    if (strcmp(name, "pf_route_m") == 0 && (value == 0 || value == 1)) {
        g_opt_pf_route_m = value;
        return 1;
    }
    if (strcmp(name, "pf_dn") == 0 && (value == 0 || value == 1)) {
        g_opt_pf_dn = value;
        return 1;
    }
    if (strcmp(name, "route_sel") == 0 && (value == 0 || value == 1)) {
        g_opt_route_sel = value;
        return 1;
    }
    if (strcmp(name, "flow") == 0 && (value == 0 || value == 1)) {
        g_opt_flow = value;
        return 1;
    }
    if (strcmp(name, "flow_delay") == 0 && value >= 0 && value <= 100000) {
        g_opt_flow_delay = value;
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
    int32_t P, ring, xraw, orings, conv, dyn, xq_in;   /* as struct MqGeo in kernels/mq.h */
} MqGeo;
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
#define MQ_SEL_BYTES 512            /* the gate/up kernel's selection area in LDS */
#define MQ_XDMA_GAIN 40             /* mq_geo: cost units the vector's LDS DMA saves (measured ~2 us a launch) */
#define MQ_CONV_GAIN 60             /* mq_geo: cost units converter waves save (XQ off the weights' path); by
                                     * default only for the IQ formats, where they measured faster (C4 IQ3_XXS
                                     * 12.2 -> 11.2 us); the K-quants' stepping waves need all 16 */
#define MQ_XQ_SEGS_PER_WAVE 128     /* segments a converter wave turns into XQ at most (MQ_XQP passes of 16) */
static size_t mq_xq_bytes(int64_t n) { return (size_t)(n / 256) * 832 + 3 * (size_t)(n / 16) * 4; }
/* matrix-core format codes: 0..2 the K-quants (matvec and the FFN kernels),
 * 3..4 IQ2_XS and IQ3_XXS (matvec) */
static int mq_code(int t) {
    switch (t) {
    case SEPIA_T_Q2_K: return 0;
    case SEPIA_T_Q3_K: return 1;
    case 12: return 2;
    case 17: return 3;
    case 18: return 4;
    default: return -1;
    }
}
static const int k_mq_words[5] = { 7, 7, 9, 5, 7 };   /* padded words per lane (MQ<T>::Wp) */
static const size_t k_mq_table[5] = { 0, 0, 0, 4096, 1024 };   /* LDS codebook bytes (MQ<T>::table_bytes) */
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
     * converter waves (DMA into the XQ place, converted there); 1 and 2 need
     * the vector's size (raw_bytes) */
    const int64_t segs = (int64_t)raw_bytes / 64, cv_need = (segs + MQ_XQ_SEGS_PER_WAVE - 1) / MQ_XQ_SEGS_PER_WAVE;
    /* a forced mode the launch cannot take (converter waves for the FFN
     * launches) leaves the choice to the planner */
    const int forced = (g_opt_mq_x == 3 && !allow_conv) ? 0 : g_opt_mq_x;
    for (int mode = 0; mode <= (raw_bytes > 0 ? (allow_conv ? 2 : 1) : 0); mode++) {
        if (raw_bytes > 0 && (forced ? forced != mode + 1 : (mode == 2 && mc < 3))) continue;
        for (int P = 1; P <= 16 && P <= nq; P++) {
            if (g_opt_mq_p && P != g_opt_mq_p) continue;
            for (int C = 1; C * P <= 16 && C <= n_items; C++) {
                if (g_opt_mq_c && C != g_opt_mq_c) continue;
                const int nw = C * P;
                int cv = 0;
                if (mode == 2) {
                    if (nw + cv_need > 16) continue;
                    cv = 16 - nw < 4 ? 16 - nw : 4;
                    if (cv < cv_need) cv = (int)cv_need;
                }
                const int64_t spw = ((n_items + C - 1) / C) * ((nq + P - 1) / P);
                const size_t o_raw = align256(fixed + (size_t)n_items * P * 64);
                const size_t base = mode == 1 ? align256(o_raw + raw_bytes) : mode == 2 ? align256(o_raw + 16) : o_raw;
                if (base + (size_t)nw * wm > g_lds_max) continue;
                size_t ring = ((g_lds_max - base) / (size_t)nw) & ~(size_t)1023;
                if (ring > 4 * wm) ring = 4 * wm;
                if (g_opt_mq_s) {
                    ring = (size_t)g_opt_mq_s * wm;
                    if (base + (size_t)nw * ring > g_lds_max) continue;
                }
                int64_t S = (int64_t)(ring / w1);
                if (S > 4) S = 4;
                if (S > spw) S = spw;
                /* the vector by DMA ahead of the weights saves about as
                 * much as MQ_XDMA_GAIN cost units, converter waves more */
                const int64_t cost = spw * ((S >= 2 || spw == 1) ? 10 : 16) -
                                     (mode == 1 ? MQ_XDMA_GAIN : mode == 2 ? MQ_CONV_GAIN : 0);
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
                    geo->conv = cv;
                    geo->dyn = 0;
                    geo->xq_in = 0;
                    *threads = 64u * (unsigned)(nw + cv);
                    *lds = base + (size_t)nw * ring;
                }
            }
        }
    }
    return found;
}

/* mq_geo for a launch whose steps are dealt at run time (MqDyn): every
 * quad of an item has its partial (P = nq), the vector comes by LDS DMA
 * into a raw copy, and the waves and ring stages give the most steps in
 * flight (then the most waves). */
static int mq_geo_dyn(int mc, int wmax, int64_t n_items, int64_t nq, size_t fixed, size_t raw_bytes, unsigned *threads,
                      MqGeo *geo, size_t *lds) {
    if (raw_bytes == 0 || nq > 16) return 0;
    const size_t w1 = (size_t)k_mq_words[mc] * 1024, wm = (size_t)wmax * 1024;
    const size_t o_raw = align256(fixed + (size_t)n_items * nq * 64);
    const size_t base = align256(o_raw + raw_bytes);
    int64_t best = -1;
    int found = 0;
    for (int nw = 16; nw >= 1; nw--) {
        if (base + (size_t)nw * wm > g_lds_max) continue;
        size_t ring = ((g_lds_max - base) / (size_t)nw) & ~(size_t)1023;
        if (ring > 4 * wm) ring = 4 * wm;
        int64_t S = (int64_t)(ring / w1);
        if (S > 4) S = 4;
        int64_t fl = (int64_t)nw * S;
        if (fl > n_items * nq) fl = n_items * nq;
        if (fl > best) {
            best = fl;
            found = 1;
            geo->P = (int32_t)nq;
            geo->ring = (int32_t)ring;
            geo->xraw = (int32_t)o_raw;
            geo->orings = (int32_t)base;
            geo->conv = 0;
            geo->dyn = 1;
            geo->xq_in = 0;
            *threads = 64u * (unsigned)nw;
            *lds = base + (size_t)nw * ring;
        }
    }
    return found;
}

/* Shapes the matrix-core kernels take: a format with a decoder, 4-byte
 * aligned rows of a multiple of 4 blocks, row offsets within 32 bits. */
static int mq_shape_ok(int type, int64_t n_blocks, int64_t rows, uintptr_t base, uint64_t row_bytes) {
    return g_opt_mq && mq_code(type) >= 0 && n_blocks >= 4 && n_blocks % 4 == 0 && base % 4 == 0 &&
           row_bytes % 4 == 0 && (uint64_t)rows * row_bytes < (1ull << 32);
}

static int mq_plan(int type, int64_t n_blocks, int64_t rows, uintptr_t base, uint64_t row_bytes, unsigned *threads,
                   size_t *lds, unsigned *grid, MqGeo *geo) {
    if (!mq_shape_ok(type, n_blocks, rows, base, row_bytes)) return -1;
    const int mc = mq_code(type);
    const int64_t tiles = (rows + 15) / 16;
    const int64_t per = (tiles + MQ_CUS - 1) / MQ_CUS;     /* row groups per workgroup */
    *grid = (unsigned)((tiles + per - 1) / per);
    if (!mq_geo(mc, k_mq_words[mc], per, n_blocks / 4, MQ_ZERO + mq_xq_bytes(256 * n_blocks) + k_mq_table[mc],
                (size_t)1024 * n_blocks, 1, threads, geo, lds))
        return -1;
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
    if (!need_batch(op) || !prep_in(w, op) || !prep_in(x, op) || !prep_out(y, op)) return 0;
    const uint8_t *wp = w->dev + w_off;
    unsigned mq_threads, mq_grid;
    size_t mq_lds;
    MqGeo mgeo;
    const int kmq = mq_plan(ggml_type, n_blocks, out_dim, (uintptr_t)wp, row_bytes, &mq_threads, &mq_lds, &mq_grid,
                            &mgeo);
    if (kmq >= 0) {
        int32_t nb32 = (int32_t)n_blocks;
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
    if (!need_batch(op) || !prep_in(raw, op) || !prep_out(out, op)) return 0;
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
    MqGeo gu_geo, dn_geo;
    int32_t gu_hxq;                 /* gate/up writes h in XQ form, the down launch takes it so */
} MqFfnPlan;
#define MQ_DN_CNT_OFF 64            /* first down arrival counter (u32 index in the counter region) */
static int mq_proj_ok(const MoeProj *p, int64_t rows) {
    return mq_code(p->type) <= 2 && mq_shape_ok(p->type, p->n_blocks, rows, (uintptr_t)p->base, p->row_bytes) &&
           p->stride % 4 == 0;
}
/* Workgroups per slot for slots of byte weights br (routed) and bs (shared):
 * at most MQ_CUS in all (unless one per slot is already more), at most
 * `tiles` per slot, the bytes per workgroup as even as whole counts allow
 * (proportional shares rounded down, then one more workgroup at a time to
 * the kind with the most bytes per workgroup while it fits). */
static void mq_split(int32_t topk, int32_t n_shared, double br, double bs, int64_t tiles, int32_t *wr, int32_t *ws) {
    const double tot = topk * br + n_shared * bs;
    int64_t r = (int64_t)(MQ_CUS * br / tot), sh = (int64_t)(MQ_CUS * bs / tot);
    if (r < 1) r = 1;
    if (sh < 1) sh = 1;
    if (r > tiles) r = tiles;
    if (sh > tiles) sh = tiles;
    for (;;) {
        const int64_t used = topk * r + n_shared * sh;
        const int can_r = topk > 0 && r < tiles && used + topk <= MQ_CUS;
        const int can_s = n_shared > 0 && sh < tiles && used + n_shared <= MQ_CUS;
        if (can_r && (!can_s || br / (double)r >= bs / (double)sh)) r++;
        else if (can_s) sh++;
        else break;
    }
    *wr = (int32_t)r;
    *ws = (int32_t)sh;
}
static int mq_ffn_plan(const MoeProj *g, const MoeProj *u, const MoeProj *d, const MoeProj *sg, const MoeProj *su,
                       const MoeProj *sd, int32_t topk, int32_t n_shared, int64_t H, int64_t I, MqFfnPlan *pl) {
    if (!g_opt_mq || H % 1024 || I % 1024) return 0;
    const MoeProj *ps[6] = { g, u, d, sg, su, sd };
    const int64_t rows[6] = { I, I, H, I, I, H };
    for (int i = 0; i < (n_shared > 0 ? 6 : 3); i++)
        if (!mq_proj_ok(ps[i], rows[i])) return 0;
    if (g->type != u->type || (n_shared > 0 && sg->type != su->type)) return 0;
    const int64_t tiles_i = (I + 15) / 16, tiles_h = (H + 15) / 16;
    if (n_shared + topk > 1 && MQ_DN_CNT_OFF + tiles_h > MQ_FLOW_FLAG_OFF) return 0;
    /* both slot kinds share a geometry: planned for the format of the
     * routed slots (the shared ones when there are none), with rings that
     * hold a step of either */
    const int kg = mq_code(topk > 0 ? g->type : sg->type), kd = mq_code(topk > 0 ? d->type : sd->type);
    int wgu = k_mq_words[kg], wdn = k_mq_words[kd];
    if (n_shared > 0 && k_mq_words[mq_code(sg->type)] > wgu) wgu = k_mq_words[mq_code(sg->type)];
    if (n_shared > 0 && k_mq_words[mq_code(sd->type)] > wdn) wdn = k_mq_words[mq_code(sd->type)];
    mq_split(topk, n_shared, (double)g->row_bytes, n_shared > 0 ? (double)sg->row_bytes : 1.0, tiles_i,
             &pl->gu_wps_r, &pl->gu_wps_s);
    mq_split(topk, n_shared, (double)d->row_bytes, n_shared > 0 ? (double)sd->row_bytes : 1.0, tiles_h,
             &pl->dn_wps_r, &pl->dn_wps_s);
    const int32_t gmin = pl->gu_wps_r < pl->gu_wps_s || n_shared == 0 ? pl->gu_wps_r : pl->gu_wps_s;
    const int32_t dmin = pl->dn_wps_r < pl->dn_wps_s || n_shared == 0 ? pl->dn_wps_r : pl->dn_wps_s;
    const int64_t nk_gu = (tiles_i + gmin - 1) / gmin, nk_dn = (tiles_h + dmin - 1) / dmin;
    if (!mq_geo(kg, wgu, 2 * nk_gu, H / 1024, MQ_ZERO + mq_xq_bytes(H) + MQ_SEL_BYTES, (size_t)H * 4, 0,
                &pl->gu_threads, &pl->gu_geo, &pl->gu_lds))
        return 0;
    const size_t dn_fixed = MQ_ZERO + mq_xq_bytes(I) + (size_t)nk_dn * 4 + 256;
    /* h crosses in XQ form (the down launch only DMAs it into place) unless
     * an experimental launch that reads f32 h is switched on */
    pl->gu_hxq = g_opt_hxq && !(g_opt_mix || g_opt_dnrows || g_opt_dyn);
    if (pl->gu_hxq) {
        if (!mq_geo(kd, wdn, nk_dn, I / 1024, dn_fixed, 0, 0, &pl->dn_threads, &pl->dn_geo, &pl->dn_lds)) return 0;
        pl->dn_geo.xq_in = 1;
    } else if (!(g_opt_dyn && !g_opt_mq_x && mq_geo_dyn(kd, wdn, nk_dn, I / 1024, dn_fixed, (size_t)I * 4,
                                                         &pl->dn_threads, &pl->dn_geo, &pl->dn_lds)) &&
               !mq_geo(kd, wdn, nk_dn, I / 1024, dn_fixed, (size_t)I * 4, 0, &pl->dn_threads, &pl->dn_geo,
                       &pl->dn_lds)) {
        return 0;
    }
    pl->gu_grid = (unsigned)(topk * pl->gu_wps_r + n_shared * pl->gu_wps_s);
    pl->dn_grid = (unsigned)(topk * pl->dn_wps_r + n_shared * pl->dn_wps_s);
    return 1;
}

/* LDS of the prefill projection kernels (PF_LDS_BYTES in kernels/prefill.h):
 * the whole 160 KB (tiles, raw-block stages, row tables at the top). */
#define PF_LDS_BYTES 163840
/* Formats the prefill projections decode (kernels/prefill.h). */
static int pf_type_ok(int t) {
    return t == SEPIA_T_Q2_K || t == SEPIA_T_Q3_K || t == 12 || t == 13 || t == 14 || t == 17 || t == 18 || t == 23;
}
/* Formats the prefill integer pipelines take as exact codes (Q2_K, Q3_K, Q4_K). */
static int pf_type_int(int t) { return t == SEPIA_T_Q2_K || t == SEPIA_T_Q3_K || t == 12; }

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
    for (int i = 0; i < (ns > 0 ? 6 : 3); i++)
        if (!pf_type_ok(ps[i]->type) || ((uintptr_t)ps[i]->base | ps[i]->stride | ps[i]->row_bytes) & 1) {
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
    const int64_t P = T * n_sel;
    /* the pipelines address activation rows with 32-bit byte offsets */
    if (umax > 65535 || (H + 255) / 256 > MAX_GRID || (uint64_t)T * H * 2 >= (1ull << 32) ||
        (uint64_t)P * I * 2 >= (1ull << 32) || (T * H + 255) / 256 > MAX_GRID) {
        LOG("%s: batch too large", op);
        return 0;
    }
    if (H % 256 || I % 256) {
        LOG("%s: hidden and inter must be multiples of 256", op);
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
    PF_REGION(o_nu, 8);   /* n_units, then the "x has a nonzero lo part" flag */
    PF_REGION(o_s16, T * H / 16 * 4);
    PF_REGION(o_xh, T * H * 2);
    PF_REGION(o_xl, T * H * 2);
    PF_REGION(o_hh, P * I * 2);
    PF_REGION(o_hl, P * I * 2);
    PF_REGION(o_yp, P * H * 4);
#undef PF_REGION
    uint8_t *s = (uint8_t *)scratch(o, op);
    if (!s) return 0;
    float *logits = (float *)(s + o_logits), *sel_w = (float *)(s + o_w), *yp = (float *)(s + o_yp);
    void *xh = s + o_xh, *xl = s + o_xl, *hh = s + o_hh, *hl = s + o_hl, *s16 = s + o_s16;
    uint32_t *lo_any = (uint32_t *)(s + o_nu) + 1;
    int32_t *sel_idx = (int32_t *)(s + o_idx), *list = (int32_t *)(s + o_list), *units = (int32_t *)(s + o_units),
            *n_units = (int32_t *)(s + o_nu);

    SepiaGpuBuf *ins[] = { L->router_w, L->router_bias, x, L->gate.buf, L->up.buf, L->down.buf, L->s_gate.buf,
                           L->s_up.buf, L->s_down.buf };
    for (size_t i = 0; i < sizeof ins / sizeof ins[0]; i++)
        if (ins[i] && !prep_in(ins[i], op)) return 0;
    if (!prep_out(y, op) || (route_out && !prep_out(route_out, op))) return 0;

    const float *rw = (const float *)(L->router_w->dev + L->router_w_off);
    const float *rb = (const float *)(L->router_bias->dev + L->router_bias_off);
    int64_t ld = H, hid = H, inter = I, tt = T, ntot = n_tot;
    float rs = L->route_scale, gsc = L->global_scale;
    int32_t nr32 = nr, ns32 = ns, tk32 = tk, nsel32 = n_sel;
    void *a_rt[] = { &x->dev, &tt, &rw, &ld, &ntot, &hid, &logits };
    const int rt_m = g_opt_pf_route_m && ((((uintptr_t)x->dev | (uintptr_t)rw) & 15) == 0) && (ld % 4) == 0 && H % 128 == 0;
    if (rt_m ? !launch2(K_PF_ROUTE_M, (unsigned)((T + 15) / 16), (unsigned)((n_tot + 15) / 16), 64, 0, a_rt, op)
             : !launch2(K_PF_ROUTE, (unsigned)((T + 31) / 32), (unsigned)((n_tot + 31) / 32), 256, 0, a_rt, op))
        return 0;
    void *a_sel[] = { &logits, &rb, &nr32, &ns32, &tk32, &rs, &gsc, &sel_idx, &sel_w };
    if (!launch(K_PF_SELECT, (unsigned)T, 64, a_sel, op)) return 0;
    void *a_grp[] = { &sel_idx, &tt, &nr32, &ns32, &tk32, &list, &units, &n_units, &lo_any };
    if (!launch(K_PF_GROUP, 1, 1024, a_grp, op)) return 0;
    int64_t nseg = T * H / 16;
    void *a_sp[] = { &x->dev, &nseg, &xh, &xl, &s16, &lo_any };
    if (!launch(K_PF_SPLIT, (unsigned)((nseg + 255) / 256), 256, a_sp, op)) return 0;
    void *a_gu[] = { (void *)&g, (void *)&u, (void *)&sg, (void *)&su, &nr32, &nsel32, &inter, &hid, &xh, &xl, &s16,
                     &lo_any, &list, &units, &n_units, &hh, &hl };
    const int gu_mode = pf_type_int(g.type) && (ns == 0 || pf_type_int(sg.type)) ? g_opt_pf_gu : 0;
    const int gu_k = gu_mode == 2 ? K_PF_GATEUP_R : gu_mode == 1 ? K_PF_GATEUP_I : K_PF_GATEUP;
    const int64_t gu_rows = gu_mode == 2 ? 64 : 32;
    if (!launch2(gu_k, (unsigned)((I + gu_rows - 1) / gu_rows), (unsigned)umax, gu_mode == 1 ? 1024 : 512,
                 PF_LDS_BYTES, a_gu, op))
        return 0;
    void *a_dn[] = { (void *)&d, (void *)&sd, &nr32, &inter, &hid, &hh, &hl, &list, &units, &n_units, &yp };
    const int dn_r = g_opt_pf_dn && pf_type_int(d.type) && (ns == 0 || pf_type_int(sd.type));
    if (!launch2(dn_r ? K_PF_DOWN_R : K_PF_DOWN, (unsigned)(dn_r ? (H + 127) / 128 : (H + 63) / 64), (unsigned)umax,
                 512, PF_LDS_BYTES, a_dn, op))
        return 0;
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

/* The fused MoE layer / expert FFN (kernels/mq_fused.h): exactly MQ_CUS
 * workgroups, one per CU (the LDS it asks for admits no second), launched
 * only when the device has that many CUs and the occupancy query confirms
 * that every workgroup is resident at once -- its grid barriers rely on it.
 * Gate/up runs on waves 1.. (wave 0 is the control wave), down on every
 * wave; both phases share the workgroup size and the rings (ring bytes per
 * wave: what the LDS leaves after the phases' tables). */
typedef struct {
    MqGeo gu, dn;
    int32_t dn_wps_r, dn_wps_s;
    uint32_t o_sel, o_gred, o_xqh, o_dred, o_flag, o_rings;
} MqFuseGeo;
typedef struct {
    const float *rw;
    int64_t ld;
    const float *bias;
    const float *x;
    int32_t n_routed, n_shared, topk, fixed;
    float route_scale, global_scale;
    int64_t inter, hidden;
    float *logits;
    int32_t *sel_idx;
    float *sel_w;
    uint8_t *xq_h;
    float *ypart;
    uint32_t *cnt, *bar, *err;
    float *y;
} MqFuseIo;
typedef struct {
    MqFuseGeo geo;
    unsigned threads;
    size_t lds;
} MqFusePlan;
#define MQ_FSEL_BYTES 1024          /* the fused kernel's selection area: idx[64], w[64], flag */

/* Gate/up units of workgroup b of G (mirror of mq_gu_range in
 * kernels/mq_fused.h): the units whose first weight byte lies in
 * [b T / G, (b + 1) T / G), us shared units of ws bytes first, then ur
 * routed ones of wr bytes. */
static int64_t cdiv_pos(int64_t a, int64_t d) { return a <= 0 ? 0 : (a + d - 1) / d; }
static void mq_gu_range(int64_t us, int64_t ws, int64_t ur, int64_t wr, int64_t G, int64_t b, int64_t *ns,
                        int64_t *nr) {
    const int64_t S = us * ws, T = S + ur * wr;
    const int64_t lo = T * b / G, hi = T * (b + 1) / G;
    int64_t a0 = 0, a1 = 0;
    if (us > 0) {
        a0 = cdiv_pos(lo, ws);
        a1 = cdiv_pos(hi, ws);
        if (a0 > us) a0 = us;
        if (a1 > us) a1 = us;
    }
    int64_t b0 = cdiv_pos(lo - S, wr), b1 = cdiv_pos(hi - S, wr);
    if (b0 > ur) b0 = ur;
    if (b1 > ur) b1 = ur;
    *ns = a1 - a0;
    *nr = b1 - b0;
}

/* Steps of one phase for the busiest wave: n_items items of nq quads on nw
 * waves of P parts, 10 per step when the ring holds two or more steps. */
static int64_t mq_phase_cost(int mc, int64_t n_items, int64_t nq, int P, int nw, size_t ring) {
    const int C = nw / P;
    const int64_t spw = ((n_items + C - 1) / C) * ((nq + P - 1) / P);
    int64_t S = (int64_t)(ring / ((size_t)k_mq_words[mc] * 1024));
    if (S > 4) S = 4;
    if (S > spw) S = spw;
    return spw * ((S >= 2 || spw == 1) ? 10 : 16);
}

static int mq_fuse_plan(const MoeProj *g, const MoeProj *u, const MoeProj *d, const MoeProj *sg, const MoeProj *su,
                        const MoeProj *sd, int32_t topk, int32_t n_shared, int64_t H, int64_t I, int router,
                        MqFusePlan *fp) {
    static int told = 0;   /* a device or layer the fused launch cannot take: said once */
    MqFfnPlan pl;
    if (!g_opt_fuse || topk < 1 || !mq_ffn_plan(g, u, d, sg, su, sd, topk, n_shared, H, I, &pl)) return 0;
    if (g_cus < MQ_CUS) {
        if (!told++) LOG("fused MoE launch off: %d compute units (it needs %d)", g_cus, MQ_CUS);
        return 0;
    }
    if ((int64_t)topk * pl.dn_wps_r + (int64_t)n_shared * pl.dn_wps_s > MQ_CUS) return 0;
    const int kg = mq_code(g->type), kd = mq_code(d->type);
    int wg = k_mq_words[kg], wd = k_mq_words[kd];
    if (n_shared > 0 && k_mq_words[mq_code(sg->type)] > wg) wg = k_mq_words[mq_code(sg->type)];
    if (n_shared > 0 && k_mq_words[mq_code(sd->type)] > wd) wd = k_mq_words[mq_code(sd->type)];
    const int wmax = wg > wd ? wg : wd;
    const int64_t tiles_i = (I + 15) / 16, tiles_h = (H + 15) / 16;
    /* the most gate/up units any workgroup gets */
    int64_t nu_max = 0;
    for (int64_t b = 0; b < MQ_CUS; b++) {
        int64_t ns, nr;
        mq_gu_range(n_shared * tiles_i, 32 * (int64_t)(n_shared > 0 ? sg->row_bytes : 0), topk * tiles_i,
                    32 * (int64_t)g->row_bytes, MQ_CUS, b, &ns, &nr);
        if (ns + nr > nu_max) nu_max = ns + nr;
    }
    if (nu_max < 1) nu_max = 1;
    const int32_t dmin = (pl.dn_wps_r < pl.dn_wps_s || n_shared == 0) ? pl.dn_wps_r : pl.dn_wps_s;
    const int64_t dnk = (tiles_h + dmin - 1) / dmin;
    const int64_t nqg = H / 1024, nqd = I / 1024;
    int64_t best = -1;
    /* gate/up runs on the waves after the control wave (all of them without
     * a router), down on every wave; waves past the last full column of P
     * parts idle in that phase */
    for (int nw = 2; nw <= 16; nw++)
        for (int Pg = 1; Pg <= nw - router && Pg <= nqg; Pg++) {
            for (int Pd = 1; Pd <= nw && Pd <= nqd; Pd++) {
                size_t o = MQ_ZERO + mq_xq_bytes(H);
                const size_t o_sel = o;
                o += MQ_FSEL_BYTES;
                const size_t o_gred = o;
                o += (size_t)2 * nu_max * Pg * 64;
                const size_t o_xqh = align256(o);
                o = o_xqh + mq_xq_bytes(I);
                const size_t o_dred = o;
                o += (size_t)dnk * Pd * 64;
                const size_t o_flag = o;
                o += (size_t)dnk * 4;
                const size_t o_rings = align256(o);
                if (o_rings + (size_t)nw * wmax * 1024 > g_lds_max) continue;
                size_t ring = ((g_lds_max - o_rings) / (size_t)nw) & ~(size_t)1023;
                if (ring > (size_t)4 * wmax * 1024) ring = (size_t)4 * wmax * 1024;
                const int64_t cost = mq_phase_cost(kg, 2 * nu_max, nqg, Pg, nw - router, ring) +
                                     mq_phase_cost(kd, dnk, nqd, Pd, nw, ring);
                if (best < 0 || cost < best) {
                    best = cost;
                    MqFuseGeo *G = &fp->geo;
                    memset(G, 0, sizeof *G);
                    G->gu.P = Pg;
                    G->dn.P = Pd;
                    G->gu.ring = G->dn.ring = (int32_t)ring;
                    G->dn_wps_r = pl.dn_wps_r;
                    G->dn_wps_s = pl.dn_wps_s;
                    G->o_sel = (uint32_t)o_sel;
                    G->o_gred = (uint32_t)o_gred;
                    G->o_xqh = (uint32_t)o_xqh;
                    G->o_dred = (uint32_t)o_dred;
                    G->o_flag = (uint32_t)o_flag;
                    G->o_rings = (uint32_t)o_rings;
                    fp->threads = 64u * (unsigned)nw;
                    fp->lds = o_rings + (size_t)nw * ring;
                }
            }
        }
    if (best < 0) {
        if (!told++) LOG("fused MoE launch off: no geometry fits %zu bytes of LDS", g_lds_max);
        return 0;
    }
    /* every workgroup resident at once: at most one per CU by LDS, and the
     * device has MQ_CUS of them */
    int nb = 0;
    const hipError_t e = hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&nb, g_fn[K_MQ_MOE], (int)fp->threads,
                                                                             fp->lds);
    if (e != hipSuccess || nb < 1 || (int64_t)nb * g_cus < MQ_CUS) {
        if (!told++)
            LOG("fused MoE launch off: occupancy query %s, %d workgroups of %u threads and %zu bytes LDS per CU",
                hipGetErrorString(e), nb, fp->threads, fp->lds);
        return 0;
    }
    return 1;
}

/* Scratch of a fused launch after `base`: XQ(h) [n_slots][XQ of I], then the
 * down partial rows [n_slots][H] f32. */
static size_t mq_fuse_scratch(int n_slots, int64_t H, int64_t I) {
    return (((size_t)n_slots * mq_xq_bytes(I) + 255) & ~(size_t)255) + (size_t)n_slots * (size_t)H * 4;
}

static int mq_fuse_launch(const char *op, const MoeProj *g, const MoeProj *u, const MoeProj *d, const MoeProj *sg,
                          const MoeProj *su, const MoeProj *sd, MqFuseIo *io, uint8_t *scr, const MqFusePlan *fp) {
    io->xq_h = scr;
    io->ypart = (float *)(scr + (((size_t)(io->topk + io->n_shared) * mq_xq_bytes(io->inter) + 255) & ~(size_t)255));
    io->cnt = (uint32_t *)g_scratch + MQ_DN_CNT_OFF;
    io->bar = (uint32_t *)g_scratch + MQ_BAR_WORD;
    io->err = (uint32_t *)g_scratch + MQ_ERR_WORD;
    MqFuseGeo geo = fp->geo;
    void *args[] = { (void *)g, (void *)u, (void *)d, (void *)sg, (void *)su, (void *)sd, io, &geo };
    if (!launch_lds(K_MQ_MOE, MQ_CUS, fp->threads, fp->lds, args, op)) return 0;
    g_fused_pending = 1;
    return 1;
}

/* One expert's FFN as one launch of sepia_mq_ffn (kernels/mq_flow.h):
 * MQ_CUS workgroups of 16 waves, one per CU. Workgroup b owns gate/up units
 * [b U / G, (b + 1) U / G) (U = I / 16 units of 16 gate and 16 up rows) on
 * waves 0 .. ngu - 1 and down row groups on the next nd1 waves; workgroups
 * without units run down only (nd0 waves) and take dh row groups instead of
 * dl, chosen so that every workgroup streams about the same bytes. Geometry
 * per role as mq_geo: the fewest steps for the busiest wave, every step in
 * flight at the start where the LDS allows. Mirrors struct MqFlowGeo. */
typedef struct {
    MqGeo gu, d1, d0;
    int32_t ngu, nd1, nd0;
    int32_t dl, dh, drem;
    int32_t free_delay;
    uint32_t o_xqh, o_gred, o_dred, o_ctl, o_rings;
} MqFlowGeo;
typedef struct {
    const float *x;
    float *y;
    int64_t inter, hidden;
    uint8_t *xq_h;
    uint32_t *hcnt, *flags, *err;
} MqFlowIo;
#define MQ_FLOW_WAVES 16

/* Best split of n_items items of nq quads over at most max_waves waves with
 * rings from `budget` bytes: P parts, C columns, S stages. Cost: the
 * busiest wave's steps, each step not in flight at the start counted
 * `late` more. Returns the cost, or -1 when nothing fits. */
static int64_t mq_flow_role(int mc, int64_t n_items, int64_t nq, int max_waves, size_t budget, int64_t per_step,
                            int64_t late, int *Pb, int *Cb, int *Sb) {
    const size_t w1 = (size_t)k_mq_words[mc] * 1024;
    int64_t best = -1;
    for (int P = 1; P <= max_waves && P <= nq; P++)
        for (int C = 1; C * P <= max_waves && C <= n_items; C++) {
            const int64_t spw = ((n_items + C - 1) / C) * ((nq + P - 1) / P);
            int64_t S = spw < 4 ? spw : 4;
            while (S > 1 && (size_t)(C * P) * (size_t)S * w1 > budget) S--;
            if ((size_t)(C * P) * (size_t)S * w1 > budget) continue;
            const int64_t cost = per_step * spw + late * (spw - S);
            if (best < 0 || cost < best || (cost == best && C * P < *Pb * *Cb)) {
                best = cost;
                *Pb = P;
                *Cb = C;
                *Sb = (int)S;
            }
        }
    return best;
}

static int mq_flow_plan(const MoeProj *g, const MoeProj *u, const MoeProj *d, int64_t H, int64_t I, MqFlowGeo *G,
                        unsigned *threads, size_t *lds) {
    static int told = 0;
    if (!g_opt_flow || g->type != u->type || g->row_bytes != u->row_bytes || !mq_proj_ok(g, I) || !mq_proj_ok(u, I) ||
        !mq_proj_ok(d, H) || H % 256 || I % 256)
        return 0;
    if (g_cus < MQ_CUS) {
        if (!told++) LOG("flow FFN launch off: %d compute units (it needs %d)", g_cus, MQ_CUS);
        return 0;
    }
    const int kg = mq_code(g->type), kd = mq_code(d->type);
    const int64_t Gn = MQ_CUS, U = I / 16, D = H / 16;
    const int64_t n_unit = U < Gn ? U : Gn, n_free = Gn - n_unit, nu_max = (U + Gn - 1) / Gn;
    const int64_t wu = 32 * (int64_t)g->row_bytes, wd = 16 * (int64_t)d->row_bytes;
    /* down row groups: dl per workgroup with units, dh per other, one more
     * for the first drem workgroups */
    int64_t best = -1, dl = 0, dh = 0, drem = 0;
    for (int64_t l = 0; l * n_unit <= D; l++) {
        const int64_t R = D - l * n_unit;
        int64_t h = 0, r = R;
        if (n_free > 0) {
            h = R / n_free;
            r = R - h * n_free;
        } else if (R >= Gn) {
            continue;
        }
        int64_t c = nu_max * wu + (l + (r > 0)) * wd;
        if (n_free > 0 && (h + (r > 0)) * wd > c) c = (h + (r > 0)) * wd;
        if (best < 0 || c < best) {
            best = c;
            dl = l;
            dh = h;
            drem = r;
        }
    }
    if (best < 0) return 0;
    const int64_t items_d1 = dl + (drem > 0), items_d0 = n_free > 0 ? dh + (drem > 0) : 0;
    const int64_t nqg = H / 1024, nqd = I / 1024;
    memset(G, 0, sizeof *G);
    size_t o = MQ_ZERO + mq_xq_bytes(H);
    G->o_xqh = (uint32_t)align256(o);
    o = G->o_xqh + mq_xq_bytes(I);
    G->o_gred = (uint32_t)o;
    o += (size_t)2 * nu_max * MQ_FLOW_WAVES * 64;
    G->o_dred = (uint32_t)o;
    o += (size_t)(items_d1 > items_d0 ? items_d1 : items_d0) * MQ_FLOW_WAVES * 64;
    G->o_ctl = (uint32_t)o;
    o += 64;
    G->o_rings = (uint32_t)align256(o);
    if (G->o_rings >= g_lds_max) return 0;
    const size_t budget = g_lds_max - G->o_rings;
    const size_t wg1 = (size_t)k_mq_words[kg] * 1024, wd1 = (size_t)k_mq_words[kd] * 1024;
    /* workgroups with units: gate/up (critical: it gates every down wave)
     * and down waves share the 16 waves and the ring budget */
    int64_t bu = -1;
    for (int ngu = 1; ngu < MQ_FLOW_WAVES; ngu++) {
        /* the waves past the gate/up ones turn x into XQ: four lanes per
         * segment, at most 8 passes (MQ_XQP in kernels/mq_flow.h) */
        if (H / 16 > 8 * 16 * (MQ_FLOW_WAVES - ngu)) break;
        int Pg = 0, Cg = 0, Sg = 0;
        const int64_t cg = mq_flow_role(kg, 2 * nu_max, nqg, ngu, budget, 10, 6, &Pg, &Cg, &Sg);
        if (cg < 0 || Pg * Cg != ngu) continue;
        const size_t used = (size_t)ngu * (size_t)Sg * wg1;
        int Pd = 1, Cd = 0, Sd = 0;
        int64_t cd = 0;
        if (items_d1 > 0) {
            cd = mq_flow_role(kd, items_d1, nqd, MQ_FLOW_WAVES - ngu, budget - used, 4, 10, &Pd, &Cd, &Sd);
            if (cd < 0) continue;
        }
        if (bu < 0 || cg + cd < bu) {
            bu = cg + cd;
            G->gu.P = Pg;
            G->gu.ring = (int32_t)((size_t)Sg * wg1);
            G->ngu = ngu;
            G->d1.P = Pd;
            G->d1.ring = (int32_t)((size_t)(Sd > 0 ? Sd : 1) * wd1);
            G->nd1 = Pd * Cd;
        }
    }
    if (bu < 0) {
        if (!told++) LOG("flow FFN launch off: no geometry fits %zu bytes of LDS", g_lds_max);
        return 0;
    }
    size_t need = G->o_rings + (size_t)G->ngu * G->gu.ring + (size_t)G->nd1 * G->d1.ring;
    G->d0.P = 1;
    G->d0.ring = (int32_t)wd1;
    if (items_d0 > 0) {
        int P = 0, C = 0, S = 0;
        if (mq_flow_role(kd, items_d0, nqd, MQ_FLOW_WAVES, budget, 4, 10, &P, &C, &S) < 0) return 0;
        G->d0.P = P;
        G->d0.ring = (int32_t)((size_t)S * wd1);
        G->nd0 = P * C;
        const size_t n0 = G->o_rings + (size_t)G->nd0 * G->d0.ring;
        if (n0 > need) need = n0;
    }
    G->dl = (int32_t)dl;
    G->dh = (int32_t)dh;
    G->drem = (int32_t)drem;
    G->free_delay = g_opt_flow_delay;
    *threads = 64u * MQ_FLOW_WAVES;
    *lds = need;
    int nb = 0;
    const hipError_t e = hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&nb, g_fn[K_MQ_FFN], (int)*threads, *lds);
    if (e != hipSuccess || nb < 1 || (int64_t)nb * g_cus < MQ_CUS) {
        if (!told++)
            LOG("flow FFN launch off: occupancy query %s, %d workgroups of %u threads and %zu bytes LDS per CU",
                hipGetErrorString(e), nb, *threads, *lds);
        return 0;
    }
    return 1;
}

static int mq_flow_launch(const char *op, const MoeProj *g, const MoeProj *u, const MoeProj *d, int32_t expert,
                          int64_t H, int64_t I, const uint8_t *xdev, float *ydev, uint8_t *scr, const MqFlowGeo *fg,
                          unsigned threads, size_t lds) {
    MqFlowIo io;
    io.x = (const float *)xdev;
    io.y = ydev;
    io.inter = I;
    io.hidden = H;
    io.xq_h = scr;
    io.hcnt = (uint32_t *)g_scratch + MQ_FLOW_HCNT_WORD;
    io.flags = (uint32_t *)g_scratch + MQ_FLOW_FLAG_OFF;
    io.err = (uint32_t *)g_scratch + MQ_ERR_WORD;
    MqFlowGeo geo = *fg;
    void *args[] = { (void *)g, (void *)u, (void *)d, &expert, &io, &geo };
    if (!launch_lds(K_MQ_FFN, MQ_CUS, threads, lds, args, op)) return 0;
    g_fused_pending = 1;
    return 1;
}

/* The MoE decode's gate/up as one launch of sepia_mq_gateup_mix
 * (kernels/mq_mix.h): MQ_CUS workgroups of 16 waves; wave 0 selects, waves
 * 1..15 stream. Workgroup b takes shared units [b us / G, (b + 1) us / G)
 * and routed units up to about T (b + 1) / G bytes in all (a unit: 16 rows
 * of one slot's gate and up). Mirrors struct MqMixGeo. */
typedef struct {
    MqGeo gu;
    uint32_t o_sel, o_ctl, o_gred, o_rings;
    int32_t nstream;
} MqMixGeo;
static int64_t mq_mix_rbefore(int64_t us, int64_t ws, int64_t ur, int64_t wr, int64_t G, int64_t b) {
    const int64_t T = us * ws + ur * wr;
    const int64_t f = T * b / G - (b * us / G) * ws;
    const int64_t r = f <= 0 ? 0 : f / wr;
    return r < ur ? r : ur;
}
static int mq_mix_plan(const MoeProj *g, const MoeProj *sg, int32_t topk, int32_t n_shared, int64_t H, int64_t I,
                       MqMixGeo *G, unsigned *threads, size_t *lds) {
    if (!g_opt_mix || topk < 1 || H / 16 > 8 * 15 * 16 || I % 16) return 0;
    const int64_t Gn = MQ_CUS, tiles_i = I / 16, us = (int64_t)n_shared * tiles_i, ur = (int64_t)topk * tiles_i;
    const int64_t ws = n_shared > 0 ? 32 * (int64_t)sg->row_bytes : 0, wr = 32 * (int64_t)g->row_bytes;
    const int64_t T = us * ws + ur * wr;
    /* the routed split is monotone when no workgroup's shared units outweigh its byte share */
    if (T / Gn < ws * ((us + Gn - 1) / Gn)) return 0;
    int64_t nu_max = 1;
    for (int64_t b = 0; b < Gn; b++) {
        const int64_t ns = (b + 1) * us / Gn - b * us / Gn;
        const int64_t nr = mq_mix_rbefore(us, ws, ur, wr, Gn, b + 1) - mq_mix_rbefore(us, ws, ur, wr, Gn, b);
        if (nr < 0) return 0;
        if (ns + nr > nu_max) nu_max = ns + nr;
    }
    int wmax = k_mq_words[mq_code(g->type)];
    if (n_shared > 0 && k_mq_words[mq_code(sg->type)] > wmax) wmax = k_mq_words[mq_code(sg->type)];
    const size_t wm = (size_t)wmax * 1024;
    const int64_t nq = H / 1024;
    memset(G, 0, sizeof *G);
    size_t o = MQ_ZERO + mq_xq_bytes(H);
    G->o_sel = (uint32_t)align256(o);
    G->o_ctl = G->o_sel + MQ_FSEL_BYTES;
    G->o_gred = G->o_ctl + 64;
    int64_t best = -1;
    for (int P = 1; P <= 15 && P <= nq; P++) {
        if (g_opt_mq_p && P != g_opt_mq_p) continue;
        const int C = g_opt_mq_c && g_opt_mq_c * P <= 15 ? g_opt_mq_c : 15 / P;
        const size_t o_rings = align256((size_t)G->o_gred + (size_t)2 * nu_max * P * 64);
        if (o_rings + (size_t)(P * C) * wm > g_lds_max) continue;
        size_t ring = ((g_lds_max - o_rings) / (size_t)(P * C)) & ~(size_t)1023;
        if (ring > 4 * wm) ring = 4 * wm;
        const int64_t spw = ((2 * nu_max + C - 1) / C) * ((nq + P - 1) / P);
        const int64_t S = (int64_t)(ring / wm);
        const int64_t cost = spw * ((S >= 2 || spw == 1) ? 10 : 16);
        if (best < 0 || cost < best) {
            best = cost;
            G->gu.P = P;
            G->gu.ring = (int32_t)ring;
            G->o_rings = (uint32_t)o_rings;
            G->nstream = P * C;
            *lds = o_rings + (size_t)(P * C) * ring;
        }
    }
    if (best < 0) return 0;
    *threads = 1024;
    return 1;
}

/* The MoE decode's down as one launch of sepia_mq_down_rows
 * (kernels/mq_rows.h): MQ_CUS workgroups of 16 waves; workgroup b owns row
 * groups [b T / G, (b + 1) T / G) of every slot, with every slot's XQ(h) in
 * its LDS; routed and shared rows stream on their own waves at once. The
 * split of waves and ring stages: the fewest steps for the busier role, then
 * the most stages. Mirrors struct MqRowsGeo. */
typedef struct {
    MqGeo gr, gs;
    int32_t nwr, nws;
    uint32_t o_red, o_rings_s;
} MqRowsGeo;
static int mq_rows_plan(const MoeProj *d, const MoeProj *sd, int32_t topk, int32_t n_shared, int64_t H, int64_t I,
                        MqRowsGeo *G, unsigned *threads, size_t *lds) {
    const int n_slots = topk + n_shared;
    if (!g_opt_dnrows || topk < 1 || n_slots < 2 || topk > 64 || H % 16 || (I / 16) * n_slots > 4 * 1024) return 0;
    const int64_t T = H / 16, nrg = (T + MQ_CUS - 1) / MQ_CUS, nq = I / 1024;
    const int kd = mq_code(d->type), ks = n_shared > 0 ? mq_code(sd->type) : kd;
    const size_t wr1 = (size_t)k_mq_words[kd] * 1024, ws1 = (size_t)k_mq_words[ks] * 1024;
    const size_t xq_all = (size_t)n_slots * 4 * (size_t)I;
    int64_t best = -1, best_fl = 0;
    memset(G, 0, sizeof *G);
    for (int Pr = 1; Pr <= 16 && Pr <= nq; Pr++)
        for (int Cr = 1; Pr * Cr <= 16 && Cr <= topk * nrg; Cr++)
            for (int Ps = 1; Ps <= nq; Ps++)
                for (int Cs = (n_shared > 0 ? 1 : 0); Pr * Cr + Ps * Cs <= 16 && Cs <= n_shared * nrg; Cs++) {
                    const int nwr = Pr * Cr, nws = Ps * Cs;
                    const size_t o_red = align256(MQ_ZERO + xq_all + 256);   /* the experts just below */
                    const size_t o_rings =
                        align256(o_red + (size_t)topk * nrg * Pr * 64 + (size_t)n_shared * nrg * Ps * 64);
                    const size_t avail = g_lds_max;
                    if (o_rings + (size_t)nwr * wr1 + (size_t)nws * ws1 > avail) continue;
                    const int64_t spw_r = ((topk * nrg + Cr - 1) / Cr) * ((nq + Pr - 1) / Pr);
                    const int64_t spw_s = Cs ? ((n_shared * nrg + Cs - 1) / Cs) * ((nq + Ps - 1) / Ps) : 0;
                    /* stages: as many as the LDS holds, the same number for both roles */
                    int64_t S = 4;
                    while (S > 1 && o_rings + (size_t)nwr * S * wr1 + (size_t)nws * S * ws1 > avail) S--;
                    const int64_t spw = spw_r > spw_s ? spw_r : spw_s;
                    const int64_t cost = spw * ((S >= 2 || spw == 1) ? 10 : 16);
                    const int64_t fl = (int64_t)(nwr + nws) * S;
                    if (best < 0 || cost < best || (cost == best && fl > best_fl)) {
                        best = cost;
                        best_fl = fl;
                        G->gr.P = Pr;
                        G->gr.ring = (int32_t)(S * wr1);
                        G->gr.orings = (int32_t)o_rings;
                        G->gs.P = Ps;
                        G->gs.ring = (int32_t)(S * ws1);
                        G->nwr = nwr;
                        G->nws = nws;
                        G->o_red = (uint32_t)o_red;
                        G->o_rings_s = (uint32_t)(o_rings + (size_t)nwr * S * wr1);
                        *lds = G->o_rings_s + (size_t)nws * S * ws1;
                    }
                }
    if (best < 0) return 0;
    *threads = 1024;
    return 1;
}

/* The SwiGLU expert FFN over n_slots = topk + n_shared slots: routed slot s
 * uses expert sel_idx[s] (or fixed + s when sel_idx is NULL), then come the
 * shared experts. One slot without weights stores y; several slots add
 * sel_w[s] * their output into y. Uses the matrix-core kernels when the
 * formats and shapes fit, else the tile kernels, else the generic
 * one-wave-per-row kernels. scr: scratch for the slots' f32 h vectors. */
static int ffn_launch(const char *op, const MoeProj *g, const MoeProj *u, const MoeProj *d, const MoeProj *sg,
                      const MoeProj *su, const MoeProj *sd, const int32_t *sel_idx, const float *sel_w, int32_t fixed,
                      int32_t topk, int32_t n_shared, int64_t H, int64_t I, const uint8_t *xdev, float *ydev,
                      uint8_t *scr, const MqRoute *route) {
    int32_t n_slots = topk + n_shared;
    int64_t inter = I, hid = H;
    MqFfnPlan pl;
    if (mq_ffn_plan(g, u, d, sg, su, sd, topk, n_shared, H, I, &pl)) {
        int32_t inter32 = (int32_t)I;
        float *h = (float *)scr;
        float *ypart = (float *)(scr + (size_t)n_slots * (size_t)I * 4);
        uint32_t *cnt = (uint32_t *)g_scratch + MQ_DN_CNT_OFF;
        MqRoute rt;
        memset(&rt, 0, sizeof rt);
        if (route) rt = *route;
        MqMixGeo mg;
        unsigned mix_threads;
        size_t mix_lds;
        if (route && mq_mix_plan(g, sg, topk, n_shared, H, I, &mg, &mix_threads, &mix_lds)) {
            void *a_mx[] = { (void *)g, (void *)u, (void *)sg, (void *)su, &rt, &topk, &n_shared, &inter32, &xdev, &h,
                             &mg };
            if (!launch_lds(K_MQ_GU_MIX, MQ_CUS, mix_threads, mix_lds, a_mx, op)) return 0;
        } else {
            void *a_gu[] = { (void *)g, (void *)u, (void *)sg, (void *)su, &sel_idx, &fixed, &topk, &inter32,
                             &pl.gu_wps_r, &pl.gu_wps_s, &xdev, &h, &pl.gu_geo, &rt, &pl.gu_hxq };
            if (!launch_lds(K_MQ_GU, pl.gu_grid, pl.gu_threads, pl.gu_lds, a_gu, op)) return 0;
        }
        MqRowsGeo rg;
        unsigned rows_threads;
        size_t rows_lds;
        if (sel_idx && sel_w && mq_rows_plan(d, sd, topk, n_shared, H, I, &rg, &rows_threads, &rows_lds)) {
            void *a_rw[] = { (void *)d, (void *)sd, &sel_idx, &sel_w, &topk, &n_shared, &inter32, &hid, &h, &ydev, &rg };
            return launch_lds(K_MQ_DN_ROWS, MQ_CUS, rows_threads, rows_lds, a_rw, op);
        }
        void *a_dn[] = { (void *)d, (void *)sd, &sel_idx, &sel_w, &fixed, &topk, &n_shared, &inter32, &hid, &h, &ydev,
                         &pl.dn_geo, &pl.dn_wps_r, &pl.dn_wps_s, &ypart, &cnt };
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

int sepia_gpu_moe_decode(const SepiaMoeLayerDesc *L, SepiaGpuBuf *x, SepiaGpuBuf *y, SepiaGpuBuf *route_out) {
    const char *op = "moe_decode";
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
    const size_t need_f = mq_fuse_scratch(n_slots, H, I), need_s = ffn_scratch_bytes(n_slots, I, H);
    uint8_t *s = (uint8_t *)scratch(o_h + (need_f > need_s ? need_f : need_s), op);
    if (!s) return 0;
    float *logits = (float *)(s + o_logits), *sel_w = (float *)(s + o_w);
    int32_t *sel_idx = (int32_t *)(s + o_idx);
    uint32_t *counter = (uint32_t *)g_scratch;

    SepiaGpuBuf *ins[] = { L->router_w, L->router_bias, x, L->gate.buf, L->up.buf, L->down.buf, L->s_gate.buf,
                           L->s_up.buf, L->s_down.buf };
    for (size_t i = 0; i < sizeof ins / sizeof ins[0]; i++)
        if (ins[i] && !prep_in(ins[i], op)) return 0;
    if (!prep_out(y, op) || (route_out && !prep_out(route_out, op))) return 0;

    const float *rw = (const float *)(L->router_w->dev + L->router_w_off);
    const float *rb = (const float *)(L->router_bias->dev + L->router_bias_off);
    int64_t ld = H, hid = H;
    int32_t nr = L->n_routed, ns = L->n_shared, tk = L->topk;
    float rs = L->route_scale, gsc = L->global_scale;
    MqFusePlan fp;
    if (mq_fuse_plan(&g, &u, &d, &sg, &su, &sd, tk, ns, H, I, 1, &fp)) {
        MqFuseIo io;
        memset(&io, 0, sizeof io);
        io.rw = rw;
        io.ld = ld;
        io.bias = rb;
        io.x = (const float *)x->dev;
        io.n_routed = nr;
        io.n_shared = ns;
        io.topk = tk;
        io.route_scale = rs;
        io.global_scale = gsc;
        io.inter = I;
        io.hidden = H;
        io.logits = logits;
        io.sel_idx = sel_idx;
        io.sel_w = sel_w;
        io.y = (float *)y->dev;
        if (!mq_fuse_launch(op, &g, &u, &d, &sg, &su, &sd, &io, s + o_h, &fp)) return 0;
    } else {
    /* with the matrix-core FFN the gate/up launch selects from the logits;
     * otherwise the router's last workgroup does */
    MqFfnPlan pl;
    const int in_kernel = !g_opt_route_sel && mq_ffn_plan(&g, &u, &d, &sg, &su, &sd, tk, ns, H, I, &pl);
    int32_t select = !in_kernel;
    void *a_route[] = { &rw, &ld, &rb, &x->dev, &hid, &nr, &ns, &tk, &rs, &gsc, &logits, &sel_idx, &sel_w, &counter,
                        &select };
    if (!launch(K_MOE_ROUTE, (unsigned)n_tot, 256, a_route, op)) return 0;

    const MqRoute rt = { logits, rb, nr, ns, rs, gsc, sel_idx, sel_w };
    if (!ffn_launch(op, &g, &u, &d, &sg, &su, &sd, sel_idx, sel_w, 0, tk, ns, H, I, x->dev, (float *)y->dev, s + o_h,
                    in_kernel ? &rt : NULL))
        return 0;
    }

    if (route_out) {
        hipError_t e = hipMemcpyAsync(route_out->dev, sel_idx, (size_t)L->topk * 4, hipMemcpyDeviceToDevice, g_stream);
        if (e == hipSuccess)
            e = hipMemcpyAsync(route_out->dev + (size_t)L->topk * 4, sel_w, (size_t)n_slots * 4,
                               hipMemcpyDeviceToDevice, g_stream);
        if (e != hipSuccess) {
            LOG("%s: route_out copy failed: %s", op, hipGetErrorString(e));
            return 0;
        }
    }
    return 1;
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
    const size_t need_f = mq_fuse_scratch(1, hidden, inter), need_s = ffn_scratch_bytes(1, inter, hidden);
    uint8_t *scr = (uint8_t *)scratch(need_f > need_s ? need_f : need_s, op);
    if (!scr) return 0;
    if (!prep_in(gate->buf, op) || !prep_in(up->buf, op) || !prep_in(down->buf, op) || !prep_in(x, op) ||
        !prep_out(y, op))
        return 0;
    MqFlowGeo flg;
    unsigned fl_threads;
    size_t fl_lds;
    if (mq_flow_plan(&g, &u, &d, hidden, inter, &flg, &fl_threads, &fl_lds))
        return mq_flow_launch(op, &g, &u, &d, expert, hidden, inter, x->dev, (float *)y->dev, scr, &flg, fl_threads,
                              fl_lds);
    MqFusePlan fp;
    if (mq_fuse_plan(&g, &u, &d, &none, &none, &none, 1, 0, hidden, inter, 0, &fp)) {
        MqFuseIo io;
        memset(&io, 0, sizeof io);
        io.x = (const float *)x->dev;
        io.topk = 1;
        io.fixed = expert;
        io.inter = inter;
        io.hidden = hidden;
        io.y = (float *)y->dev;
        return mq_fuse_launch(op, &g, &u, &d, &none, &none, &none, &io, scr, &fp);
    }
    return ffn_launch(op, &g, &u, &d, &none, &none, &none, NULL, NULL, expert, 1, 0, hidden, inter, x->dev,
                      (float *)y->dev, scr, NULL);
}
