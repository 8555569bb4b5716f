/* include/sepia_hip_ext.h -- additive entry points of libsepia_hip.so that have
 * no counterpart in the reference's src/sepia_gpu.h. Nothing here changes
 * the 30 drop-in functions; sepia.c keeps working without these.
 *
 * Same conventions as sepia_gpu.h: 1 / non-NULL on success, 0 / NULL after a
 * "sepia: hip: ..." log line on failure, single host thread, one stream,
 * every op needs an open batch.
 */
#ifndef SEPIA_HIP_EXT_H
#define SEPIA_HIP_EXT_H
#include "sepia_gpu.h"

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF type ids the reference's src/quants.h:6-10 lacks (ggml enum values,
 * reference tools/gguf_inspect.py:71-77). */
#define SEPIA_T_Q2_K    10
#define SEPIA_T_Q3_K    11
#define SEPIA_T_IQ2_XXS 16

/* One projection of a stack of experts: expert e's row-major quantized
 * matrix starts at byte off + e * stride of buf (GGUF stores routed experts
 * as one 3-D tensor, so the stride is uniform). */
typedef struct {
    SepiaGpuBuf *buf;
    size_t off;
    size_t stride;
    int ggml_type;
} SepiaExpertTensor;

/* One sparse MoE layer (reference src/sepia.c:1377-1470 and :3831-3974;
 * spec docs/architecture-notes.md:342-474). */
typedef struct {
    int64_t hidden;                 /* 6144 for Inkling */
    int64_t inter;                  /* moe_intermediate_size, 3072 */
    int n_routed, n_shared, topk;   /* 256, 2, 6 */
    float route_scale;              /* 8.0 */
    float global_scale;             /* per-layer ffn_gscale */
    SepiaGpuBuf *router_w;          /* f32 [n_routed + n_shared, hidden] */
    size_t router_w_off;
    SepiaGpuBuf *router_bias;       /* f32 [n_routed], selection only */
    size_t router_bias_off;
    SepiaExpertTensor gate, up;     /* routed, [inter, hidden] each */
    SepiaExpertTensor down;         /* routed, [hidden, inter] */
    SepiaExpertTensor s_gate, s_up; /* shared, [inter, hidden] */
    SepiaExpertTensor s_down;       /* shared, [hidden, inter] */
} SepiaMoeLayerDesc;

/* y = MoE(x) for one token, entirely on the GPU (router, selection, the
 * selected and shared experts, weighted sum) with no host round trip.
 * x, y: f32 [hidden] at offset 0. route_out (optional, may be NULL): receives
 * int32 idx[topk] followed by f32 w[topk + n_shared] (routed weights, then
 * shared gammas) -- the content of the reference's --route-log record. */
int sepia_gpu_moe_decode(const SepiaMoeLayerDesc *layer, SepiaGpuBuf *x, SepiaGpuBuf *y,
                         SepiaGpuBuf *route_out);

/* sepia_gpu_moe_decode with no allocation. No counterpart in the
 * reference: it is for callers that cannot allocate device memory -- code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc. Every scratch byte (router logits, selection, h, per-slot
 * partial rows, arrival counters) lives in one fixed array of 4 MiB per
 * device, part of the library's own device code; a C3 layer (hidden 6144,
 * inter 3072, 8 slots) needs about 0.36 MiB of it. A layer that needs more
 * is rejected (0 and a log line) before anything is queued. The caller
 * still passes inputs and outputs. The array keeps the last call's contents
 * and the call clears the counters it needs itself; calls that overlap on
 * one device (another stream, another thread) race on it. Results are those
 * of sepia_gpu_moe_decode, bit for bit. */
int sepia_hip_moe_decode_noalloc(const SepiaMoeLayerDesc *layer, SepiaGpuBuf *x, SepiaGpuBuf *y,
                                 SepiaGpuBuf *route_out);

/* The same layer for n_tokens tokens at once (prefill; reference
 * src/sepia.c:1377-1470 applied to each token): y[t] = MoE(x[t]) with each
 * token's routing exactly as sepia_gpu_moe_decode's up to the summation
 * order of the router's f32 dot products. Tokens are grouped by expert and
 * every expert's weights are read once per 32 tokens: a layer of Q2_K,
 * Q3_K and Q4_K projections on the int8 matrix cores (activations as 23-bit
 * digit planes, exact integer products), one of the real checkpoint's
 * formats (IQ2_XS, IQ3_XXS, IQ4_XS, Q5_K, Q6_K, Q8_0) on the f16 ones
 * (weights as exact f16 integer codes, activations as f16 hi + lo planes),
 * any other mix of Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ2_XS, IQ3_XXS, IQ4_XS on
 * the bf16 ones (weights and activations as bf16 hi + lo pairs), all with
 * f32 accumulation. Rows 4-byte aligned for the first two (else the bf16
 * kernels; Q8_0 has no other). x, y: f32 [n_tokens][hidden] at offset 0.
 * route_out (optional): int32 idx[n_tokens][topk] followed by f32
 * w[n_tokens][topk + n_shared]. */
int sepia_gpu_moe_prefill(const SepiaMoeLayerDesc *layer, int64_t n_tokens, SepiaGpuBuf *x, SepiaGpuBuf *y,
                          SepiaGpuBuf *route_out);

/* One routed expert: y = down(silu(gate x) * up x) for expert `expert` of
 * stacks holding n_experts experts (reference src/sepia.c:2993-3017,
 * real_expert_ffn), as two launches (fused gate/up/SwiGLU, then down).
 * x, y: f32 [hidden] at offset 0. */
int sepia_gpu_expert_ffn(const SepiaExpertTensor *gate, const SepiaExpertTensor *up, const SepiaExpertTensor *down,
                         int n_experts, int expert, int64_t hidden, int64_t inter, SepiaGpuBuf *x, SepiaGpuBuf *y);

/* Launch timing: between start and stop every launch is bracketed by a pair
 * of HIP events on the stream it runs on; stop waits for the stream and adds
 * each launch's duration to its kernel's total. query reads the totals of a
 * kernel by name (e.g. "sepia_moe_gateup"); reset clears them. Not for use
 * inside a stream capture. */
int sepia_hip_profile_start(void);
int sepia_hip_profile_stop(void);
int sepia_hip_profile_query(const char *kernel, int64_t *launches, double *total_ms);
void sepia_hip_profile_reset(void);

/* Benchmark and test support. Fills n_blocks blocks of `ggml_type` at byte
 * `off` of buf with seeded random bytes, then sets every f16 scale field of
 * each block to a value uniform in [lo, hi] (rounded to f16). */
int sepia_hip_synth_blocks(int ggml_type, SepiaGpuBuf *buf, size_t off, int64_t n_blocks,
                           uint64_t seed, float lo, float hi);

/* Installs the 256-entry IQ2_XXS codebook (u64 per entry, byte j = magnitude
 * of weight j). The real table is not available to this build; until one is
 * installed IQ2_XXS is rejected as unsupported. Needs init. */
int sepia_hip_set_iq2xxs_grid(const uint64_t *grid256);

/* Grows the library's scratch region (router logits, selections, h, partial
 * rows) to at least `bytes` now, so that later calls of the same or smaller
 * shapes allocate nothing. A call whose scratch would have to grow while the
 * stream is being captured fails instead (an allocation cannot be captured):
 * run the call once, or reserve, before beginning a capture. Needs init. */
int sepia_hip_reserve_scratch(size_t bytes);

/* Bytes of the library's growable scratch region (0 before its first use).
 * No counterpart in the reference. */
size_t sepia_hip_scratch_bytes(void);

/* Device and pinned-host allocations the library has made since it loaded
 * (hipMalloc, hipHostMalloc). No counterpart in the reference; tests of the
 * allocation-free entry check that it leaves the count unchanged. */
uint64_t sepia_hip_alloc_count(void);

/* Bytes copied from shared buffers' host copies to their device copies since
 * init. sepia_gpu_host_ptr marks every 64 KiB chunk of a shared buffer
 * host-written; each op then uploads the marked parts of exactly the range
 * it reads and unmarks the chunks that range covers whole, so a weight slab
 * filled once is uploaded once however many batches read it (tests read
 * this counter to check that), while bytes beside a range already read can
 * still be written through the pointer handed out earlier. */
uint64_t sepia_hip_uploaded_bytes(void);

/* The first device error a kernel recorded since the last call, 0 if none,
 * and clears it. A kernel records one when a bounded spin wait expires (code
 * 5): its launch's outputs are then invalid. sepia_gpu_end checks and
 * clears it itself and fails the batch (logging the code); callers that run
 * the library's launches without ending a batch (a captured graph replayed
 * on the library's stream) call this after synchronizing. No counterpart in
 * the reference, whose Metal kernels have no spin waits. */
unsigned sepia_hip_take_device_error(void);

/* Measurement support: one launch of `grid` workgroups that reads `bytes`
 * of buf from byte `off` (both multiples of 16) with plain streaming loads
 * and does nothing else, for the HBM read ceiling of a single launch at a
 * given size. No counterpart in the reference. */
int sepia_hip_read_probe(SepiaGpuBuf *buf, size_t off, size_t bytes, unsigned grid);
/* The same read through the decode kernels' staging path (no counterpart in
 * the reference; a measurement reference): grid workgroups of `threads`
 * threads, each wave streaming its steps of kb KB (kb wave-wide 16-byte LDS
 * DMAs) through a private ring of `stages` stages, waiting for the oldest
 * stage, reading it back and refilling it, with no compute. (kb, stages) is
 * one of (7,1) (7,2) (4,1) (4,2) (4,4) (2,4) (1,4); the rings must fit the
 * LDS. Kernel sepia_read_probe_dma. */
int sepia_hip_read_probe_dma(SepiaGpuBuf *buf, size_t off, size_t bytes, unsigned grid, unsigned threads, int kb,
                             int stages);

/* The hipStream_t every op is issued on (for hipEvent timing). */
void *sepia_hip_stream(void);

/* Kernel-selection switches for tests and tuning (returns 1 if name and
 * value are known):
 *   "mq" 1/0      the matrix-core kernels (matvec and expert FFN) for
 *                 Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_0, IQ2_XS, IQ3_XXS and
 *                 IQ4_XS (default 1);
 *   "tile" 1/0    the tile kernels where the matrix-core ones do not apply
 *                 (0 = the generic one-wave-per-row kernels);
 *   "tile_t" 0..  automatic or forced row steps per tile workgroup;
 *   "mq_p", "mq_c", "mq_s" 0..  automatic or forced matrix-core geometry
 *                 (parts per item, items side by side, ring stages);
 *   "mq_x" 0..4   how matrix-core kernels fetch their vector: 0 = the
 *                 planner's choice, 1 = loads from global memory, 2 = LDS
 *                 DMA issued ahead of the weight prologue, 3 = converter
 *                 waves (DMA into the XQ place, converted there while the
 *                 other waves issue and decode their first step), 4 = the
 *                 same conversion by the first stepping waves before they
 *                 issue their own weights (FFN gate/up launches only);
 *   "mq_scope" 0..3  the mq_p/mq_c/mq_s/mq_x overrides apply to every
 *                 matrix-core launch (0) or only to the matvec (1), the
 *                 expert FFN's gate/up (2) or its down (3) launches;
 *   "mq_rdelay" 0..4096  KB of weights a routed gate/up workgroup of the MoE
 *                 decode layer is charged for waiting on the selection when
 *                 workgroups are split between routed and shared experts
 *                 (default 80);
 *   "mq_gufac", "mq_dnfac" 25..400  percent scale on the routed formats'
 *                 relative decode cost in the gate/up and down splits
 *                 between routed and shared experts (default 100);
 *   "pf_q" 1/0    prefill projections of layers whose six projections are
 *                 all Q2_K/Q3_K/Q4_K on the int8 matrix cores (1, default),
 *                 or on the bf16 kernels (0);
 *   "pf_h" 1/0    prefill projections of layers whose six projections are
 *                 all in the real checkpoint's formats (IQ2_XS, IQ3_XXS,
 *                 IQ4_XS, Q5_K, Q6_K, Q8_0) with 4-byte-aligned rows on the
 *                 f16 matrix cores (1, default), or on the bf16 kernels (0;
 *                 they take no Q8_0, so such layers are then refused);
 *   "pf_route_m" 1/0  prefill router logits on the f32 matrix cores when x
 *                 and the router rows are 16-byte aligned (default 1). */
int sepia_hip_set_option(const char *name, int value);
/*   ("wait_ticks" 0..  the kernels' spin-wait bound in 100 MHz ticks; 0 =
 *                 the default 2 s. For tests of the expiry report.) */

/* ---- The on-disk stores straight into HBM -------------------------------
 * The reference reads resident-manifest.json + resident.bin (mmap'd) and
 * the sepia-index sidecar, then preads each routed expert from the GGUF
 * parts when it is used (src/sepia.c:1853-2104; docs/container.md:123-257).
 * Here both stores go to device memory once: resident.bin as one private
 * buffer, and every expert of a MoE layer into one private buffer per
 * layer, so the layer runs with no host reads. Parsing is host-only; the
 * uploads need sepia_gpu_init and run outside a batch (they synchronize the
 * library's stream). Failures log one line and return NULL/0. */

/* One tensor of resident-manifest.json. shape[0] is the fastest dimension
 * (GGUF order): a 2-D weight is [in_dim, out_dim], a stacked 3-D one
 * [in_dim, out_dim, n_stack]. */
typedef struct {
    const char *name;
    int ggml_type;
    int n_dims;
    int64_t shape[4];
    int64_t offset;     /* into resident.bin and its device copy */
    int64_t nbytes;
} SepiaResidentTensor;

typedef struct SepiaResidentTable SepiaResidentTable;

/* Replaces manifest_load (src/sepia.c:1876-1910): parses the manifest's
 * "tensors" array ({name, ggml_type, offset, nbytes, shape[1..4]}) and
 * checks every [offset, offset + nbytes) against resident_bin_path's size. */
SepiaResidentTable *sepia_hip_manifest_load(const char *manifest_path, const char *resident_bin_path);
size_t sepia_hip_manifest_count(const SepiaResidentTable *t);
const SepiaResidentTensor *sepia_hip_manifest_tensor(const SepiaResidentTable *t, size_t i);
/* Replaces resident_find (src/sepia.c:1912-1916): the first tensor of that
 * name, NULL if none. */
const SepiaResidentTensor *sepia_hip_manifest_find(const SepiaResidentTable *t, const char *name);
/* resident.bin into one private device buffer (the manifest's offsets hold
 * in it); the reference mmaps the file instead (src/sepia.c:2655-2670). */
SepiaGpuBuf *sepia_hip_manifest_upload(const SepiaResidentTable *t);
void sepia_hip_manifest_free(SepiaResidentTable *t);

/* One routed expert's slice of a GGUF part (struct ExpertSlot,
 * src/sepia.c:1995-2000). */
typedef struct {
    int part_idx;
    int64_t abs_offset;
    int64_t nbytes;
    int ggml_type;
} SepiaExpertSlot;

typedef struct SepiaExpertIndex SepiaExpertIndex;

/* Replaces index_load (src/sepia.c:2036-2080): n_experts_per_layer, the
 * parts[] file list and every moe_layers{} layer's gate/up/down "experts"
 * arrays of {part_file, abs_offset, nbytes, ggml_type}. */
SepiaExpertIndex *sepia_hip_index_load(const char *index_path);
int sepia_hip_index_n_experts(const SepiaExpertIndex *idx);
int sepia_hip_index_n_parts(const SepiaExpertIndex *idx);
const char *sepia_hip_index_part(const SepiaExpertIndex *idx, int i);
/* 1 if the index has this MoE layer. */
int sepia_hip_index_has_layer(const SepiaExpertIndex *idx, int layer);
/* The slice of (layer, kind 0 gate / 1 up / 2 down, expert); 0 if absent. */
int sepia_hip_index_slot(const SepiaExpertIndex *idx, int layer, int kind, int expert, SepiaExpertSlot *out);
/* Every expert of one layer's gate, up and down from the GGUF parts under
 * gguf_dir (NULL: "inkling-gguf" beside the index file, as the reference
 * derives it, src/sepia.c:1823-1834) into one private device buffer: the
 * three stacks back to back, expert e of kind k at out[k].off + e *
 * out[k].stride. The slices of one kind must share their type and size;
 * runs of experts that lie back to back in a part are read as one range.
 * Replaces the reference's per-use pread (docs/container.md:245-252). */
SepiaGpuBuf *sepia_hip_index_upload_layer(const SepiaExpertIndex *idx, const char *gguf_dir, int layer,
                                          SepiaExpertTensor out[3]);
void sepia_hip_index_free(SepiaExpertIndex *idx);

/* A MoE layer's descriptor from the two stores, resolving what the
 * reference's real_load does per layer (src/sepia.c:2770-2777):
 * blk.<layer>.ffn_gate_inp.weight (f32 router [hidden, n_routed + n_shared]),
 * exp_probs_b.bias (f32 [n_routed]), ffn_gscale.weight (f32 [1], read from
 * resident.bin into global_scale), ffn_{gate,up,down}_shexp.weight (shared
 * stacks, n_shared = their stack count; absent: no shared experts) in the
 * resident upload, and the routed experts of upload_layer. hidden and inter
 * come from the shapes, and every matrix's bytes are checked against them.
 * 1 on success. */
int sepia_hip_moe_layer_from_stores(const SepiaResidentTable *t, SepiaGpuBuf *resident, int layer,
                                    const SepiaExpertTensor experts[3], int n_routed, int topk, float route_scale,
                                    SepiaMoeLayerDesc *out);

#ifdef __cplusplus
}
#endif
#endif
