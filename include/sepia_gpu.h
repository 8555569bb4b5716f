/* include/sepia_gpu.h -- the GPU symbol surface of SEPIA's engine, implemented
 * for AMD Instinct MI355X (gfx950) by libsepia_hip.so (sepia_amd/csrc/sepia_hip.c).
 *
 * Drop-in replacement for the reference's src/sepia_gpu.h: the same 30
 * functions with the same prototypes, argument meaning and error convention,
 * so src/sepia.c links against libsepia_hip.so instead of the Metal shim
 * (src/sepia_metal.m) or the stub (src/sepia_gpu_stub.c) without source
 * changes. Each declaration cites the reference line it replaces.
 *
 * Conventions (src/sepia_gpu.h:1-3):
 *   - every function returns 1 / a non-NULL pointer on success and 0 / NULL
 *     on failure after logging one "sepia: hip: ..." line to stderr; nothing
 *     ever exits -- the caller decides whether a failure is fatal;
 *   - single host thread only, no locking (src/sepia_metal.m:42-49);
 *   - ops run in issue order on one HIP stream; results are visible to the
 *     host after sepia_gpu_end().
 *
 * Memory model on a discrete GPU (the reference assumes unified memory):
 *   - sepia_gpu_alloc(len, 0) "shared" buffers have device memory plus a
 *     pinned host copy. host_ptr returns the host copy. Host writes are
 *     uploaded when an op that reads the buffer is issued; device results
 *     are downloaded by sepia_gpu_end().
 *   - sepia_gpu_alloc(len, 1) "private" buffers are device-only.
 *   - sepia_gpu_wrap_mmap copies the caller's read-only mapping into HBM
 *     once (weights stay resident); host_ptr returns the caller's base.
 *   - every operand range is bounds-checked against its buffer before a
 *     launch; an out-of-range request fails with 0 instead of reaching the GPU.
 */
#ifndef SEPIA_GPU_H
#define SEPIA_GPU_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* src/sepia_gpu.h:9 -- 1 once sepia_gpu_init has succeeded. */
int  sepia_gpu_available(void);
/* src/sepia_gpu.h:10 -- selects device 0, creates the stream and loads the
 * prebuilt gfx950 code object sepia_kernels.hsaco from `kernel_dir` (the
 * counterpart of compiling metal_dir's *.metal). 1 on success. */
int  sepia_gpu_init(const char *kernel_dir);
/* src/sepia_gpu.h:11 */
void sepia_gpu_shutdown(void);
/* src/sepia_gpu.h:12 -- device marketing name, NULL before init. */
const char *sepia_gpu_device_name(void);

typedef struct SepiaGpuBuf SepiaGpuBuf;     /* src/sepia_gpu.h:19 (opaque) */

/* src/sepia_gpu.h:33 -- base must be page-aligned; the bytes are copied into
 * a resident HBM buffer; the mapping is never freed here. */
SepiaGpuBuf *sepia_gpu_wrap_mmap(void *base, size_t len);
/* src/sepia_gpu.h:38 */
SepiaGpuBuf *sepia_gpu_alloc(size_t len, int gpu_private);
/* src/sepia_gpu.h:43 -- NULL is a no-op. Waits for the stream first. */
void sepia_gpu_free(SepiaGpuBuf *b);
/* src/sepia_gpu.h:48 -- host copy of a shared buffer, the wrapped base for a
 * wrap_mmap buffer, NULL for private buffers and NULL b. */
void *sepia_gpu_host_ptr(SepiaGpuBuf *b);
/* src/sepia_gpu.h:52 -- device virtual address, 0 for NULL b. */
uint64_t sepia_gpu_gpu_addr(SepiaGpuBuf *b);
/* src/sepia_gpu.h:61 -- x[i] += 0 over n_floats floats, synchronous. */
int sepia_gpu_selftest_touch(SepiaGpuBuf *buf, size_t n_floats);

/* src/sepia_gpu.h:86-88 -- batching. begin opens a batch (0 if one is open);
 * flush hands queued work to the GPU and keeps the batch open; end waits for
 * every queued op, downloads shared outputs and closes the batch. Every op
 * below requires an open batch. */
int sepia_gpu_begin(void);
int sepia_gpu_flush(void);
int sepia_gpu_end(void);

/* src/sepia_gpu.h:102 */
int sepia_gpu_rmsnorm(SepiaGpuBuf *w, SepiaGpuBuf *x, SepiaGpuBuf *y, int64_t rows, int64_t n, float eps);
/* src/sepia_gpu.h:108 */
int sepia_gpu_matvec(SepiaGpuBuf *w, SepiaGpuBuf *x, SepiaGpuBuf *y, int64_t out_dim, int64_t in_dim);
/* src/sepia_gpu.h:113 */
int sepia_gpu_silu_mul(SepiaGpuBuf *g, SepiaGpuBuf *u, SepiaGpuBuf *z, int64_t n);
/* src/sepia_gpu.h:116 */
int sepia_gpu_add(SepiaGpuBuf *a, SepiaGpuBuf *b, SepiaGpuBuf *out, int64_t n);
/* src/sepia_gpu.h:122 */
int sepia_gpu_softmax(SepiaGpuBuf *x, SepiaGpuBuf *y, int64_t rows, int64_t n);
/* src/sepia_gpu.h:128 */
int sepia_gpu_sconv(SepiaGpuBuf *w, SepiaGpuBuf *hist, SepiaGpuBuf *in, SepiaGpuBuf *out,
                    int64_t C, int64_t K, int64_t T);

/* src/sepia_gpu.h:147 -- y[o] = deq(W[o,:]) . x for W [out_dim, in_dim] of
 * GGUF type `ggml_type` starting at byte w_off of w. Types: Q8_0, Q2_K, Q3_K,
 * Q4_K, Q5_K, Q6_K, IQ2_XS, IQ3_XXS, IQ4_XS, and IQ2_XXS once a codebook is
 * installed (sepia_hip_set_iq2xxs_grid). f32 x, y and accumulation. */
int sepia_gpu_matvec_q(int ggml_type, SepiaGpuBuf *w, size_t w_off, SepiaGpuBuf *x, SepiaGpuBuf *y,
                       int64_t out_dim, int64_t in_dim);
/* src/sepia_gpu.h:160 -- n weights of raw blocks at raw_off -> n floats,
 * bit-identical to the reference's dequantize_row (also F16). */
int sepia_gpu_dequant_rows(int ggml_type, SepiaGpuBuf *raw, size_t raw_off, SepiaGpuBuf *out, int64_t n);

/* src/sepia_gpu.h:209 and :226 -- banded attention is outside this
 * library's scope (the quantized-weight path); both log and return 0. */
int sepia_gpu_rel_project(SepiaGpuBuf *r_vec, SepiaGpuBuf *rel_proj, SepiaGpuBuf *rel_logits,
                          int64_t T, int64_t H, int64_t d_rel, int64_t rel_extent);
int sepia_gpu_banded_attn(SepiaGpuBuf *q, SepiaGpuBuf *k, SepiaGpuBuf *v, SepiaGpuBuf *rel_logits,
                          SepiaGpuBuf *attn_out,
                          const int64_t *kv_lo, const int64_t *kv_hi, const float *tau,
                          int64_t T, int64_t H, int64_t Hkv, int64_t Dh, int64_t rel_extent,
                          int64_t q_pos_base, int64_t kv_dim, float inv_head_dim);

/* src/sepia_gpu.h:249-254 -- weight operand at a byte offset. */
int sepia_gpu_matvec_off(SepiaGpuBuf *w, size_t w_off, SepiaGpuBuf *x, SepiaGpuBuf *y, int64_t out_dim, int64_t in_dim);
int sepia_gpu_rmsnorm_off(SepiaGpuBuf *w, size_t w_off, SepiaGpuBuf *x, SepiaGpuBuf *y, int64_t rows, int64_t n, float eps);
int sepia_gpu_sconv_off(SepiaGpuBuf *w, size_t w_off, SepiaGpuBuf *hist, SepiaGpuBuf *in, SepiaGpuBuf *out,
                        int64_t C, int64_t K, int64_t T);
int sepia_gpu_rel_project_off(SepiaGpuBuf *r_vec, SepiaGpuBuf *rel_proj, size_t rel_proj_off, SepiaGpuBuf *rel_logits,
                              int64_t T, int64_t H, int64_t d_rel, int64_t rel_extent);
/* src/sepia_gpu.h:264 -- n floats, independent byte offsets. */
int sepia_gpu_copy(SepiaGpuBuf *src, size_t src_off, SepiaGpuBuf *dst, size_t dst_off, int64_t n);
/* src/sepia_gpu.h:272 */
int sepia_gpu_scale(float scale, SepiaGpuBuf *x, SepiaGpuBuf *y, int64_t n);
/* src/sepia_gpu.h:285 -- K-1 <= 15. */
int sepia_gpu_sconv_hist_roll(SepiaGpuBuf *hist, SepiaGpuBuf *in, int64_t C, int64_t K, int64_t T);

#ifdef __cplusplus
}
#endif
#endif
