/* oracle/sepia_oracle.h -- CPU oracle for the quantized-weight hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (sepia_amd/, include/)
 * links, loads or calls this library; only tests/, __graft_entry__.smoke()
 * and bench.py's CPU-baseline leg do, and only as the checker or as the
 * timed CPU baseline.
 *
 * Every function restates the reference's CPU algorithm with the same
 * rounding order (compiled with -ffp-contract=off); each cites the
 * reference file:line it follows. Pinning status per function is listed in
 * sepia_oracle.c's header comment.
 */
#ifndef SEPIA_ORACLE_H
#define SEPIA_ORACLE_H
#include <stddef.h>
#include <stdint.h>

/* GGUF type ids (ggml enum ggml_type; reference src/quants.h:6-10 for the
 * ids it supports, tools/gguf_inspect.py:62-84 for Q2_K/Q3_K/IQ2_XXS). */
enum {
    ORC_T_F32 = 0, ORC_T_F16 = 1, ORC_T_Q8_0 = 8, ORC_T_Q2_K = 10, ORC_T_Q3_K = 11,
    ORC_T_Q4_K = 12, ORC_T_Q5_K = 13, ORC_T_Q6_K = 14, ORC_T_IQ2_XXS = 16,
    ORC_T_IQ2_XS = 17, ORC_T_IQ3_XXS = 18, ORC_T_IQ4_XS = 23,
};

int     orc_supported(int type);
int64_t orc_block_elems(int type);                /* 0 if unsupported */
size_t  orc_block_bytes(int type);                /* 0 if unsupported */
size_t  orc_row_bytes(int type, int64_t n);       /* 0 if unsupported or n % block != 0 */
float   orc_f16_to_f32(uint16_t h);

/* Installs a 256-entry IQ2_XXS codebook (little-endian u64 per entry). The
 * real table is not available offline; without one IQ2_XXS is unsupported. */
void    orc_set_iq2xxs_grid(const uint64_t *grid256);

/* 1 on success, 0 if the type is unsupported or n is not block-aligned. */
int orc_dequantize_row(int type, const void *src, float *dst, int64_t n);

/* y[o] = (float) sum_i (double)deq(W[o,i]) * (double)x[i], sequential in i.
 * threads > 1 splits rows over pthreads (identical results). 1 ok, 0 bad args. */
int orc_qlinear(int type, const void *w, int64_t out_dim, int64_t in_dim,
                const float *x, float *y, int threads);

/* f32 rows, double accumulate (router logits). */
void orc_linear_f32(const float *w, int64_t out_dim, int64_t in_dim, const float *x, float *y);

float orc_sigmoid(float x);
float orc_silu(float x);
float orc_logsigmoid(float x);
void  orc_silu_mul(const float *g, const float *u, float *z, int64_t n);

/* Router selection + mixing weights. logits: [n_routed + n_shared]; bias:
 * [n_routed]. idx: [topk]; weights: [topk + n_shared] (routed first).
 * orc_route_select = orc_route_topk then orc_route_weights. */
void orc_route_topk(const float *logits, const float *bias, int n_routed, int topk, int *idx);
void orc_route_weights(const float *logits, int n_routed, int n_shared, const int *idx, int topk,
                       double route_scale, double global_scale, float *weights);
void orc_route_select(const float *logits, const float *bias, int n_routed, int n_shared, int topk,
                      double route_scale, double global_scale, int *idx, float *weights);

/* One quantized expert: y = down(silu(gate x) * up x). */
int orc_expert_ffn(int t_gate, const void *gate, int t_up, const void *up, int t_down, const void *down,
                   int64_t hidden, int64_t inter, const float *x, float *y, int threads);

typedef struct {
    int64_t hidden, inter;
    int n_routed, n_shared, topk;
    double route_scale, global_scale;
    const float *router_w;       /* [n_routed + n_shared, hidden] f32 */
    const float *router_bias;    /* [n_routed] */
    int t_gate, t_up, t_down;    /* routed expert types */
    const void *const *gate;     /* [n_routed] pointers to [inter, hidden] quant rows */
    const void *const *up;
    const void *const *down;     /* [n_routed] pointers to [hidden, inter] quant rows */
    int ts_gate, ts_up, ts_down; /* shared expert types */
    const void *const *s_gate;   /* [n_shared] */
    const void *const *s_up;
    const void *const *s_down;
} OrcMoeLayer;

/* Full MoE decode layer for one token. If force_idx is non-NULL, those topk
 * indices replace the router's selection (weights are still computed from
 * the raw logits). logits_out [n_routed+n_shared], idx_out [topk],
 * w_out [topk+n_shared] may be NULL. 1 ok, 0 bad args. */
int orc_moe_layer(const OrcMoeLayer *L, const float *x, float *y, const int *force_idx,
                  float *logits_out, int *idx_out, float *w_out, int threads);

/* Attention (src/sepia.c attn_forward_chunk, in the split of the GPU ABI
 * src/sepia_gpu.h sepia_gpu_rel_project / sepia_gpu_banded_attn). */
void orc_rel_project(const float *r_vec, const float *rel_proj, float *rel_logits, int64_t T, int64_t H,
                     int64_t d_rel, int64_t rel_extent);
int orc_banded_attn(const float *q, const float *k, const float *v, const float *rel_logits, float *out,
                    const int64_t *kv_lo, const int64_t *kv_hi, const float *tau, int64_t T, int64_t H, int64_t Hkv,
                    int64_t Dh, int64_t rel_extent, int64_t q_pos_base, int64_t kv_dim, float inv_head_dim);

#endif
