// mv.h -- full-row tile matvec for quantized rows (decode, batch 1).
//
// A 384-thread workgroup owns S*J whole rows. The row's U = in_dim / 64
// units (64-weight pieces of a block) are spread over U lanes and each lane
// keeps its unit's x planes in registers while it walks J rows, S rows per
// step (S = 384 / U; U must divide 384: 3072, 4096 and 6144 columns give
// U = 48, 64, 96). Per workgroup:
//   1. the lane issues the loads of its unit for all J rows;
//   2. while they are in flight the workgroup stages x in LDS in XP form
//      (qdot.h) -- or, when x already comes in XP form from the previous
//      kernel, reads it from there;
//   3. integer unit dots (qdot.h), a butterfly over the `seg` lanes of the
//      row that share a wave, then a short LDS sum across waves.
// Rows never span workgroups, so no workgroup waits for or talks to another.
#pragma once
#include "common.h"
#include "qdot.h"

#ifndef MV_NT
#define MV_NT 384
#endif

struct MvGeo {
    int32_t U;     // units per row
    int32_t S;     // rows per step (384 / U)
    int32_t seg;   // lanes per in-wave partial sum (largest power of two dividing U, <= 64)
    int32_t pad;
};

// LDS carve-up: x planes (3n bytes), scales and sums (n/16 floats each),
// row partials (S * J * (U / seg) floats), then scratch floats.
struct MvSmem {
    int8_t *planes;
    float *scale, *sum, *red, *extra;
};
__device__ __forceinline__ MvSmem mv_smem(uint8_t *base, int64_t n, int rows_red) {
    MvSmem m;
    m.planes = (int8_t *)base;
    m.scale = (float *)(base + 3 * n);
    m.sum = m.scale + n / 16;
    m.red = m.sum + n / 16;
    m.extra = m.red + ((rows_red + 3) & ~3);   // keep extra 16-byte aligned
    return m;
}

// x staging is split in two so that x's loads are issued before the weight
// loads: a wave's loads retire in order, so a wait for x issued after the
// weights would also wait for every weight. Each thread holds up to MV_XQ
// quads (n <= 4 * 384 * MV_XQ = 9216 columns).
#ifndef MV_XQ
#define MV_XQ 6
#endif
struct XQuads {
    float4 v[MV_XQ];
};

__device__ __forceinline__ void mv_load_x(const float *__restrict__ x, int64_t n, XQuads &xq) {
    const float4 *x4 = (const float4 *)x;
#pragma unroll
    for (int p = 0; p < MV_XQ; p++) {
        const int64_t q = threadIdx.x + (int64_t)p * MV_NT;
        xq.v[p] = q < n / 4 ? x4[q] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
}

// The loaded quads -> XP in LDS (n a multiple of 16, so each 4-lane segment
// group is entirely inside or outside the vector).
__device__ __forceinline__ void mv_stage_x(const XQuads &xq, int64_t n, const MvSmem &m) {
#pragma unroll
    for (int p = 0; p < MV_XQ; p++) {
        const int64_t q = threadIdx.x + (int64_t)p * MV_NT;
        if (q < n / 4) xp_quad(xq.v[p], q, m.planes, m.scale, m.sum, n);
    }
}

template <int T, int J>
__device__ __forceinline__ void mv_issue(const uint8_t *__restrict__ W, uint64_t row_bytes, int64_t rows,
                                         int64_t r0, const MvGeo &g, typename QU<T>::Data (&d)[J]) {
    const int t = threadIdx.x, u = t % g.U, s = t / g.U;
    const uint64_t col_off = (uint64_t)(u >> 2) * QU<T>::bytes;
#pragma unroll
    for (int j = 0; j < J; j++) {
        int64_t r = r0 + (int64_t)j * g.S + s;
        r = r < rows ? r : rows - 1;
        d[j] = QU<T>::load(W + (uint64_t)r * row_bytes + col_off, u & 3);
    }
}

// Unit dots of J rows, summed over the row's lanes within each wave; the
// first lane of each `seg` group stores its partial at red[(j*S + s) * nseg + u/seg].
template <int T, int J>
__device__ __forceinline__ void mv_partials(const typename QU<T>::Data (&d)[J], const XU &X, const MvGeo &g,
                                            float *red) {
    const int t = threadIdx.x, u = t % g.U, s = t / g.U;
    const int nseg = g.U / g.seg;
#pragma unroll
    for (int j = 0; j < J; j++) {
        float a = QU<T>::dot(d[j], u & 3, X);
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1)
            if (off < g.seg) a += __shfl_xor(a, off, SEPIA_WAVE);
        if ((u & (g.seg - 1)) == 0) red[(j * g.S + s) * nseg + u / g.seg] = a;
    }
}

// Row rr (0 <= rr < S*J) of the tile from the partials.
__device__ __forceinline__ float mv_row_sum(const float *red, int rr, const MvGeo &g) {
    const int nseg = g.U / g.seg;
    float s = 0.0f;
    for (int i = 0; i < nseg; i++) s += red[rr * nseg + i];
    return s;
}

// y = W x for one quantized matrix; grid = ceil(rows / (S*J)).
template <int T, int J>
__device__ __forceinline__ void mv_full_body(const uint8_t *__restrict__ W, uint64_t row_bytes, int64_t rows,
                                             int64_t n, MvGeo g, const float *__restrict__ x,
                                             float *__restrict__ y) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const MvSmem m = mv_smem(smem, n, g.S * J * (g.U / g.seg));
    const int64_t r0 = (int64_t)blockIdx.x * g.S * J;
    XQuads xq;
    mv_load_x(x, n, xq);
    typename QU<T>::Data d[J];
    mv_issue<T, J>(W, row_bytes, rows, r0, g, d);
    mv_stage_x(xq, n, m);
    __syncthreads();
    XU X;
    const int u = threadIdx.x % g.U;
    load_xu<T>(XPView{m.planes, m.scale, m.sum, n}, u >> 2, u & 3, X);
    mv_partials<T, J>(d, X, g, m.red);
    __syncthreads();
    const int rr = threadIdx.x;
    if (rr < g.S * J && r0 + rr < rows) y[r0 + rr] = mv_row_sum(m.red, rr, g);
}

#define SEPIA_MV_KERNEL(name, T, J)                                                                 \
    extern "C" __global__ __launch_bounds__(MV_NT) void sepia_mv_##name##_j##J(                   \
        const uint8_t *__restrict__ W, uint64_t row_bytes, int64_t rows, int64_t n, MvGeo g,      \
        const float *__restrict__ x, float *__restrict__ y) {                                     \
        mv_full_body<T, J>(W, row_bytes, rows, n, g, x, y);                                       \
    }

// ------------------------------------------------------------------ FFN ---
// One projection family of a stack of experts: expert e's quant rows start
// at base + e * stride, row r at + r * row_bytes.
struct MoeProj {
    const uint8_t *base;
    uint64_t stride;
    uint64_t row_bytes;
    int64_t n_blocks;
    int32_t type;
    int32_t pad;
};

// Per-slot XP arrays of the SwiGLU activations h (inter columns each).
struct HxpArgs {
    int8_t *planes;   // [slot][3][inter]
    float *scale;     // [slot][inter / 16]
    float *sum;       // [slot][inter / 16]
};

__device__ __forceinline__ int64_t slot_expert(const int32_t *sel_idx, int32_t fixed, int32_t slot, int32_t topk) {
    return slot < topk ? (sel_idx ? (int64_t)sel_idx[slot] : (int64_t)fixed + slot) : (int64_t)(slot - topk);
}

// h[slot, i] = silu(gate_i . x) * (up_i . x) for S*J rows i of one slot; h is
// written in XP form (S*J is a multiple of 16, so the tile holds whole
// segments) and, if h32 is set, as f32.
template <int T, int J>
__device__ __forceinline__ void ffn_gateup_tile(const MoeProj &G, const MoeProj &Up, int64_t e, int64_t inter,
                                                int64_t hidden, MvGeo g, int32_t slot, int64_t r0,
                                                const float *__restrict__ x, const HxpArgs &hx,
                                                float *__restrict__ h32, const MvSmem &m) {
    const uint8_t *wg = G.base + e * G.stride, *wu = Up.base + e * Up.stride;
    XQuads xq;
    mv_load_x(x, hidden, xq);
    typename QU<T>::Data dg[J], du[J];
    mv_issue<T, J>(wg, G.row_bytes, inter, r0, g, dg);
    mv_issue<T, J>(wu, Up.row_bytes, inter, r0, g, du);
    mv_stage_x(xq, hidden, m);
    __syncthreads();
    XU X;
    const int u = threadIdx.x % g.U;
    load_xu<T>(XPView{m.planes, m.scale, m.sum, hidden}, u >> 2, u & 3, X);
    const int nred = g.S * J * (g.U / g.seg);
    mv_partials<T, J>(dg, X, g, m.red);
    mv_partials<T, J>(du, X, g, m.red + nred);
    __syncthreads();
    const int rr = threadIdx.x;
    float *hv = m.extra;                                   // S*J activations of this tile
    if (rr < g.S * J) {
        const float gv = mv_row_sum(m.red, rr, g);
        const float uv = mv_row_sum(m.red + nred, rr, g);
        const float hval = (r0 + rr < inter) ? silu_f32(gv) * uv : 0.0f;
        hv[rr] = hval;
        if (h32 && r0 + rr < inter) h32[(int64_t)slot * inter + r0 + rr] = hval;
    }
    __syncthreads();
    const int q = threadIdx.x;                             // one quad of h per thread
    if (q < g.S * J / 4 && r0 + 4 * q < inter) {
        const float4 v = *(const float4 *)&hv[4 * q];
        xp_quad(v, r0 / 4 + q, hx.planes + (int64_t)slot * 3 * inter, hx.scale + (int64_t)slot * (inter / 16),
                hx.sum + (int64_t)slot * (inter / 16), inter);
    }
}

// grid = n_slots * ceil(inter / (S*J)). Routed slots (< topk) take their
// expert from sel_idx (or fixed_expert + slot); later slots are the shared
// experts. Workgroups with blockIdx < zero_blocks also clear y_zero[0..y_n).
extern "C" __global__ __launch_bounds__(MV_NT) void sepia_ffn_gateup(
    MoeProj gate, MoeProj up, MoeProj s_gate, MoeProj s_up, const int32_t *__restrict__ sel_idx,
    int32_t fixed_expert, int32_t topk, int64_t inter, int64_t hidden, MvGeo g, int32_t J,
    const float *__restrict__ x, HxpArgs hx, float *__restrict__ h32, float *__restrict__ y_zero, int64_t y_n) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    if (y_zero) {
        for (int64_t i = (int64_t)blockIdx.x * MV_NT + threadIdx.x; i < y_n; i += (int64_t)gridDim.x * MV_NT)
            y_zero[i] = 0.0f;
    }
    const int64_t rows_per = (int64_t)g.S * J;
    const int64_t tiles = (inter + rows_per - 1) / rows_per;
    const int32_t slot = (int32_t)(blockIdx.x / tiles);
    const int64_t r0 = (blockIdx.x % tiles) * rows_per;
    const bool routed = slot < topk;
    const MoeProj &G = routed ? gate : s_gate;
    const MoeProj &U = routed ? up : s_up;
    const int64_t e = slot_expert(sel_idx, fixed_expert, slot, topk);
    // the red area holds the gate and the up partials; extra follows both
    const MvSmem mm = mv_smem(smem, hidden, 2 * g.S * J * (g.U / g.seg));
#define GU_CASE(TT, JJ)                                                                          \
    if (G.type == TT && J == JJ) {                                                               \
        ffn_gateup_tile<TT, JJ>(G, U, e, inter, hidden, g, slot, r0, x, hx, h32, mm);            \
        return;                                                                                  \
    }
    GU_CASE(ST_Q2_K, 2) GU_CASE(ST_Q2_K, 4) GU_CASE(ST_Q3_K, 2) GU_CASE(ST_Q3_K, 4)
    GU_CASE(ST_Q4_K, 2) GU_CASE(ST_Q4_K, 4)
#undef GU_CASE
}

// y[d] (+)= w_slot * (down_slot[d, :] . h_slot) for S*J rows d of one slot,
// with h_slot read in XP form from global memory.
template <int T, int J>
__device__ __forceinline__ void ffn_down_tile(const MoeProj &P, int64_t e, int64_t inter, int64_t hidden, MvGeo g,
                                              int32_t slot, int64_t r0, const HxpArgs &hx, float w,
                                              float *__restrict__ y, bool accumulate, const MvSmem &m) {
    typename QU<T>::Data d[J];
    mv_issue<T, J>(P.base + e * P.stride, P.row_bytes, hidden, r0, g, d);
    XU X;
    const int u = threadIdx.x % g.U;
    const XPView xv{hx.planes + (int64_t)slot * 3 * inter, hx.scale + (int64_t)slot * (inter / 16),
                    hx.sum + (int64_t)slot * (inter / 16), inter};
    load_xu<T>(xv, u >> 2, u & 3, X);
    mv_partials<T, J>(d, X, g, m.red);
    __syncthreads();
    const int rr = threadIdx.x;
    if (rr < g.S * J && r0 + rr < hidden) {
        const float v = mv_row_sum(m.red, rr, g);
        if (accumulate)
            atomicAdd(&y[r0 + rr], w * v);
        else
            y[r0 + rr] = w * v;
    }
}

// grid = n_slots * ceil(hidden / (S*J)). With one slot and no weights y is
// stored; otherwise every slot adds w_slot * its rows into y (cleared by
// sepia_ffn_gateup), the routed weights then the shared gammas of sel_w.
extern "C" __global__ __launch_bounds__(MV_NT) void sepia_ffn_down(
    MoeProj down, MoeProj s_down, const int32_t *__restrict__ sel_idx, const float *__restrict__ sel_w,
    int32_t fixed_expert, int32_t topk, int32_t n_slots, int64_t inter, int64_t hidden, MvGeo g, int32_t J,
    HxpArgs hx, float *__restrict__ y) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int64_t rows_per = (int64_t)g.S * J;
    const int64_t tiles = (hidden + rows_per - 1) / rows_per;
    const int32_t slot = (int32_t)(blockIdx.x / tiles);
    const int64_t r0 = (blockIdx.x % tiles) * rows_per;
    const bool routed = slot < topk;
    const MoeProj &P = routed ? down : s_down;
    const int64_t e = slot_expert(sel_idx, fixed_expert, slot, topk);
    const float w = sel_w ? sel_w[slot] : 1.0f;
    const bool accumulate = n_slots > 1;
    MvSmem m;
    m.red = (float *)smem;
#define DN_CASE(TT, JJ)                                                                          \
    if (P.type == TT && J == JJ) {                                                               \
        ffn_down_tile<TT, JJ>(P, e, inter, hidden, g, slot, r0, hx, w, y, accumulate, m);        \
        return;                                                                                  \
    }
    DN_CASE(ST_Q2_K, 2) DN_CASE(ST_Q2_K, 4) DN_CASE(ST_Q3_K, 2) DN_CASE(ST_Q3_K, 4)
    DN_CASE(ST_Q4_K, 2) DN_CASE(ST_Q4_K, 4)
#undef DN_CASE
}
