// mv.h -- tile kernels for quantized matvecs at decode batch 1: the plain
// matvec, the fused gate/up/SwiGLU launch and the down launch of the expert
// FFN (one launch covers every expert slot of a MoE layer).
//
// A 384-thread workgroup owns T*S whole rows of one matrix (two for
// gate/up). A row of U = in_dim / 64 units (64-weight pieces of a block) is
// spread over U lanes; S = 384 / U rows sit side by side and the workgroup
// walks T such steps. U is a multiple of 16 dividing 384 (in_dim 1024,
// 2048, 3072, 4096, 6144, ..., 24576), so every row's lanes start on a
// 16-lane DPP row.
//
// Per workgroup:
//   1. each lane issues its x loads (or x-plane loads), then the loads of
//      its unit for all T rows (and both matrices), in the order they are
//      consumed -- a wave's loads retire in order, so the first row's dot can
//      start while later rows are still in flight;
//   2. with the weights in flight the workgroup converts x into digit planes
//      in LDS (qdot.h) -- one 16-column segment per thread, v_perm packing --
//      unless x already comes as planes from an earlier launch;
//   3. each lane loads its unit's planes into registers once and forms one
//      integer unit dot per row; a 16-lane DPP sum and a short LDS sum give
//      each row.
// Rows never span workgroups, so no workgroup waits for or talks to another.
// The grid is sized to the 256 CUs (T chosen so that the matrix takes about
// one workgroup per CU), and a MoE launch simply stacks the slots' tiles.
#pragma once
#include "common.h"
#include "qdot.h"

#define MV_NT 384     // threads per workgroup
#define MV_JMAX 3     // row steps per workgroup (loads in flight per lane and matrix)
#define MV_XSEG 2     // x segments converted per thread: in_dim <= 2 * 16 * 384

struct TileGeo {
    int32_t U;      // units per row
    int32_t S;      // rows per step (MV_NT / U)
    int32_t T;      // steps per workgroup, 1..MV_JMAX
    int32_t tiles;  // workgroups per matrix: ceil(ceil(rows / S) / T)
};

// Dynamic LDS: x planes (3n bytes), xs and gs (n/16 floats each), then the
// row partials (MATS * T * S * U/16 floats).
struct TileSmem {
    int8_t *planes;
    float *xs, *gs, *red;
};
__device__ __forceinline__ TileSmem tile_smem(uint8_t *base, int64_t n) {
    TileSmem m;
    m.planes = (int8_t *)base;
    m.xs = (float *)(base + 3 * n);
    m.gs = m.xs + n / 16;
    m.red = m.gs + n / 16;
    return m;
}

// ---- x staging: f32 x -> XP in LDS, one segment per thread and round.
struct XStage {
    float4 v[MV_XSEG][4];
};
__device__ __forceinline__ void xs_load(const float *__restrict__ x, int64_t n, XStage &st) {
    const float4 *x4 = (const float4 *)x;
#pragma unroll
    for (int i = 0; i < MV_XSEG; i++) {
        const int64_t seg = threadIdx.x + (int64_t)i * MV_NT;
        if (seg < n / 16) {
#pragma unroll
            for (int c = 0; c < 4; c++) st.v[i][c] = x4[4 * seg + c];
        }
    }
}
__device__ __forceinline__ void xs_convert(const XStage &st, int64_t n, const TileSmem &m) {
#pragma unroll
    for (int i = 0; i < MV_XSEG; i++) {
        const int64_t seg = threadIdx.x + (int64_t)i * MV_NT;
        if (seg < n / 16) xp_store(xp_segment(st.v[i]), m.planes, m.xs, m.gs, n, seg);
    }
}

// ---- DPP sum over the 16 lanes of a row (every lane gets the sum).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float sum16(float v) {
    v += dpp_f32<0xB1>(v);    // quad_perm [1,0,3,2]
    v += dpp_f32<0x4E>(v);    // quad_perm [2,3,0,1]
    v += dpp_f32<0x141>(v);   // row_half_mirror
    v += dpp_f32<0x140>(v);   // row_mirror
    return v;
}

// ---- weights of MATS matrices for the lane's unit, T rows from row0.
template <int T, int MATS>
struct TileData {
    typename QU<T>::Data d[MV_JMAX][MATS];
};
template <int T, int MATS>
__device__ __forceinline__ void tile_issue(const uint8_t *const (&W)[MATS], uint64_t row_bytes, int64_t rows,
                                           int64_t r0, const TileGeo &g, int u, int s, TileData<T, MATS> &td) {
    const uint64_t col_off = (uint64_t)(u >> 2) * QU<T>::bytes;
#pragma unroll
    for (int j = 0; j < MV_JMAX; j++) {
        if (j < g.T) {
            int64_t r = r0 + (int64_t)j * g.S + s;
            r = r < rows ? r : rows - 1;   // tail rows load a valid row; their sums are dropped
#pragma unroll
            for (int mt = 0; mt < MATS; mt++) td.d[j][mt] = QU<T>::load(W[mt] + (uint64_t)r * row_bytes + col_off, u & 3);
        }
    }
}

// Unit dots, 16-lane sums, partials to red[(mt*T*S + j*S + s) * U/16 + u/16].
template <int T, int MATS>
__device__ __forceinline__ void tile_dots(const TileData<T, MATS> &td, const XU &X, const TileGeo &g, int u, int s,
                                          float *red) {
    const int nq = g.U >> 4;
#pragma unroll
    for (int j = 0; j < MV_JMAX; j++) {
        if (j < g.T) {
#pragma unroll
            for (int mt = 0; mt < MATS; mt++) {
                const float a = sum16(QU<T>::dot(td.d[j][mt], u & 3, X));
                if ((u & 15) == 0) red[((mt * g.T + j) * g.S + s) * nq + (u >> 4)] = a;
            }
        }
    }
}

// Sum of row i (= j*S + s) of matrix mt from the partials.
__device__ __forceinline__ float tile_row(const float *red, int mt, int i, const TileGeo &g) {
    const int nq = g.U >> 4;
    const float *p = red + (mt * g.T * g.S + i) * nq;
    float v = 0.0f;
    for (int q = 0; q < nq; q++) v += p[q];
    return v;
}

// ---- y = W x for one matrix; grid = g.tiles.
template <int T>
__device__ __forceinline__ void mv_tile(const uint8_t *__restrict__ W, uint64_t row_bytes, int64_t rows, int64_t n,
                                        const TileGeo &g, const float *__restrict__ x, float *__restrict__ y) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const TileSmem m = tile_smem(smem, n);
    const int u = threadIdx.x % g.U, s = threadIdx.x / g.U;
    const int64_t r0 = (int64_t)blockIdx.x * g.T * g.S;
    XStage st;
    xs_load(x, n, st);
    TileData<T, 1> td;
    const uint8_t *const Wm[1] = {W};
    tile_issue<T, 1>(Wm, row_bytes, rows, r0, g, u, s, td);
    xs_convert(st, n, m);
    __syncthreads();
    XU X;
    load_xu<T>(m.planes, m.xs, m.gs, n, u >> 2, u & 3, X);
    tile_dots<T, 1>(td, X, g, u, s, m.red);
    __syncthreads();
    const int i = threadIdx.x;
    if (i < g.T * g.S && r0 + i < rows) y[r0 + i] = tile_row(m.red, 0, i, g);
}

#define SEPIA_MV_KERNEL(name, T)                                                                  \
    extern "C" __global__ __launch_bounds__(MV_NT) void sepia_mv_##name(                          \
        const uint8_t *__restrict__ W, uint64_t row_bytes, int64_t rows, int64_t n, TileGeo g,    \
        const float *__restrict__ x, float *__restrict__ y) {                                     \
        mv_tile<T>(W, row_bytes, rows, n, g, x, y);                                               \
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

// x in digit-plane form in global memory (written by the router launch).
struct XpArgs {
    const int8_t *planes;   // [3][n]
    const float *xs;        // [n / 16]
    const float *gs;        // [n / 16]
};

__device__ __forceinline__ int64_t slot_expert(const int32_t *sel_idx, int32_t fixed, int32_t slot, int32_t topk) {
    return slot < topk ? (sel_idx ? (int64_t)sel_idx[slot] : (int64_t)fixed + slot) : (int64_t)(slot - topk);
}

// h[slot, i] = silu(gate_i . x) * (up_i . x) for the T*S rows i of one tile.
// XP_IN: x's planes come from global memory (xp); else x is f32 and is
// converted in LDS.
template <int T, bool XP_IN>
__device__ __forceinline__ void gateup_tile(const MoeProj &G, const MoeProj &Up, int64_t e, int64_t inter,
                                            int64_t hidden, const TileGeo &g, int32_t slot, int64_t r0,
                                            const float *__restrict__ x, const XpArgs &xp, float *__restrict__ h) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int u = threadIdx.x % g.U, s = threadIdx.x / g.U;
    const uint8_t *const Wm[2] = {G.base + e * G.stride, Up.base + e * Up.stride};
    TileData<T, 2> td;
    XU X;
    float *red;
    if (XP_IN) {
        red = (float *)smem;
        load_xu<T>(xp.planes, xp.xs, xp.gs, hidden, u >> 2, u & 3, X);
        tile_issue<T, 2>(Wm, G.row_bytes, inter, r0, g, u, s, td);
    } else {
        const TileSmem m = tile_smem(smem, hidden);
        red = m.red;
        XStage st;
        xs_load(x, hidden, st);
        tile_issue<T, 2>(Wm, G.row_bytes, inter, r0, g, u, s, td);
        xs_convert(st, hidden, m);
        __syncthreads();
        load_xu<T>(m.planes, m.xs, m.gs, hidden, u >> 2, u & 3, X);
    }
    tile_dots<T, 2>(td, X, g, u, s, red);
    __syncthreads();
    const int i = threadIdx.x;
    if (i < g.T * g.S && r0 + i < inter) {
        const float gv = tile_row(red, 0, i, g), uv = tile_row(red, 1, i, g);
        h[(int64_t)slot * inter + r0 + i] = silu_f32(gv) * uv;
    }
}

// grid = n_slots * g.tiles. Routed slots (< topk) use type TR and take their
// expert from sel_idx (or fixed_expert + slot); the later (shared) slots use
// type TS. Workgroups also clear y_zero[0 .. y_n) when it is set (the down
// launch then accumulates into it).
template <int TR, int TS, bool XP_IN>
__device__ __forceinline__ void ffn_gateup_body(const MoeProj &gate, const MoeProj &up, const MoeProj &s_gate,
                                                const MoeProj &s_up, const int32_t *__restrict__ sel_idx,
                                                int32_t fixed_expert, int32_t topk, int64_t inter, int64_t hidden,
                                                const TileGeo &g, const float *__restrict__ x, const XpArgs &xp,
                                                float *__restrict__ h, float *__restrict__ y_zero, int64_t y_n) {
    if (y_zero) {
        for (int64_t i = (int64_t)blockIdx.x * MV_NT + threadIdx.x; i < y_n; i += (int64_t)gridDim.x * MV_NT)
            y_zero[i] = 0.0f;
    }
    const int32_t slot = (int32_t)(blockIdx.x / g.tiles);
    const int64_t r0 = (int64_t)(blockIdx.x % g.tiles) * g.T * g.S;
    const int64_t e = slot_expert(sel_idx, fixed_expert, slot, topk);
    if (slot < topk)
        gateup_tile<TR, XP_IN>(gate, up, e, inter, hidden, g, slot, r0, x, xp, h);
    else
        gateup_tile<TS, XP_IN>(s_gate, s_up, e, inter, hidden, g, slot, r0, x, xp, h);
}

#define SEPIA_FFN_GATEUP(name, TR, TS, XP_IN)                                                        \
    extern "C" __global__ __launch_bounds__(MV_NT) void sepia_ffn_gateup_##name(                     \
        MoeProj gate, MoeProj up, MoeProj s_gate, MoeProj s_up, const int32_t *__restrict__ sel_idx, \
        int32_t fixed_expert, int32_t topk, int64_t inter, int64_t hidden, TileGeo g,                \
        const float *__restrict__ x, XpArgs xp, float *__restrict__ h, float *__restrict__ y_zero,   \
        int64_t y_n) {                                                                               \
        ffn_gateup_body<TR, TS, XP_IN>(gate, up, s_gate, s_up, sel_idx, fixed_expert, topk, inter,   \
                                       hidden, g, x, xp, h, y_zero, y_n);                            \
    }

// y[d] (+)= w_slot * (down_slot[d, :] . h_slot) for the T*S rows d of one tile.
template <int T>
__device__ __forceinline__ void down_tile(const MoeProj &P, int64_t e, int64_t inter, int64_t hidden,
                                          const TileGeo &g, int64_t r0, const float *__restrict__ hs, float w,
                                          float *__restrict__ y, bool accumulate) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const TileSmem m = tile_smem(smem, inter);
    const int u = threadIdx.x % g.U, s = threadIdx.x / g.U;
    XStage st;
    xs_load(hs, inter, st);
    TileData<T, 1> td;
    const uint8_t *const Wm[1] = {P.base + e * P.stride};
    tile_issue<T, 1>(Wm, P.row_bytes, hidden, r0, g, u, s, td);
    xs_convert(st, inter, m);
    __syncthreads();
    XU X;
    load_xu<T>(m.planes, m.xs, m.gs, inter, u >> 2, u & 3, X);
    tile_dots<T, 1>(td, X, g, u, s, m.red);
    __syncthreads();
    const int i = threadIdx.x;
    if (i < g.T * g.S && r0 + i < hidden) {
        const float v = tile_row(m.red, 0, i, g);
        if (accumulate)
            atomicAdd(&y[r0 + i], w * v);
        else
            y[r0 + i] = w * v;
    }
}

// grid = n_slots * g.tiles; h is [n_slots][inter] f32. With one slot and no
// weights y is stored; otherwise every slot adds sel_w[slot] * its rows into
// y (cleared by the gate/up launch): the routed weights, then the shared
// gammas (the shared gamma scales the down output, src/sepia.c:3953-3957,
// equal to scaling h before down as src/sepia.c:1441 does).
template <int TR, int TS>
__device__ __forceinline__ void ffn_down_body(const MoeProj &down, const MoeProj &s_down,
                                              const int32_t *__restrict__ sel_idx, const float *__restrict__ sel_w,
                                              int32_t fixed_expert, int32_t topk, int32_t n_slots, int64_t inter,
                                              int64_t hidden, const TileGeo &g, const float *__restrict__ h,
                                              float *__restrict__ y) {
    const int32_t slot = (int32_t)(blockIdx.x / g.tiles);
    const int64_t r0 = (int64_t)(blockIdx.x % g.tiles) * g.T * g.S;
    const int64_t e = slot_expert(sel_idx, fixed_expert, slot, topk);
    const float w = sel_w ? sel_w[slot] : 1.0f;
    const float *hs = h + (int64_t)slot * inter;
    if (slot < topk)
        down_tile<TR>(down, e, inter, hidden, g, r0, hs, w, y, n_slots > 1);
    else
        down_tile<TS>(s_down, e, inter, hidden, g, r0, hs, w, y, n_slots > 1);
}

#define SEPIA_FFN_DOWN(name, TR, TS)                                                                 \
    extern "C" __global__ __launch_bounds__(MV_NT) void sepia_ffn_down_##name(                       \
        MoeProj down, MoeProj s_down, const int32_t *__restrict__ sel_idx,                           \
        const float *__restrict__ sel_w, int32_t fixed_expert, int32_t topk, int32_t n_slots,        \
        int64_t inter, int64_t hidden, TileGeo g, const float *__restrict__ h, float *__restrict__ y) { \
        ffn_down_body<TR, TS>(down, s_down, sel_idx, sel_w, fixed_expert, topk, n_slots, inter,     \
                              hidden, g, h, y);                                                      \
    }
