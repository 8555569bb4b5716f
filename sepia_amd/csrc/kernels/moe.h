// moe.h -- grouped MoE decode for one token (batch 1), no host round trip.
//
// The reference runs this layer as 1 + 4 x (6 + 2) separate dispatches with
// two host syncs and does routing and the weighted sum on the CPU
// (src/sepia.c:3831-3974). Here it is three stream-ordered launches:
//   sepia_moe_route        router logits [n_routed + n_shared] (and, for the
//                          FFN kernels below, the selection)
//   gate/up                every selected routed expert and every shared
//                          expert: h[slot, i] = silu(gate_i . x) * (up_i . x)
//                          (mq.h, which then also selects; else mv.h or the
//                          *_generic kernel here)
//   down                   y[d] = sum over slots of w[slot] * (down_slot[d, :] . h[slot])
// Slots 0..topk-1 are the routed selection in router order, then the shared
// experts; w holds the routed weights followed by the shared gammas.
#pragma once
#include "common.h"
#include "matvec.h"
#include "mv.h"
#include "route.h"

// ------------------------------------------------------------------ router
// Router logits [n_routed + n_shared] for one token: workgroup w computes
// router row w (f32 FMA chains, 16-byte loads issued up front). With
// `select` set the launch also runs the selection (route.h): each workgroup
// publishes its logit with an agent-scope store, waits for it to complete
// and bumps an arrival counter; the workgroup that arrives last sees every
// logit, runs the selection and puts the counter back to zero (so the launch
// can be replayed from a graph). Without it the logits are the only output
// and the matrix-core gate/up kernel selects (mq.h).
#define RT_NT 512
#define RT_ROWS 1
#define RT_C4 4   // float4 chunks per thread and row: hidden <= 512 * 4 * 4

extern "C" __global__ __launch_bounds__(RT_NT) void sepia_moe_route(
    const float *__restrict__ rw, int64_t ld, const float *__restrict__ bias, const float *__restrict__ x,
    int64_t hidden, int32_t n_routed, int32_t n_shared, int32_t topk, float route_scale, float global_scale,
    float *__restrict__ logits, int32_t *__restrict__ sel_idx, float *__restrict__ sel_w,
    uint32_t *__restrict__ counter, int32_t select) {
    sepia_kernarg_warm<320>();
    __shared__ float part[RT_NT / SEPIA_WAVE][RT_ROWS];
    __shared__ int last;
    const int n_tot = n_routed + n_shared;
    const int64_t r0 = (int64_t)blockIdx.x * RT_ROWS;
    const int t = threadIdx.x;
    float acc[RT_ROWS];
#pragma unroll
    for (int r = 0; r < RT_ROWS; r++) acc[r] = 0.0f;
    const bool vec = ((((uintptr_t)rw | (uintptr_t)x) & 15) == 0) && (ld & 3) == 0 && (hidden & 3) == 0 &&
                     hidden <= 4 * RT_NT * RT_C4;
    if (vec) {
        const int64_t n4 = hidden >> 2;
        const float4 *x4 = (const float4 *)x;
        float4 xv[RT_C4], wv[RT_ROWS][RT_C4];
#pragma unroll
        for (int c = 0; c < RT_C4; c++) {
            const int64_t i = t + (int64_t)c * RT_NT;
            if (i < n4) xv[c] = x4[i];
        }
#pragma unroll
        for (int r = 0; r < RT_ROWS; r++) {
            const int64_t row = (r0 + r < n_tot) ? r0 + r : n_tot - 1;
            const float4 *w4 = (const float4 *)(rw + row * ld);
#pragma unroll
            for (int c = 0; c < RT_C4; c++) {
                const int64_t i = t + (int64_t)c * RT_NT;
                if (i < n4) wv[r][c] = w4[i];
            }
        }
#pragma unroll
        for (int c = 0; c < RT_C4; c++) {
            const int64_t i = t + (int64_t)c * RT_NT;
            if (i < n4) {
#pragma unroll
                for (int r = 0; r < RT_ROWS; r++) {
                    acc[r] = __builtin_fmaf(wv[r][c].x, xv[c].x, acc[r]);
                    acc[r] = __builtin_fmaf(wv[r][c].y, xv[c].y, acc[r]);
                    acc[r] = __builtin_fmaf(wv[r][c].z, xv[c].z, acc[r]);
                    acc[r] = __builtin_fmaf(wv[r][c].w, xv[c].w, acc[r]);
                }
            }
        }
    } else {
        for (int64_t i = t; i < hidden; i += RT_NT) {
#pragma unroll
            for (int r = 0; r < RT_ROWS; r++) {
                const int64_t row = (r0 + r < n_tot) ? r0 + r : n_tot - 1;
                acc[r] = __builtin_fmaf(rw[row * ld + i], x[i], acc[r]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RT_ROWS; r++) {
        const float v = wave_sum_dpp(acc[r]);
        if ((t & 63) == 0) part[t >> 6][r] = v;
    }
    __syncthreads();
    if (t == 0) {
#pragma unroll
        for (int r = 0; r < RT_ROWS; r++) {
            float v = 0.0f;
            for (int q = 0; q < RT_NT / SEPIA_WAVE; q++) v += part[q][r];
            if (r0 + r < n_tot) {
                if (select) __hip_atomic_store(&logits[r0 + r], v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                else logits[r0 + r] = v;
            }
        }
        if (select) {
            __builtin_amdgcn_s_waitcnt(0);   // the logit stores have completed
            const uint32_t prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last = (prev == gridDim.x - 1);
        }
    }
    if (!select) return;
    __syncthreads();
    if (!last) return;
    if (t == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (t < SEPIA_WAVE)
        route_pick_any<true>(logits, bias, n_routed, n_shared, topk, route_scale, global_scale, sel_idx, sel_w);
}

__device__ __forceinline__ const uint8_t *moe_row(const MoeProj &P, int64_t e, int64_t r) {
    return P.base + e * P.stride + r * P.row_bytes;
}

// One wave per (slot, intermediate row); 4 rows per workgroup. sel_idx may be
// NULL: then slot s < topk is expert fixed_expert + s (a single-expert FFN).
extern "C" __global__ __launch_bounds__(256) void sepia_moe_gateup_generic(
    MoeProj gate, MoeProj up, MoeProj s_gate, MoeProj s_up, const int32_t *__restrict__ sel_idx,
    int32_t fixed_expert, int32_t topk, int64_t inter, const float *__restrict__ x, float *__restrict__ h) {
    const int64_t tiles = (inter + 3) / 4;
    const int32_t slot = (int32_t)(blockIdx.x / tiles);
    const int64_t row = (blockIdx.x % tiles) * 4 + (threadIdx.x >> 6);
    if (row >= inter) return;
    const bool routed = slot < topk;
    const int64_t e = routed ? (sel_idx ? sel_idx[slot] : fixed_expert + slot) : slot - topk;
    const MoeProj &G = routed ? gate : s_gate;
    const MoeProj &U = routed ? up : s_up;
    const float g = row_dot_any(G.type, moe_row(G, e, row), G.n_blocks, x);
    const float u = row_dot_any(U.type, moe_row(U, e, row), U.n_blocks, x);
    if ((threadIdx.x & 63) == 0) h[(int64_t)slot * inter + row] = silu_f32(g) * u;
}

// One wave per output row d; it walks every slot, so the weighted sum is
// formed in registers in a fixed order (deterministic, no atomics). With
// sel_idx NULL the routed slots are experts fixed_expert + s and, with sel_w
// NULL, every weight is 1.
extern "C" __global__ __launch_bounds__(256) void sepia_moe_down_generic(
    MoeProj down, MoeProj s_down, const int32_t *__restrict__ sel_idx, const float *__restrict__ sel_w,
    int32_t fixed_expert, int32_t topk, int32_t n_shared, int64_t inter, int64_t hidden,
    const float *__restrict__ h, float *__restrict__ y) {
    const int64_t d = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (d >= hidden) return;
    float acc = 0.0f;
    for (int32_t slot = 0; slot < topk + n_shared; slot++) {
        const bool routed = slot < topk;
        const MoeProj &P = routed ? down : s_down;
        const int64_t e = routed ? (sel_idx ? sel_idx[slot] : fixed_expert + slot) : slot - topk;
        const float v = row_dot_any(P.type, moe_row(P, e, d), P.n_blocks, h + (int64_t)slot * inter);
        acc = sel_w ? __builtin_fmaf(sel_w[slot], v, acc) : acc + v;
    }
    if ((threadIdx.x & 63) == 0) y[d] = acc;
}
