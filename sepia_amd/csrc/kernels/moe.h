// moe.h -- grouped MoE decode for one token (batch 1), no host round trip.
//
// The reference runs this layer as 1 + 4 x (6 + 2) separate dispatches with
// two host syncs and does routing and the weighted sum on the CPU
// (src/sepia.c:3831-3974). Here it is four stream-ordered launches:
//   sepia_matvec_f32   router logits [n_routed + n_shared] from the f32 router
//   sepia_moe_select   sigmoid + bias selection, top-k, mixing weights
//   sepia_moe_gateup   every selected routed expert and every shared expert:
//                      h[slot, i] = silu(gate_i . x) * (up_i . x)
//   sepia_moe_down     y[d] = sum over slots of w[slot] * (down_slot[d, :] . h[slot])
// Slots 0..topk-1 are the routed selection in router order, then the shared
// experts; w holds the routed weights followed by the shared gammas.
#pragma once
#include "common.h"
#include "matvec.h"
#include "mv.h"

struct ArgBest {
    float v;
    int32_t i;   // INT32_MAX: no candidate
};

// Larger score wins; equal scores go to the lower index (the reference's
// sequential strict '>' scan, src/sepia.c:1337-1346).
__device__ __forceinline__ ArgBest arg_better(ArgBest a, ArgBest b) {
    if (a.i == INT32_MAX) return b;
    if (b.i == INT32_MAX) return a;
    if (b.v > a.v) return b;
    if (a.v > b.v) return a;
    return (b.i < a.i) ? b : a;
}

__device__ __forceinline__ float logsigmoid_f32(float x) {
    return (x >= 0.0f) ? -log1pf(expf(-x)) : x - log1pf(expf(x));
}

// One 256-thread workgroup. Scores and the taken mask live in LDS; each of
// the topk rounds is a workgroup arg-max. The weights follow
// src/sepia.c:1355-1372 step for step (float logsigmoid and max, double sum,
// double exp(lp - lse) * route_scale * global_scale rounded to float).
extern "C" __global__ __launch_bounds__(256) void sepia_moe_select(
    const float *__restrict__ logits, const float *__restrict__ bias, int32_t n_routed, int32_t n_shared,
    int32_t topk, float route_scale, float global_scale, int32_t *__restrict__ sel_idx,
    float *__restrict__ sel_w) {
    __shared__ float score[1024];
    __shared__ int32_t taken[1024];
    __shared__ float wv[4];
    __shared__ int32_t wi[4];
    __shared__ int32_t chosen[64];
    for (int i = threadIdx.x; i < n_routed; i += 256) {
        score[i] = sigmoid_f32(logits[i]) + bias[i];
        taken[i] = 0;
    }
    __syncthreads();
    for (int k = 0; k < topk; k++) {
        ArgBest best = {0.0f, INT32_MAX};
        for (int i = threadIdx.x; i < n_routed; i += 256)
            if (!taken[i]) best = arg_better(best, ArgBest{score[i], i});
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            ArgBest o = {__shfl_xor(best.v, off, SEPIA_WAVE), __shfl_xor(best.i, off, SEPIA_WAVE)};
            best = arg_better(best, o);
        }
        if ((threadIdx.x & 63) == 0) {
            wv[threadIdx.x >> 6] = best.v;
            wi[threadIdx.x >> 6] = best.i;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            ArgBest b = {wv[0], wi[0]};
            for (int q = 1; q < 4; q++) b = arg_better(b, ArgBest{wv[q], wi[q]});
            chosen[k] = b.i;
            taken[b.i] = 1;
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const int n_sel = topk + n_shared;
        float lp[64];
        for (int k = 0; k < n_sel; k++) {
            const float raw = (k < topk) ? logits[chosen[k]] : logits[n_routed + (k - topk)];
            lp[k] = logsigmoid_f32(raw);
        }
        float lmax = lp[0];
        for (int k = 1; k < n_sel; k++) lmax = (lp[k] > lmax) ? lp[k] : lmax;
        double se = 0.0;
        for (int k = 0; k < n_sel; k++) se += exp((double)(lp[k] - lmax));
        const double lse = (double)lmax + log(se);
        const double scale = (double)route_scale * (double)global_scale;
        for (int k = 0; k < n_sel; k++) {
            double w = exp((double)lp[k] - lse);
            w *= scale;
            sel_w[k] = (float)w;
        }
        for (int k = 0; k < topk; k++) sel_idx[k] = chosen[k];
    }
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
