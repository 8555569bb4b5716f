// moe.h -- grouped MoE decode for one token (batch 1), no host round trip.
//
// The reference runs this layer as 1 + 4 x (6 + 2) separate dispatches with
// two host syncs and does routing and the weighted sum on the CPU
// (src/sepia.c:3831-3974). Here it is three stream-ordered launches:
//   sepia_moe_route        router logits [n_routed + n_shared], x in XP
//                          form, and the selection (last workgroup)
//   sepia_ffn_gateup_*     every selected routed expert and every shared
//                          expert: h[slot, i] = silu(gate_i . x) * (up_i . x)
//   sepia_ffn_down_*       y[d] = sum over slots of w[slot] * (down_slot[d, :] . h[slot])
// (mv.h for the last two; the *_generic kernels below cover formats without
// a tile decoder). Slots 0..topk-1 are the routed selection in router order,
// then the shared experts; w holds the routed weights followed by the shared
// gammas.
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

// ------------------------------------------------------------------ router
// Router logits and the selection, in one launch. Workgroup w computes
// router row w (f32 FMA chains, 16-byte loads issued up front). Each workgroup publishes its logits with agent-scope
// stores, waits for them to complete and bumps an arrival counter; the
// workgroup that arrives last sees every logit, runs the selection and puts
// the counter back to zero (so the launch can be replayed from a graph).
//
// Selection (reference src/sepia.c:1329-1375): score = sigmoid(logit) + bias
// for the routed experts, bias for selection only; topk rounds of arg-max
// with ties to the lowest index; weights over the topk selected raw logits
// and the n_shared sink logits: float log-sigmoid and max, then in double
// lse = max + log(sum exp(lp - max)) and w = exp(lp - lse) * route_scale *
// global_scale, rounded to float. Slots 0..topk-1 of sel_w are the routed
// weights (router order), then the shared gammas.
#define RT_NT 256
#define RT_ROWS 1
#define RT_C4 8   // float4 chunks per thread and row: hidden <= 256 * 4 * 8

// ---- wave-wide reductions without LDS: DPP within each 16-lane row, then
// the four row results read back as uniform values.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_f32(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
__device__ __forceinline__ float wave_max_dpp(float v) {
    v = fmaxf(v, dpp_mov<0xB1>(v));    // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp_mov<0x4E>(v));    // quad_perm [2,3,0,1]
    v = fmaxf(v, dpp_mov<0x141>(v));   // row_half_mirror
    v = fmaxf(v, dpp_mov<0x140>(v));   // row_mirror
    return fmaxf(fmaxf(lane_f32(v, 0), lane_f32(v, 16)), fmaxf(lane_f32(v, 32), lane_f32(v, 48)));
}
// Sum of lanes 0..n-1's doubles, added in lane order (the reference sums the
// selected terms sequentially); n is at most a few dozen.
__device__ __forceinline__ double lanes_sum_f64(double v, int n) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    double s = 0.0;
    for (int k = 0; k < n; k++) {
        const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, k);
        const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), k);
        s += __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
    }
    return s;
}

// Selection by one wave (wave 0 of the last workgroup); lg holds the
// n_routed + n_shared logits and score the n_routed selection scores
// (sigmoid(logit) + bias), both in LDS. Lane l keeps the scores of experts
// [l*E, l*E + E), E = ceil(n_routed / 64) <= 16, in registers. Each of the
// topk rounds takes the lane's best untaken score (strict '>', so the lowest
// index among equals), the wave maximum by DPP, and the lowest lane holding
// it -- the lowest expert index among equal scores, since lanes hold
// ascending index ranges. No LDS traffic and no barriers.
__device__ void route_select_wave(const float *lg, const float *score, int32_t n_routed, int32_t n_shared,
                                  int32_t topk, float route_scale, float global_scale, int32_t *__restrict__ sel_idx,
                                  float *__restrict__ sel_w) {
    const int lane = threadIdx.x & 63;
    const int E = (n_routed + 63) >> 6;
    float sc[16];
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const int i = lane * E + j;
        sc[j] = (j < E && i < n_routed) ? score[i] : -INFINITY;
    }
    uint32_t taken = 0;
    int my_pick = 0;                       // lane k < topk: the k-th selected expert
    for (int k = 0; k < topk; k++) {
        float best = -INFINITY;
        int bj = -1;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const int i = lane * E + j;
            if (j < E && i < n_routed && !((taken >> j) & 1u) && (bj < 0 || sc[j] > best)) {
                best = sc[j];
                bj = j;
            }
        }
        const float wmax = wave_max_dpp(bj >= 0 ? best : -INFINITY);
        const uint64_t hit = __ballot(bj >= 0 && best == wmax);
        const int win_lane = (int)__builtin_ctzll(hit);
        const int win_j = __builtin_amdgcn_readlane(bj, win_lane);
        if (lane == win_lane) taken |= 1u << win_j;
        if (lane == k) my_pick = win_lane * E + win_j;
    }
    // weights over the selected raw logits (lanes < topk) and the sinks
    const int n_sel = topk + n_shared;
    const bool on = lane < n_sel;
    const float raw = on ? ((lane < topk) ? lg[my_pick] : lg[n_routed + (lane - topk)]) : 0.0f;
    const float lp = on ? logsigmoid_f32(raw) : -INFINITY;
    const float lmax = wave_max_dpp(lp);
    const double e = on ? exp((double)(lp - lmax)) : 0.0;
    const double lse = (double)lmax + log(lanes_sum_f64(e, n_sel));
    if (on) {
        double w = exp((double)lp - lse);
        w *= (double)route_scale * (double)global_scale;
        sel_w[lane] = (float)w;
        if (lane < topk) sel_idx[lane] = my_pick;
    }
}

extern "C" __global__ __launch_bounds__(RT_NT) void sepia_moe_route(
    const float *__restrict__ rw, int64_t ld, const float *__restrict__ bias, const float *__restrict__ x,
    int64_t hidden, int32_t n_routed, int32_t n_shared, int32_t topk, float route_scale, float global_scale,
    float *__restrict__ logits, int32_t *__restrict__ sel_idx, float *__restrict__ sel_w,
    uint32_t *__restrict__ counter) {
    __shared__ float part[RT_NT / SEPIA_WAVE][RT_ROWS];
    __shared__ float lg[1024 + 64];
    __shared__ float score[1024];
    __shared__ int last;
    const int n_tot = n_routed + n_shared;
    const int64_t r0 = (int64_t)blockIdx.x * RT_ROWS;
    const int t = threadIdx.x;
    // the selection bias, loaded by every workgroup up front (1 KB, cached)
    // so that the last one does not wait for it after the arrival
    float bias_r[4];
#pragma unroll
    for (int q = 0; q < 4; q++) bias_r[q] = (t + q * RT_NT < n_routed) ? bias[t + q * RT_NT] : 0.0f;
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
        const float v = wave_sum(acc[r]);
        if ((t & 63) == 0) part[t >> 6][r] = v;
    }
    __syncthreads();
    if (t == 0) {
#pragma unroll
        for (int r = 0; r < RT_ROWS; r++) {
            float v = 0.0f;
            for (int q = 0; q < RT_NT / SEPIA_WAVE; q++) v += part[q][r];
            if (r0 + r < n_tot) __hip_atomic_store(&logits[r0 + r], v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __builtin_amdgcn_s_waitcnt(0);   // the logit stores have completed
        const uint32_t prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = (prev == gridDim.x - 1);
    }
    __syncthreads();
    if (!last) return;
    float lv[5];
#pragma unroll
    for (int q = 0; q < 5; q++)
        lv[q] = (t + q * RT_NT < n_tot) ? __hip_atomic_load(&logits[t + q * RT_NT], __ATOMIC_RELAXED,
                                                             __HIP_MEMORY_SCOPE_AGENT) : 0.0f;
    if (t == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
    for (int q = 0; q < 5; q++) {
        const int i = t + q * RT_NT;
        if (i < n_tot) lg[i] = lv[q];
        if (q < 4 && i < n_routed) score[i] = sigmoid_f32(lv[q]) + bias_r[q];
    }
    __syncthreads();
    if (t < SEPIA_WAVE) route_select_wave(lg, score, n_routed, n_shared, topk, route_scale, global_scale, sel_idx, sel_w);
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
