// route.h -- MoE expert selection by one wave (reference src/sepia.c:1329-1375).
//
// score = sigmoid(logit) + bias for the routed experts (the bias steers the
// selection only); topk rounds of arg-max with ties to the lowest index;
// weights over the topk selected raw logits and the n_shared sink logits:
// float log-sigmoid and max, then in double lse = max + log(sum exp(lp -
// max)) and w = exp(lp - lse) * route_scale * global_scale, rounded to
// float. Slots 0..topk-1 of the weights are the routed ones (selection
// order), then the shared gammas.
#pragma once
#include "common.h"

__device__ __forceinline__ float logsigmoid_f32(float x) {
    return (x >= 0.0f) ? -log1pf(expf(-x)) : x - log1pf(expf(x));
}

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
// Signed-integer key with the order of a float score (finite or infinite;
// -0 counts as +0). NaN and unused slots rank below every number: NaN at
// INT32_MIN + 1, unused slots at INT32_MIN.
__device__ __forceinline__ int32_t route_key(float v, bool ok) {
    int32_t b = __builtin_bit_cast(int32_t, v + 0.0f);
    b = b < 0 ? (b ^ 0x7FFFFFFF) : b;
    return !ok ? INT32_MIN : (v == v ? b : INT32_MIN + 1);
}
template <int CTRL>
__device__ __forceinline__ int32_t dpp_mov_i32(int32_t v) {
    return __builtin_amdgcn_update_dpp(v, v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ int32_t wave_max_i32(int32_t v) {
    v = max(v, dpp_mov_i32<0xB1>(v));    // quad_perm [1,0,3,2]
    v = max(v, dpp_mov_i32<0x4E>(v));    // quad_perm [2,3,0,1]
    v = max(v, dpp_mov_i32<0x141>(v));   // row_half_mirror
    v = max(v, dpp_mov_i32<0x140>(v));   // row_mirror
    return max(max(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
               max(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}
// Compare-exchange of two (key, slot) entries so that a comes first: the
// larger key, or the lower slot among equal keys.
__device__ __forceinline__ void route_cx(int32_t &ka, int32_t &ja, int32_t &kb, int32_t &jb) {
    const bool sw = kb > ka || (kb == ka && jb < ja);
    const int32_t tk = ka, tj = ja;
    ka = sw ? kb : ka;
    ja = sw ? jb : ja;
    kb = sw ? tk : kb;
    jb = sw ? tj : jb;
}

// Wave sum by DPP within each 16-lane row, then the four row sums read
// back as uniform values: (row 0 + row 1) + (row 2 + row 3). No LDS round
// trips (wave_sum's shuffles are LDS permutes).
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += dpp_mov<0xB1>(v);    // quad_perm [1,0,3,2]
    v += dpp_mov<0x4E>(v);    // quad_perm [2,3,0,1]
    v += dpp_mov<0x141>(v);   // row_half_mirror
    v += dpp_mov<0x140>(v);   // row_mirror
    return (lane_f32(v, 0) + lane_f32(v, 16)) + (lane_f32(v, 32) + lane_f32(v, 48));
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

// The selection, run by every lane of one wave. Lane l keeps the logits and
// scores of experts [l E, l E + E), E = ceil(n_routed / 64) <= EM, in
// registers. Each of the topk rounds takes the lane's best untaken score
// (strict '>', so the lowest index among equals), the wave maximum by DPP
// and the lowest lane holding it -- the lowest expert index among equal
// scores, since lanes hold ascending index ranges. Lane k < topk then writes
// idx[k], lane k < topk + n_shared writes w[k] (idx and w may point to LDS
// or global memory). ATOMIC: the logits come from other workgroups of the
// same launch (agent-scope loads). n_routed <= 64 * EM, topk <= 64 - n_shared.
// w NULL: the selection only (idx), without the weights' log-sum-exp.
template <int EM, bool ATOMIC>
__device__ void route_pick(const float *logits, const float *__restrict__ bias, int32_t n_routed, int32_t n_shared,
                           int32_t topk, float route_scale, float global_scale, int32_t *idx, float *w) {
    const int lane = threadIdx.x & 63;
    const int E = (n_routed + 63) >> 6;
    auto ld = [&](int i) {
        if constexpr (ATOMIC) return __hip_atomic_load(&logits[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else return logits[i];
    };
    const int n_sel = topk + n_shared;
    // the shared experts' sink logits load with the routed ones (one round trip)
    const float sink = (lane >= topk && lane < n_sel) ? ld(n_routed + (lane - topk)) : 0.0f;
    float lv[EM], sc[EM];
    bool ok[EM];
#pragma unroll
    for (int j = 0; j < EM; j++) {
        const int i = lane * E + j;
        ok[j] = j < E && i < n_routed;
        lv[j] = ok[j] ? ld(i) : 0.0f;
        sc[j] = ok[j] ? sigmoid_f32(lv[j]) + bias[i] : -INFINITY;
    }
    uint32_t taken = 0;
    int my_pick = 0;                   // lane k < topk: the k-th selected expert and its raw logit
    float my_raw = 0.0f;
    if constexpr (EM == 4) {
        // Each lane sorts its four (score key, slot) entries once, best
        // first; a round then compares only the lanes' heads, and the
        // winning lane pops its head. The same picks in the same order as
        // the scan below: the largest score, the lowest expert index among
        // equal scores (lanes hold ascending index ranges).
        int32_t k0 = route_key(sc[0], ok[0]), k1 = route_key(sc[1], ok[1]);
        int32_t k2 = route_key(sc[2], ok[2]), k3 = route_key(sc[3], ok[3]);
        int32_t j0 = 0, j1 = 1, j2 = 2, j3 = 3;
        route_cx(k0, j0, k1, j1);
        route_cx(k2, j2, k3, j3);
        route_cx(k0, j0, k2, j2);
        route_cx(k1, j1, k3, j3);
        route_cx(k1, j1, k2, j2);
        uint32_t jl = (uint32_t)j0 | ((uint32_t)j1 << 2) | ((uint32_t)j2 << 4) | ((uint32_t)j3 << 6);
        for (int k = 0; k < topk; k++) {
            const int32_t wm = wave_max_i32(k0);
            const uint64_t hit = __ballot(k0 == wm);
            const int win_lane = (int)__builtin_ctzll(hit);
            const int win_j = __builtin_amdgcn_readlane((int)(jl & 3u), win_lane);
            if (w) {
                const uint32_t hj = jl & 3u;
                const float hr = hj == 0 ? lv[0] : hj == 1 ? lv[1] : hj == 2 ? lv[2] : lv[3];
                const float raw = lane_f32(hr, win_lane);
                if (lane == k) my_raw = raw;
            }
            if (lane == win_lane) {
                k0 = k1;
                k1 = k2;
                k2 = k3;
                k3 = INT32_MIN;
                jl >>= 2;
            }
            if (lane == k) my_pick = win_lane * E + win_j;
        }
    } else for (int k = 0; k < topk; k++) {
        float best = -INFINITY, braw = 0.0f;
        int bj = -1;
#pragma unroll
        for (int j = 0; j < EM; j++) {
            if (ok[j] && !((taken >> j) & 1u) && (bj < 0 || sc[j] > best)) {
                best = sc[j];
                braw = lv[j];
                bj = j;
            }
        }
        const float wmax = wave_max_dpp(bj >= 0 ? best : -INFINITY);
        uint64_t hit = __ballot(bj >= 0 && best == wmax);
        if (!hit) hit = __ballot(bj >= 0);   // unordered scores: the lowest candidate
        const int win_lane = (int)__builtin_ctzll(hit);
        const int win_j = __builtin_amdgcn_readlane(bj, win_lane);
        const float raw = lane_f32(braw, win_lane);
        if (lane == win_lane) taken |= 1u << win_j;
        if (lane == k) {
            my_pick = win_lane * E + win_j;
            my_raw = raw;
        }
    }
    if (!w) {
        if (lane < topk) idx[lane] = my_pick;
        return;
    }
    const bool on = lane < n_sel;
    const float raw = on ? ((lane < topk) ? my_raw : sink) : 0.0f;
    const float lp = on ? logsigmoid_f32(raw) : -INFINITY;
    const float lmax = wave_max_dpp(lp);
    const double e = on ? exp((double)(lp - lmax)) : 0.0;
    const double lse = (double)lmax + log(lanes_sum_f64(e, n_sel));
    if (on) {
        double wd = exp((double)lp - lse);
        wd *= (double)route_scale * (double)global_scale;
        w[lane] = (float)wd;
        if (lane < topk) idx[lane] = my_pick;
    }
}

// route_pick with the register width the expert count needs (n_routed <=
// 1024).
template <bool ATOMIC>
__device__ __forceinline__ void route_pick_any(const float *logits, const float *__restrict__ bias, int32_t n_routed,
                                               int32_t n_shared, int32_t topk, float route_scale, float global_scale,
                                               int32_t *idx, float *w) {
    if (n_routed <= 256) route_pick<4, ATOMIC>(logits, bias, n_routed, n_shared, topk, route_scale, global_scale, idx, w);
    else route_pick<16, ATOMIC>(logits, bias, n_routed, n_shared, topk, route_scale, global_scale, idx, w);
}
