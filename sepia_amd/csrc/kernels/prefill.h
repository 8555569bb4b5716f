// prefill.h -- the MoE layer for a batch of tokens (prefill), grouped by
// expert, on the bf16 matrix cores.
//
// Every token gets exactly the decode path's result (reference
// src/sepia.c:1377-1470 per token): the same router logits up to f32
// summation order, the same selection (route.h), then
//   y[t] = sum_{k < topk} w[t][k] down_e(silu(gate_e x_t) * up_e x_t)
//        + sum_s w[t][topk + s] down_s(silu(gate_s x_t) * up_s x_t).
// Launches:
//   sepia_pf_route    logits[T][n_routed + n_shared] = x . Rw^T (f32 tiles)
//   sepia_pf_select   one wave per token: idx[T][topk], w[T][topk + n_shared]
//   sepia_pf_group    one workgroup: the (token, slot) pairs p = t * n_sel + k
//                     sorted by expert (shared expert s is expert
//                     n_routed + s) and cut into units of <= 32 pairs
//   sepia_pf_gateup   per (unit, 32-row tile): h[p][.] = silu(g) * u
//   sepia_pf_down     per (unit, 64-row tile): yp[p][.] = down_e . h[p]
//   sepia_pf_combine  y[t] = sum_k w[t][k] yp[t * n_sel + k], slot order
// The projections dequantize 128-column tiles of their weights with the
// bit-exact decoders (decode.h) from raw blocks staged in LDS, split every
// weight and activation into bf16 hi + lo (hi = bf16(v), lo = bf16(v - hi),
// together within 2^-17 |v|) and run v_mfma_f32_16x16x32_bf16 three times
// per step (hi.hi + hi.lo + lo.hi), accumulating in f32. A single bf16 term
// would miss the 1e-4 ||y||_inf bar by an order of magnitude. Results do not
// depend on how pairs are grouped into units: every output element is its
// own dot product in a fixed column order.
#pragma once
#include "common.h"
#include "decode.h"
#include "route.h"

typedef __bf16 pf_bf16x8 __attribute__((ext_vector_type(8)));
typedef float pf_f32x4 __attribute__((ext_vector_type(4)));

#define PF_MT 32     // pairs per unit (two 16-row M tiles)
#define PF_KC 128    // columns per staged tile (half a 256-column block)
#define PF_LD 136    // LDS row stride of bf16 tiles (PF_KC + 8: conflict-free fragment reads)

// ------------------------------------------------------------- router ----
// logits[t][r] = sum_k x[t][k] * Rw[r][k]: 32 tokens x 32 rows per
// workgroup, 64-column chunks through LDS; thread (ty, tx) owns tokens
// 2ty, 2ty + 1 and rows 2tx, 2tx + 1, each an FMA chain in column order.
extern "C" __global__ __launch_bounds__(256) void sepia_pf_route(const float *__restrict__ x, int64_t T,
                                                                 const float *__restrict__ rw, int64_t ld,
                                                                 int64_t n_tot, int64_t H, float *__restrict__ logits) {
    __shared__ float xs[32][65], ws[32][65];
    const int tid = threadIdx.x, ty = tid >> 4, tx = tid & 15;
    const int64_t t0 = (int64_t)blockIdx.x * 32, r0 = (int64_t)blockIdx.y * 32;
    float acc[2][2] = {{0.0f, 0.0f}, {0.0f, 0.0f}};
    for (int64_t k0 = 0; k0 < H; k0 += 64) {
        for (int i = tid; i < 32 * 64; i += 256) {
            const int rr = i >> 6, c = i & 63;
            const int64_t k = k0 + c;
            xs[rr][c] = (t0 + rr < T && k < H) ? x[(t0 + rr) * H + k] : 0.0f;
            ws[rr][c] = (r0 + rr < n_tot && k < H) ? rw[(r0 + rr) * ld + k] : 0.0f;
        }
        __syncthreads();
#pragma unroll 8
        for (int c = 0; c < 64; c++) {
#pragma unroll
            for (int a = 0; a < 2; a++)
#pragma unroll
                for (int b = 0; b < 2; b++) acc[a][b] = __builtin_fmaf(xs[2 * ty + a][c], ws[2 * tx + b][c], acc[a][b]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 2; b++) {
            const int64_t t = t0 + 2 * ty + a, r = r0 + 2 * tx + b;
            if (t < T && r < n_tot) logits[t * n_tot + r] = acc[a][b];
        }
}

// One wave per token (route.h).
extern "C" __global__ __launch_bounds__(64) void sepia_pf_select(const float *__restrict__ logits,
                                                                 const float *__restrict__ bias, int32_t n_routed,
                                                                 int32_t n_shared, int32_t topk, float route_scale,
                                                                 float global_scale, int32_t *__restrict__ idx,
                                                                 float *__restrict__ w) {
    const int64_t t = blockIdx.x;
    const int n_sel = topk + n_shared;
    route_pick_any<false>(logits + t * (n_routed + n_shared), bias, n_routed, n_shared, topk, route_scale,
                          global_scale, idx + t * topk, w + t * n_sel);
}

// ------------------------------------------------------------- grouping --
// One workgroup. Pairs p = t * n_sel + k: expert idx[t][k] for k < topk,
// n_routed + (k - topk) after. list[] holds the pairs grouped by expert
// (ascending expert; within an expert in arrival order, which does not
// affect any result), units[u] = {expert, first list position, count <=
// PF_MT}, n_units[0] their number. E = n_routed + n_shared <= 1088.
extern "C" __global__ __launch_bounds__(1024) void sepia_pf_group(const int32_t *__restrict__ idx, int64_t T,
                                                                  int32_t n_routed, int32_t n_shared, int32_t topk,
                                                                  int32_t *__restrict__ list,
                                                                  int32_t *__restrict__ units,
                                                                  int32_t *__restrict__ n_units) {
    __shared__ int32_t cnt[1088], off[1089], fill[1088], uoff[1089];
    const int E = n_routed + n_shared, n_sel = topk + n_shared;
    const int64_t P = T * n_sel;
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
        cnt[e] = 0;
        fill[e] = 0;
    }
    __syncthreads();
    auto expert_of = [&](int64_t p) {
        const int64_t t = p / n_sel;
        const int k = (int)(p - t * n_sel);
        return k < topk ? idx[t * topk + k] : n_routed + (k - topk);
    };
    for (int64_t p = threadIdx.x; p < P; p += blockDim.x) atomicAdd(&cnt[expert_of(p)], 1);
    __syncthreads();
    if (threadIdx.x == 0) {
        int a = 0, u = 0;
        for (int e = 0; e < E; e++) {
            off[e] = a;
            uoff[e] = u;
            a += cnt[e];
            u += (cnt[e] + PF_MT - 1) / PF_MT;
        }
        off[E] = a;
        uoff[E] = u;
        n_units[0] = u;
    }
    __syncthreads();
    for (int64_t p = threadIdx.x; p < P; p += blockDim.x) {
        const int e = expert_of(p);
        list[off[e] + atomicAdd(&fill[e], 1)] = (int32_t)p;
    }
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
        for (int j = 0; j < (cnt[e] + PF_MT - 1) / PF_MT; j++) {
            int32_t *un = units + 3 * (uoff[e] + j);
            un[0] = e;
            un[1] = off[e] + PF_MT * j;
            un[2] = cnt[e] - PF_MT * j < PF_MT ? cnt[e] - PF_MT * j : PF_MT;
        }
    }
}

// --------------------------------------------------------- tile helpers --
// v = hi + lo with hi = bf16(v), lo = bf16(v - hi) (round to nearest even).
__device__ __forceinline__ void pf_split(float v, __bf16 &hi, __bf16 &lo) {
    hi = (__bf16)v;
    lo = (__bf16)(v - (float)hi);
}

// Stage PF_KC columns [k0, k0 + PF_KC) of nr f32 rows (row i at src_row(i),
// zero rows beyond nv) as bf16 hi / lo tiles [32][PF_LD].
template <class RowFn>
__device__ __forceinline__ void pf_stage_act(const RowFn &src_row, int nv, int64_t k0, __bf16 (*ah)[PF_LD],
                                             __bf16 (*al)[PF_LD]) {
    for (int i = threadIdx.x; i < 32 * (PF_KC / 4); i += blockDim.x) {
        const int m = i / (PF_KC / 4), c4 = i - m * (PF_KC / 4);
        float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (m < nv) v = *(const float4 *)(src_row(m) + k0 + 4 * c4);
        const float a[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 4; j++) pf_split(a[j], ah[m][4 * c4 + j], al[m][4 * c4 + j]);
    }
}

// Raw bytes of block blk of rows r0 .. r0 + nr - 1 (rows past `rows` repeat
// the last one) into LDS, 2 bytes at a time (blocks are 2-byte aligned).
template <int T>
__device__ __forceinline__ void pf_stage_raw(const uint8_t *W, uint64_t row_bytes, int64_t rows, int64_t r0, int nr,
                                             int64_t blk, uint8_t *raw) {
    constexpr int bb = Fmt<T>::bytes, hw = bb / 2;
    for (int i = threadIdx.x; i < nr * hw; i += blockDim.x) {
        const int r = i / hw, c = i - r * hw;
        int64_t row = r0 + r;
        row = row < rows ? row : rows - 1;
        ((uint16_t *)raw)[r * hw + c] = *(const uint16_t *)(W + row * row_bytes + blk * bb + 2 * c);
    }
}

// Dequantize parts h4 .. h4 + 3 (PF_KC columns) of the nr staged blocks to
// bf16 hi / lo tiles [nr][PF_LD]: thread i takes part i % 4 of row i / 4.
template <int T>
__device__ __forceinline__ void pf_dequant(const uint8_t *raw, int nr, int h4, __bf16 (*bh)[PF_LD],
                                           __bf16 (*bl)[PF_LD]) {
    for (int i = threadIdx.x; i < nr * 4; i += blockDim.x) {
        const int r = i >> 2, q = i & 3;
        float v[32];
        decode_part<T>(raw + r * Fmt<T>::bytes, h4 + q, v);
#pragma unroll
        for (int j = 0; j < 32; j++) pf_split(v[j], bh[r][32 * q + j], bl[r][32 * q + j]);
    }
}

// acc += A[m0 .. m0+15][.] . B[n0 .. n0+15][.]^T over the staged PF_KC
// columns, three MFMAs (hi.hi, hi.lo, lo.hi) per 32 columns.
__device__ __forceinline__ void pf_mma(pf_f32x4 &acc, __bf16 (*ah)[PF_LD], __bf16 (*al)[PF_LD], int m0,
                                       __bf16 (*bh)[PF_LD], __bf16 (*bl)[PF_LD], int n0) {
    const int l = threadIdx.x & 63, r = l & 15, kq = 8 * (l >> 4);
#pragma unroll
    for (int kk = 0; kk < PF_KC; kk += 32) {
        const pf_bf16x8 a_h = *(const pf_bf16x8 *)&ah[m0 + r][kk + kq];
        const pf_bf16x8 a_l = *(const pf_bf16x8 *)&al[m0 + r][kk + kq];
        const pf_bf16x8 b_h = *(const pf_bf16x8 *)&bh[n0 + r][kk + kq];
        const pf_bf16x8 b_l = *(const pf_bf16x8 *)&bl[n0 + r][kk + kq];
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_h, b_h, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_h, b_l, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_l, b_h, acc, 0, 0, 0);
    }
}

// One projection family of a stack of experts (as MqProj in mq.h).
struct PfProj {
    const uint8_t *base;
    uint64_t stride;
    uint64_t row_bytes;
    int64_t n_blocks;
    int32_t type;
    int32_t pad;
};

// ------------------------------------------------------------- gate/up ---
// Workgroup (unit u, rows 32 by .. 32 by + 31 of I): wave w computes the
// 16x16 tile (pairs 16 (w >> 1) .., rows 16 (w & 1) ..) of gate and of up;
// h[p][row] = silu(gate) * up.
// LDS of the gate/up workgroup (one set for every format).
struct PfGuLds {
    __bf16 ah[32][PF_LD], al[32][PF_LD];
    __bf16 gh[32][PF_LD], gl[32][PF_LD], uh[32][PF_LD], ul[32][PF_LD];
    uint8_t rawg[32 * 212], rawu[32 * 212];
};

template <int T>
__device__ __forceinline__ void pf_gateup_t(PfGuLds &S, const uint8_t *Wg, const uint8_t *Wu, uint64_t row_bytes,
                                            int64_t nb, int64_t I, int64_t H, const float *__restrict__ x, int n_sel,
                                            const int32_t *pairs, int nv, int64_t r0, float *__restrict__ h) {
    auto &ah = S.ah, &al = S.al, &gh = S.gh, &gl = S.gl, &uh = S.uh, &ul = S.ul;
    uint8_t *rawg = S.rawg, *rawu = S.rawu;
    const int w = threadIdx.x >> 6, m0 = 16 * (w >> 1), n0 = 16 * (w & 1);
    pf_f32x4 g = {0.0f, 0.0f, 0.0f, 0.0f}, u = {0.0f, 0.0f, 0.0f, 0.0f};
    auto xrow = [&](int m) { return x + (int64_t)(pairs[m] / n_sel) * H; };
    for (int64_t blk = 0; blk < nb; blk++) {
        pf_stage_raw<T>(Wg, row_bytes, I, r0, 32, blk, rawg);
        pf_stage_raw<T>(Wu, row_bytes, I, r0, 32, blk, rawu);
        __syncthreads();
        for (int h4 = 0; h4 < 8; h4 += 4) {
            pf_stage_act(xrow, nv, blk * 256 + 32 * h4, ah, al);
            pf_dequant<T>(rawg, 32, h4, gh, gl);
            pf_dequant<T>(rawu, 32, h4, uh, ul);
            __syncthreads();
            pf_mma(g, ah, al, m0, gh, gl, n0);
            pf_mma(u, ah, al, m0, uh, ul, n0);
            __syncthreads();
        }
    }
    const int l = threadIdx.x & 63;
    const int64_t row = r0 + n0 + (l & 15);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int m = m0 + 4 * (l >> 4) + i;
        if (m < nv && row < I) h[(int64_t)pairs[m] * I + row] = silu_f32(g[i]) * u[i];
    }
}

extern "C" __global__ __launch_bounds__(256) void sepia_pf_gateup(
    PfProj gate, PfProj up, PfProj s_gate, PfProj s_up, int32_t n_routed, int32_t n_sel, int64_t I, int64_t H,
    const float *__restrict__ x, const int32_t *__restrict__ list, const int32_t *__restrict__ units,
    const int32_t *__restrict__ n_units, float *__restrict__ h) {
    if ((int32_t)blockIdx.x >= n_units[0]) return;
    const int32_t *un = units + 3 * blockIdx.x;
    const int32_t e = un[0], nv = un[2];
    const int32_t *pairs = list + un[1];
    const bool routed = e < n_routed;
    const PfProj &G = routed ? gate : s_gate, &U = routed ? up : s_up;
    const int64_t ei = routed ? e : e - n_routed;
    const uint8_t *wg = G.base + ei * G.stride, *wu = U.base + ei * U.stride;
    const int64_t r0 = (int64_t)blockIdx.y * 32;
    __shared__ __attribute__((aligned(16))) PfGuLds S;
    switch (G.type) {
#define PF_GU(TT) case TT: pf_gateup_t<TT>(S, wg, wu, G.row_bytes, G.n_blocks, I, H, x, n_sel, pairs, nv, r0, h); break;
        PF_GU(ST_Q2_K) PF_GU(ST_Q3_K) PF_GU(ST_Q4_K) PF_GU(ST_Q5_K) PF_GU(ST_Q6_K)
        PF_GU(ST_IQ2_XS) PF_GU(ST_IQ3_XXS) PF_GU(ST_IQ4_XS)
#undef PF_GU
    default: break;
    }
}

// ---------------------------------------------------------------- down ---
// Workgroup (unit u, rows 64 by .. 64 by + 63 of H): wave w computes the
// rows 16 w .. for both 16-pair M tiles; yp[p][row] = down . h[p].
// LDS of the down workgroup.
struct PfDnLds {
    __bf16 ah[32][PF_LD], al[32][PF_LD];
    __bf16 bh[64][PF_LD], bl[64][PF_LD];
    uint8_t raw[64 * 212];
};

template <int T>
__device__ __forceinline__ void pf_down_t(PfDnLds &S, const uint8_t *Wd, uint64_t row_bytes, int64_t nb, int64_t I,
                                          int64_t H, const float *__restrict__ h, const int32_t *pairs, int nv,
                                          int64_t r0, float *__restrict__ yp) {
    auto &ah = S.ah, &al = S.al;
    auto &bh = S.bh, &bl = S.bl;
    uint8_t *raw = S.raw;
    const int w = threadIdx.x >> 6, n0 = 16 * w;
    pf_f32x4 acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
    auto hrow = [&](int m) { return h + (int64_t)pairs[m] * I; };
    for (int64_t blk = 0; blk < nb; blk++) {
        pf_stage_raw<T>(Wd, row_bytes, H, r0, 64, blk, raw);
        __syncthreads();
        for (int h4 = 0; h4 < 8; h4 += 4) {
            pf_stage_act(hrow, nv, blk * 256 + 32 * h4, ah, al);
            pf_dequant<T>(raw, 64, h4, bh, bl);
            __syncthreads();
            pf_mma(acc0, ah, al, 0, bh, bl, n0);
            pf_mma(acc1, ah, al, 16, bh, bl, n0);
            __syncthreads();
        }
    }
    const int l = threadIdx.x & 63;
    const int64_t row = r0 + n0 + (l & 15);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int m = 4 * (l >> 4) + i;
        if (m < nv && row < H) yp[(int64_t)pairs[m] * H + row] = acc0[i];
        if (m + 16 < nv && row < H) yp[(int64_t)pairs[m + 16] * H + row] = acc1[i];
    }
}

extern "C" __global__ __launch_bounds__(256) void sepia_pf_down(
    PfProj down, PfProj s_down, int32_t n_routed, int64_t I, int64_t H, const float *__restrict__ h,
    const int32_t *__restrict__ list, const int32_t *__restrict__ units, const int32_t *__restrict__ n_units,
    float *__restrict__ yp) {
    if ((int32_t)blockIdx.x >= n_units[0]) return;
    const int32_t *un = units + 3 * blockIdx.x;
    const int32_t e = un[0], nv = un[2];
    const int32_t *pairs = list + un[1];
    const bool routed = e < n_routed;
    const PfProj &D = routed ? down : s_down;
    const int64_t ei = routed ? e : e - n_routed;
    const uint8_t *wd = D.base + ei * D.stride;
    const int64_t r0 = (int64_t)blockIdx.y * 64;
    __shared__ __attribute__((aligned(16))) PfDnLds S;
    switch (D.type) {
#define PF_DN(TT) case TT: pf_down_t<TT>(S, wd, D.row_bytes, D.n_blocks, I, H, h, pairs, nv, r0, yp); break;
        PF_DN(ST_Q2_K) PF_DN(ST_Q3_K) PF_DN(ST_Q4_K) PF_DN(ST_Q5_K) PF_DN(ST_Q6_K)
        PF_DN(ST_IQ2_XS) PF_DN(ST_IQ3_XXS) PF_DN(ST_IQ4_XS)
#undef PF_DN
    default: break;
    }
}

// ------------------------------------------------------------- combine ---
// y[t][d] = sum_{k < n_sel} w[t][k] * yp[t * n_sel + k][d], in slot order
// (routed weights, then the shared gammas, applied to the down output as
// src/sepia.c:3953-3957 does).
extern "C" __global__ __launch_bounds__(256) void sepia_pf_combine(const float *__restrict__ yp,
                                                                   const float *__restrict__ w, int32_t n_sel,
                                                                   int64_t T, int64_t H, float *__restrict__ y) {
    const int64_t t = blockIdx.y, d = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= T || d >= H) return;
    float acc = 0.0f;
    for (int k = 0; k < n_sel; k++) acc = __builtin_fmaf(w[t * n_sel + k], yp[(t * n_sel + k) * H + d], acc);
    y[t * H + d] = acc;
}
