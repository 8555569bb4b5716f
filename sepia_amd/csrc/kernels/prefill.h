// prefill.h -- the MoE layer for a batch of tokens (prefill), grouped by
// expert, on the bf16 matrix cores.
//
// Every token gets exactly the decode path's result (reference
// src/sepia.c:1377-1470 per token): the same router logits up to f32
// summation order, the same selection (route.h), then
//   y[t] = sum_{k < topk} w[t][k] down_e(silu(gate_e x_t) * up_e x_t)
//        + sum_s w[t][topk + s] down_s(silu(gate_s x_t) * up_s x_t).
// Launches:
//   sepia_pf_route(_m) logits[T][n_routed + n_shared] = x . Rw^T (f32 tiles,
//                     or the f32 matrix cores)
//   sepia_pf_select   one wave per token: idx[T][topk], w[T][topk + n_shared]
//   sepia_pf_group    one workgroup: the (token, slot) pairs p = t * n_sel + k
//                     sorted by expert (shared expert s is expert
//                     n_routed + s) and cut into units of <= 32 pairs
//   projections       a layer whose six projections are all Q2_K, Q3_K or
//                     Q4_K runs them on the int8 matrix cores (prefill_q.h:
//                     sepia_pf_quant, sepia_pf_gateup_q, sepia_pf_down_q);
//                     any other layer on the bf16 matrix cores here:
//     sepia_pf_split    x as bf16 hi / lo
//     sepia_pf_gateup   per (32-row tile, unit): h[p][.] = silu(g) * u (bf16 hi / lo)
//     sepia_pf_down     per (64-row tile, unit): yp[p][.] = down_e . h[p]
//   sepia_pf_combine  y[t] = sum_k w[t][k] yp[t * n_sel + k], slot order
// The bf16 projections stream raw weight blocks and the unit's activation
// rows into LDS by DMA ahead of use, dequantize the weights bit-exactly into
// bf16 hi + lo tiles and run the bf16 matrix cores with f32 accumulation;
// activations are hi + lo too (hi = bf16(v), lo = bf16(v - hi), together
// within 2^-17 |v|; a single bf16 term would miss the 1e-4 ||y||_inf bar by
// an order of magnitude), three MFMAs per 32 columns (hi.hi + hi.lo + lo.hi).
// Results do not depend on how pairs are grouped into units: every output
// element is its own dot product in a fixed column order.
#pragma once
#include "common.h"
#include "decode.h"
#include "mq.h"
#include "route.h"

typedef __bf16 pf_bf16x8 __attribute__((ext_vector_type(8)));
typedef float pf_f32x4 __attribute__((ext_vector_type(4)));

#define PF_MT 32     // pairs per unit (two 16-row M tiles)

// (row slice x, unit y) of this workgroup in a (slices x units) launch of
// a unit kernel. The hardware deals consecutive workgroup ids to the 8 XCDs
// in turn; when the unit count is a multiple of 8 the units are dealt to
// the XCDs the same way (XCD c runs units c, c + 8, ..., each over all its
// slices in a row), so the workgroups of a unit, which all read that unit's
// activation rows, share one XCD's L2. The f16 kernels use it (their C5
// layer in the real formats: 3.79 -> 3.02 ms); the int8 ones measured no
// better with it (1.90 -> 1.93 ms) and keep the launch order.
struct PfSlot {
    int32_t x, y;
};
__device__ __forceinline__ PfSlot pf_slot() {
    const uint32_t gx = gridDim.x;
    if (gridDim.y % 8u) return PfSlot{(int32_t)blockIdx.x, (int32_t)blockIdx.y};
    const uint32_t lid = blockIdx.y * gx + blockIdx.x, k = lid >> 3;
    return PfSlot{(int32_t)(k % gx), (int32_t)(8u * (k / gx) + (lid & 7u))};
}


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

// The same logits on the f32 matrix cores: one workgroup of four waves per
// 16-token x 16-row tile (grid: T / 16 x n_tot / 16), wave w taking the
// columns [w H / 4, (w + 1) H / 4) in steps of 16 (so 544 tiles of C5 keep
// every SIMD busy, with a quarter of the dependent MFMA chain each). Lane l
// loads columns 4 (l >> 4) .. + 3 of the step for token / row l & 15 as one
// float4; MFMA i of the step takes component i, so the four MFMAs cover the
// step's 16 columns once each. The four quarter sums are added in LDS in
// wave order (f32 products, f32 sums; only the summation order differs
// from sepia_pf_route). Needs x, rw and ld 16-byte aligned and H a multiple
// of 512 (the host checks).
typedef float pf_f32x4v __attribute__((ext_vector_type(4)));
extern "C" __global__ __launch_bounds__(256) void sepia_pf_route_m(const float *__restrict__ x, int64_t T,
                                                                   const float *__restrict__ rw, int64_t ld,
                                                                   int64_t n_tot, int64_t H, float *__restrict__ logits) {
    __shared__ pf_f32x4 part[3][64];
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63, r = l & 15, g = l >> 4;
    const int64_t t0 = (int64_t)blockIdx.x * 16, r0 = (int64_t)blockIdx.y * 16;
    const int64_t t = t0 + r < T ? t0 + r : T - 1, rr = r0 + r < n_tot ? r0 + r : n_tot - 1;
    const int64_t c0 = (int64_t)w * (H / 4);
    const pf_f32x4v *xa = (const pf_f32x4v *)(x + t * H + c0) + g, *wa = (const pf_f32x4v *)(rw + rr * ld + c0) + g;
    pf_f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    // eight steps in registers while the next eight load (n a multiple of 8)
    const int64_t n = H / 64;
    pf_f32x4v a[8], b[8];
#pragma unroll
    for (int u = 0; u < 8; u++) {
        a[u] = xa[4 * u];
        b[u] = wa[4 * u];
    }
    for (int64_t k = 0; k < n; k += 8) {
        pf_f32x4v a2[8], b2[8];
        const bool more = k + 8 < n;
        if (more) {
#pragma unroll
            for (int u = 0; u < 8; u++) {
                a2[u] = xa[4 * (k + 8 + u)];
                b2[u] = wa[4 * (k + 8 + u)];
            }
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
#pragma unroll
            for (int i = 0; i < 4; i++) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u][i], b[u][i], acc, 0, 0, 0);
        }
        if (more) {
#pragma unroll
            for (int u = 0; u < 8; u++) {
                a[u] = a2[u];
                b[u] = b2[u];
            }
        }
    }
    // acc[i]: token t0 + 4 g + i, row r0 + r; quarters 1..3 to LDS, added to quarter 0 in order
    if (w > 0) part[w - 1][l] = acc;
    __syncthreads();
    if (w > 0) return;
#pragma unroll
    for (int q = 0; q < 3; q++) {
        const pf_f32x4 v = part[q][l];
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i] += v[i];
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int64_t tt = t0 + 4 * g + i, ro = r0 + r;
        if (tt < T && ro < n_tot) logits[tt * n_tot + ro] = acc[i];
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

// ---------------------------------------------------- activations split --
// hi[i] = bf16(x[i]), lo[i] = bf16(x[i] - hi[i]) (round to nearest even).
__device__ __forceinline__ void pf_split(float v, __bf16 &hi, __bf16 &lo) {
    hi = (__bf16)v;
    lo = (__bf16)(v - (float)hi);
}
// Segment i (16 values) of x: hi / lo as above.
extern "C" __global__ __launch_bounds__(256) void sepia_pf_split(const float *__restrict__ x, int64_t n_seg,
                                                                 __bf16 *__restrict__ hi, __bf16 *__restrict__ lo) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n_seg) return;
    const float4 *x4 = (const float4 *)(x + 16 * i);
    float v[16];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const float4 t = x4[c];
        v[4 * c] = t.x;
        v[4 * c + 1] = t.y;
        v[4 * c + 2] = t.z;
        v[4 * c + 3] = t.w;
    }
    __bf16 h[16], l[16];
#pragma unroll
    for (int k = 0; k < 16; k++) pf_split(v[k], h[k], l[k]);
    uint4 *ho = (uint4 *)(hi + 16 * i), *lw = (uint4 *)(lo + 16 * i);
    ho[0] = ((const uint4 *)h)[0];
    ho[1] = ((const uint4 *)h)[1];
    lw[0] = ((const uint4 *)l)[0];
    lw[1] = ((const uint4 *)l)[1];
}

// ----------------------------------------------------------- pipelines ---
// A projection workgroup computes a 32-pair x R-row tile (R = 32 gate and
// 32 up rows, or 64 down rows) over K = the projection's input width, one
// 256-column block per step:
//   step b: wait for block b's DMAs; issue block b + 1's (activations as
//           bf16 hi / lo rows, weights as raw blocks); dequantize block b's
//           raw weights (bit-exact decoders) into bf16 hi / lo tiles; three
//           MFMAs per 32 columns (hi.hi + hi.lo + lo.hi).
// Everything a step reads arrives by LDS DMA one step ahead, so the loads
// of block b + 1 fly while block b computes.
// Tiles are [rows][256] bf16 with 512-byte rows; the 16-byte chunk c of row
// r sits at chunk c ^ (r & 15), so the 16 rows of an MFMA fragment read hit
// 16 different bank groups.
#define PF_RDMAX 54   // dwords of a staged raw block window (Q6_K: 210 bytes + misalignment)
#define PF_TILE 16384 // bytes of a [32][256] bf16 tile

__device__ __forceinline__ uint32_t pf_lds(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)p;
}
__device__ __forceinline__ const uint8_t *pf_uniform(const void *p) {
    const uint64_t b = (uint64_t)(uintptr_t)p;
    return (const uint8_t *)(uintptr_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32))
                                         << 32) |
                                        (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b));
}
// LDS DMA: lane l's 16 (or 4) bytes at base + voff land at lds + 16 l (4 l),
// after the five wait states of SEPIA_DMA_WAIT (mq.h: a VALU write of the
// base's SGPRs or an SALU write of M0 may come right before the asm).
__device__ __forceinline__ void pf_dma16(const void *base, uint32_t voff, uint32_t lds) {
    asm volatile(SEPIA_DMA_WAIT "global_load_lds_dwordx4 %0, %1" : : "v"(voff), "s"(pf_uniform(base)), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ void pf_dma4(const void *base, uint32_t voff, uint32_t lds) {
    asm volatile(SEPIA_DMA_WAIT "global_load_lds_dword %0, %1" : : "v"(voff), "s"(pf_uniform(base)), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ uint32_t pf_swz(int r, int chunk) { return (uint32_t)r * 512u + ((uint32_t)(chunk ^ (r & 15)) << 4); }

// Activation rows of the unit into a tile pair (hi, lo) at dst: row m comes
// from element offset roff[m] (bf16 units) + 256 b of src_hi / src_lo. One
// wave instruction moves two rows of one of the two tiles.
__device__ __forceinline__ void pf_issue_act(const __bf16 *src_hi, const __bf16 *src_lo, const uint32_t *roff,
                                             int64_t b, uint8_t *dst, bool with_lo = true) {
    const int nw = (int)(blockDim.x >> 6), w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    for (int j = w; j < (with_lo ? 32 : 16); j += nw) {
        const int hl = j >> 4, rp = j & 15, row = 2 * rp + (lane >> 5), p = lane & 31;
        const uint32_t voff = 2u * (roff[row] + 256u * (uint32_t)b) + ((uint32_t)(p ^ (row & 15)) << 4);
        pf_dma16(hl ? (const void *)src_lo : (const void *)src_hi, voff, pf_lds(dst + hl * PF_TILE + 2 * rp * 512));
    }
}

// Raw blocks b of nr rows (rows r0 .. r0 + nr - 1 of a matrix of `rows`
// rows; rows past the end repeat the last one) into dst, row k at k * 4 RD:
// each row's 4-byte-aligned window that holds the block.
template <int T>
__device__ __forceinline__ void pf_issue_raw(const uint8_t *W, uint64_t row_bytes, int64_t rows, int64_t r0, int nr,
                                             int64_t b, uint8_t *dst) {
    constexpr int BB = Fmt<T>::bytes, RD = (BB + 6) / 4;
    const int nw = (int)(blockDim.x >> 6), w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const uint8_t *Wa = (const uint8_t *)((uintptr_t)W & ~(uintptr_t)3);
    const uint32_t delta = (uint32_t)((uintptr_t)W & 3);
    const int n_ins = (nr * RD + 63) >> 6;
    for (int j = w; j < n_ins; j += nw) {
        const int i = 64 * j + lane;
        if (i < nr * RD) {
            const int r = i / RD, d = i - r * RD;
            int64_t rr = r0 + r;
            rr = rr < rows ? rr : rows - 1;
            const uint64_t off = delta + (uint64_t)rr * row_bytes + (uint64_t)b * BB;
            pf_dma4(Wa, (uint32_t)(off & ~(uint64_t)3) + 4u * (uint32_t)d, pf_lds(dst + 256 * j));
        }
    }
}

// Dequantize the staged raw blocks into bf16 (hi, lo) tiles: nper rows of
// W0 into dst0 and, with W1, nper rows of W1 (staged after them) into dst1;
// each lo tile lies lo_off bytes after its hi tile. 64 rows x 8 parts of
// 32 weights: one part per thread at 512 threads.
template <int T>
__device__ __forceinline__ void pf_dequant_raw(const uint8_t *raw, const uint8_t *W0, const uint8_t *W1, int nper,
                                               uint64_t row_bytes, int64_t rows, int64_t r0, int64_t b, uint8_t *dst0,
                                               uint8_t *dst1, uint32_t lo_off) {
    constexpr int BB = Fmt<T>::bytes, RD = (BB + 6) / 4;
    const int nr = W1 ? 2 * nper : nper;
    for (int i = threadIdx.x; i < nr * 8; i += blockDim.x) {
        const int q = i & 7, rg = i >> 3;
        const int mat = rg >= nper, r = rg - mat * nper;
        const uint8_t *W = mat ? W1 : W0;
        int64_t rr = r0 + r;
        rr = rr < rows ? rr : rows - 1;
        const uint32_t mis = (uint32_t)(((uintptr_t)W & 3) + (uint64_t)rr * row_bytes + (uint64_t)b * BB) & 3u;
        float v[32];
        decode_part<T>(raw + (size_t)(mat * nper + r) * RD * 4 + mis, q, v);
        uint8_t *dst = mat ? dst1 : dst0;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            __bf16 hh[8], ll[8];
#pragma unroll
            for (int j = 0; j < 8; j++) pf_split(v[8 * c + j], hh[j], ll[j]);
            const uint32_t o = pf_swz(r, 4 * q + c);
            *(uint4 *)(dst + o) = *(const uint4 *)hh;
            *(uint4 *)(dst + lo_off + o) = *(const uint4 *)ll;
        }
    }
}

// acc += A[m0 .. m0 + 15][.] . B[n0 .. n0 + 15][.]^T over the 256 staged
// columns (A: a 32-row tile pair hi, lo; B: hi tile, its lo b_lo bytes on).
__device__ __forceinline__ void pf_mma256(pf_f32x4 &acc, const uint8_t *A, int m0, const uint8_t *B, int n0,
                                          uint32_t b_lo) {
    const int l = threadIdx.x & 63, r = l & 15, g = l >> 4;
#pragma unroll
    for (int kk = 0; kk < 256; kk += 32) {
        const uint32_t oa = pf_swz(m0 + r, kk / 8 + g), ob = pf_swz(n0 + r, kk / 8 + g);
        const pf_bf16x8 a_h = *(const pf_bf16x8 *)(A + oa), a_l = *(const pf_bf16x8 *)(A + PF_TILE + oa);
        const pf_bf16x8 b_h = *(const pf_bf16x8 *)(B + ob), b_l = *(const pf_bf16x8 *)(B + b_lo + ob);
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

// LDS of both projection kernels (PF_LDS_BYTES, dynamic): two activation
// tile pairs (steps b, b + 1), the weight tile pairs, two raw areas.
#define PF_O_B (4 * PF_TILE)
#define PF_O_RAW (8 * PF_TILE)
#define PF_RAW_BYTES (64 * PF_RDMAX * 4)
#define PF_LDS_BYTES 163840                        // the whole 160 KB
#define PF_O_ROFF (PF_LDS_BYTES - 2 * PF_MT * 4)   // row tables at the top (both paths)

// ------------------------------------------------------------- gate/up ---
// Workgroup (rows 32 bx .. 32 bx + 31 of I, unit by), 8 waves: wave w
// computes the 16x16 tile (pairs 16 ((w >> 1) & 1) .., rows 16 (w & 1) ..)
// of gate (w < 4) or up (w >= 4); the up waves hand their tile to the gate
// waves through LDS, which store h[p][row] = silu(gate) * up as bf16 hi / lo
// for the down kernel. The grid runs a unit's row tiles side by side, so
// its activation rows stay in L2.
template <int T>
__device__ __forceinline__ void pf_gateup_t(uint8_t *smem, const uint8_t *Wg, const uint8_t *Wu, uint64_t row_bytes,
                                            int64_t nb, int64_t I, const __bf16 *xh, const __bf16 *xl,
                                            const uint32_t *roff, const int32_t *pair, int nv, int64_t r0,
                                            __bf16 *__restrict__ hh, __bf16 *__restrict__ hl) {
    const int w = threadIdx.x >> 6, m0 = 16 * ((w >> 1) & 1), n0 = 16 * (w & 1), up_w = w >> 2;
    uint8_t *Bg = smem + PF_O_B, *Bu = smem + PF_O_B + 2 * PF_TILE;
    pf_f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    auto issue = [&](int64_t b) {
        const int buf = (int)(b & 1);
        pf_issue_act(xh, xl, roff, b, smem + buf * 2 * PF_TILE);
        uint8_t *raw = smem + PF_O_RAW + buf * PF_RAW_BYTES;
        pf_issue_raw<T>(Wg, row_bytes, I, r0, 32, b, raw);
        pf_issue_raw<T>(Wu, row_bytes, I, r0, 32, b, raw + 32 * ((Fmt<T>::bytes + 6) / 4) * 4);
    };
    issue(0);
    for (int64_t b = 0; b < nb; b++) {
        __builtin_amdgcn_s_waitcnt(0);   // this wave's DMAs of step b
        __syncthreads();                 // everyone's, and step b - 1's reads are done
        if (b + 1 < nb) issue(b + 1);
        const int buf = (int)(b & 1);
        pf_dequant_raw<T>(smem + PF_O_RAW + buf * PF_RAW_BYTES, Wg, Wu, 32, row_bytes, I, r0, b, Bg, Bu, PF_TILE);
        __syncthreads();
        const uint8_t *A = smem + buf * 2 * PF_TILE;
        pf_mma256(acc, A, m0, up_w ? Bu : Bg, n0, PF_TILE);
    }
    // the up tiles through LDS (the raw areas are free now)
    __syncthreads();
    const int l = threadIdx.x & 63;
    float *xch = (float *)(smem + PF_O_RAW) + (w & 3) * 256 + l * 4;
    if (up_w) *(pf_f32x4 *)xch = acc;
    __syncthreads();
    if (up_w) return;
    const pf_f32x4 u = *(const pf_f32x4 *)xch;
    const int64_t row = r0 + n0 + (l & 15);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int m = m0 + 4 * (l >> 4) + i;
        if (m < nv && row < I) {
            __bf16 a, c;
            pf_split(silu_f32(acc[i]) * u[i], a, c);
            hh[(int64_t)pair[m] * I + row] = a;
            hl[(int64_t)pair[m] * I + row] = c;
        }
    }
}

// vmcnt(n) for a run-time n (0 .. 63).
__device__ __forceinline__ void pf_wait_vm(int n) {
    switch (n) {
#define PF_W(k) case k: __builtin_amdgcn_s_waitcnt(mq_wc_vm(k)); break;
        PF_W(0) PF_W(1) PF_W(2) PF_W(3) PF_W(4) PF_W(5) PF_W(6) PF_W(7) PF_W(8) PF_W(9) PF_W(10) PF_W(11)
        PF_W(12) PF_W(13) PF_W(14) PF_W(15) PF_W(16) PF_W(17) PF_W(18) PF_W(19) PF_W(20) PF_W(21) PF_W(22)
        PF_W(23) PF_W(24) PF_W(25) PF_W(26) PF_W(27) PF_W(28) PF_W(29) PF_W(30) PF_W(31) PF_W(32) PF_W(33)
        PF_W(34) PF_W(35) PF_W(36) PF_W(37) PF_W(38) PF_W(39) PF_W(40) PF_W(41) PF_W(42) PF_W(43) PF_W(44)
        PF_W(45) PF_W(46) PF_W(47)
#undef PF_W
    default: __builtin_amdgcn_s_waitcnt(mq_wc_vm(0)); break;
    }
}
// The unit's rows: roff[m] = element offset of pair m's activation row (rows
// past nv repeat row 0), pair[m] its pair index.
__device__ __forceinline__ void pf_unit_rows(const int32_t *pairs, int nv, bool by_token, int32_t n_sel, int64_t ld,
                                             uint8_t *smem, uint32_t *&roff, int32_t *&pair) {
    roff = (uint32_t *)(smem + PF_O_ROFF);
    pair = (int32_t *)(roff + PF_MT);
    if (threadIdx.x < PF_MT) {
        const int m = threadIdx.x < (unsigned)nv ? (int)threadIdx.x : 0;
        const int32_t p = pairs[m];
        pair[threadIdx.x] = p;
        roff[threadIdx.x] = (uint32_t)((by_token ? (int64_t)(p / n_sel) : (int64_t)p) * ld);
    }
    __syncthreads();
}

extern "C" __global__ __launch_bounds__(512) void sepia_pf_gateup(
    PfProj gate, PfProj up, PfProj s_gate, PfProj s_up, int32_t n_routed, int32_t n_sel, int64_t I, int64_t H,
    const __bf16 *__restrict__ xh, const __bf16 *__restrict__ xl, const int32_t *__restrict__ list,
    const int32_t *__restrict__ units,
    const int32_t *__restrict__ n_units, __bf16 *__restrict__ hh, __bf16 *__restrict__ hl) {
    if ((int32_t)blockIdx.y >= n_units[0]) return;
    extern __shared__ __attribute__((aligned(16))) uint8_t pf_smem[];
    uint8_t *smem = pf_smem;
    const int32_t *un = units + 3 * blockIdx.y;
    const int32_t e = un[0], nv = un[2];
    const bool routed = e < n_routed;
    const PfProj &G = routed ? gate : s_gate, &U = routed ? up : s_up;
    const int64_t ei = routed ? e : e - n_routed;
    const uint8_t *wg = G.base + ei * G.stride, *wu = U.base + ei * U.stride;
    const int64_t r0 = (int64_t)blockIdx.x * 32;
    uint32_t *roff;
    int32_t *pair;
    pf_unit_rows(list + un[1], nv, true, n_sel, H, smem, roff, pair);
    switch (G.type) {
#define PF_GU(TT) case TT: pf_gateup_t<TT>(smem, wg, wu, G.row_bytes, G.n_blocks, I, xh, xl, roff, pair, nv, r0, hh, hl); break;
        PF_GU(ST_Q2_K) PF_GU(ST_Q3_K) PF_GU(ST_Q4_K) PF_GU(ST_Q5_K) PF_GU(ST_Q6_K)
        PF_GU(ST_IQ2_XS) PF_GU(ST_IQ3_XXS) PF_GU(ST_IQ4_XS)
#undef PF_GU
    default: break;
    }
}

// ---------------------------------------------------------------- down ---
// Workgroup (rows 64 bx .. 64 bx + 63 of H, unit by), 8 waves: wave w
// computes rows 16 (w & 3) .. of the 16-pair M tile w >> 2;
// yp[p][row] = down . h[p].
template <int T>
__device__ __forceinline__ void pf_down_t(uint8_t *smem, const uint8_t *Wd, uint64_t row_bytes, int64_t nb, int64_t H,
                                          const __bf16 *hh, const __bf16 *hl, const uint32_t *roff, const int32_t *pair,
                                          int nv, int64_t r0, float *__restrict__ yp) {
    const int w = threadIdx.x >> 6, n0 = 16 * (w & 3), m0 = 16 * (w >> 2);
    uint8_t *Bt = smem + PF_O_B;   // [64][256] hi, then lo (2 PF_TILE on)
    pf_f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    auto issue = [&](int64_t b) {
        const int buf = (int)(b & 1);
        pf_issue_act(hh, hl, roff, b, smem + buf * 2 * PF_TILE);
        pf_issue_raw<T>(Wd, row_bytes, H, r0, 64, b, smem + PF_O_RAW + buf * PF_RAW_BYTES);
    };
    issue(0);
    for (int64_t b = 0; b < nb; b++) {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (b + 1 < nb) issue(b + 1);
        const int buf = (int)(b & 1);
        pf_dequant_raw<T>(smem + PF_O_RAW + buf * PF_RAW_BYTES, Wd, nullptr, 64, row_bytes, H, r0, b, Bt, nullptr,
                          2 * PF_TILE);
        __syncthreads();
        const uint8_t *A = smem + buf * 2 * PF_TILE;
        pf_mma256(acc, A, m0, Bt, n0, 2 * PF_TILE);
    }
    const int l = threadIdx.x & 63;
    const int64_t row = r0 + n0 + (l & 15);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int m = m0 + 4 * (l >> 4) + i;
        if (m < nv && row < H) yp[(int64_t)pair[m] * H + row] = acc[i];
    }
}

extern "C" __global__ __launch_bounds__(512) void sepia_pf_down(
    PfProj down, PfProj s_down, int32_t n_routed, int64_t I, int64_t H, const __bf16 *__restrict__ hh,
    const __bf16 *__restrict__ hl, const int32_t *__restrict__ list, const int32_t *__restrict__ units,
    const int32_t *__restrict__ n_units, float *__restrict__ yp) {
    if ((int32_t)blockIdx.y >= n_units[0]) return;
    extern __shared__ __attribute__((aligned(16))) uint8_t pf_smem[];
    uint8_t *smem = pf_smem;
    const int32_t *un = units + 3 * blockIdx.y;
    const int32_t e = un[0], nv = un[2];
    const bool routed = e < n_routed;
    const PfProj &D = routed ? down : s_down;
    const int64_t ei = routed ? e : e - n_routed;
    const uint8_t *wd = D.base + ei * D.stride;
    const int64_t r0 = (int64_t)blockIdx.x * 64;
    uint32_t *roff;
    int32_t *pair;
    pf_unit_rows(list + un[1], nv, false, 1, I, smem, roff, pair);
    switch (D.type) {
#define PF_DN(TT) case TT: pf_down_t<TT>(smem, wd, D.row_bytes, D.n_blocks, H, hh, hl, roff, pair, nv, r0, yp); break;
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
