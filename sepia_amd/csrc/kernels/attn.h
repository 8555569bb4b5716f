// attn.h -- the attention half of the GPU ABI (reference src/sepia_gpu.h:
// rel_project :209, banded_attn :226, rel_project_off :253): the dense
// relative-position projection and the banded, GQA, online-softmax
// attention of the reference's attn_forward_chunk (src/sepia.c:1203-1247),
// in f32 throughout.
//
// Banded attention is split over the kv range ("flash-decoding"): a
// workgroup takes one token, one kv head (all the query heads that share
// it, so each k and v row is read once for the group) and one span of kv
// positions, walks the span in steps of ATT_CH rows with an online softmax
// and writes a partial (max, sum, weighted v) per head; a second launch
// folds a token's partials in span order. Per kv step:
//   scores: 16 lanes per kv row, each lane 8 of the 128 dims as two 16-byte
//           loads (a row is 512 contiguous bytes), the group's q from LDS,
//           sums over the 16 lanes by shuffles;
//   softmax: one wave per head over the step's ATT_CH scores;
//   p . v:   each thread owns output dims (consecutive threads, consecutive
//           dims, so each v row is one coalesced read).
// Token bounds (kv_lo, kv_hi, tau) arrive in the kernel arguments, ATT_TB
// tokens a launch, so no transient device copy of the caller's host arrays
// is needed.
// Precision follows the reference's CPU loop: scores are f32 dot products
// plus the band bias added in double and rounded once; each weight is
// exp(score - max) rounded to f32; the running sums of weights and of
// weighted v rows are double (f32 sums over 10^5 kv rows drift past the
// reference's 2e-4 relative gate, whose floor is 1e-3 of the largest
// output).
#pragma once
#include "common.h"

#define ATT_RP_ROWS 8       // (t, h) rows per rel-project workgroup
#define ATT_RP_DCH 64       // d_rel columns staged per pass
#define ATT_CH 128          // kv rows per step
#define ATT_TB 64           // tokens per launch
#define ATT_GMAX 16         // query heads per kv head
#define ATT_DMAX 128        // head dim

// rel_logits[th, r] = sum_d r_vec[th, d] * rel_proj[d, r], an f32 FMA chain
// in d order. Grid (ceil(R / 256), ceil(TH / ATT_RP_ROWS)), 256 threads:
// thread r of the tile computes ATT_RP_ROWS rows, so each rel_proj value is
// read once per workgroup.
extern "C" __global__ __launch_bounds__(256) void sepia_rel_project_f32(
    const float *__restrict__ r_vec, const float *__restrict__ rel_proj, float *__restrict__ rel_logits,
    int64_t TH, int32_t d_rel, int32_t R) {
    __shared__ float rv[ATT_RP_ROWS][ATT_RP_DCH];
    const int64_t th0 = (int64_t)blockIdx.y * ATT_RP_ROWS;
    const int nrow = (int)(TH - th0 < ATT_RP_ROWS ? TH - th0 : ATT_RP_ROWS);
    const int r = (int)blockIdx.x * 256 + (int)threadIdx.x;
    float acc[ATT_RP_ROWS];
#pragma unroll
    for (int i = 0; i < ATT_RP_ROWS; i++) acc[i] = 0.0f;
    for (int d0 = 0; d0 < d_rel; d0 += ATT_RP_DCH) {
        const int nd = d_rel - d0 < ATT_RP_DCH ? d_rel - d0 : ATT_RP_DCH;
        __syncthreads();
        for (int i = threadIdx.x; i < ATT_RP_ROWS * ATT_RP_DCH; i += 256) {
            const int row = i / ATT_RP_DCH, d = i % ATT_RP_DCH;
            rv[row][d] = (row < nrow && d < nd) ? r_vec[(th0 + row) * d_rel + d0 + d] : 0.0f;
        }
        __syncthreads();
        if (r < R) {
            for (int d = 0; d < nd; d++) {
                const float p = rel_proj[(int64_t)(d0 + d) * R + r];
#pragma unroll
                for (int i = 0; i < ATT_RP_ROWS; i++) acc[i] = __builtin_fmaf(rv[i][d], p, acc[i]);
            }
        }
    }
    if (r >= R) return;
#pragma unroll
    for (int i = 0; i < ATT_RP_ROWS; i++)
        if (i < nrow) rel_logits[(th0 + i) * R + r] = acc[i];
}

// Bounds of the launch's tokens: kv positions [lo, hi] (inclusive) and the
// bias scale of each.
struct AttnTok {
    int32_t lo[ATT_TB], hi[ATT_TB];
    float tau[ATT_TB];
};

__device__ __forceinline__ float att_sum16(float v) {
    v += __shfl_xor(v, 8, 16);
    v += __shfl_xor(v, 4, 16);
    v += __shfl_xor(v, 2, 16);
    v += __shfl_xor(v, 1, 16);
    return v;
}
__device__ __forceinline__ float att_wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Workgroup (span x, kv head hk, token z of the launch), 256 threads: query
// heads hk G .. hk G + G - 1 of token t = t0 + z over kv positions
// [lo + x span, min(hi, lo + (x + 1) span - 1)]. Score = (q . k) *
// inv_head_dim + (dist < R ? rel_logits[t, h, dist] * tau : 0), dist =
// q_pos - kv. Partial of head h: part[((z H + h) nsplit + x) (Dh + 2) ..]
// = weighted v [Dh], then the running max and sum, as doubles. Spans past
// hi write nothing (the fold counts the spans itself).
extern "C" __global__ __launch_bounds__(256) void sepia_attn_partial(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
    const float *__restrict__ rel_logits, AttnTok tok, int32_t t0, int32_t H, int32_t Hkv, int32_t Dh, int32_t R,
    int64_t q_pos_base, int64_t kv_dim, float inv_head_dim, int32_t nsplit, int32_t span, double *__restrict__ part) {
    __shared__ float qs[ATT_GMAX * ATT_DMAX];
    __shared__ float ps[ATT_GMAX * ATT_CH];
    __shared__ float mrun[ATT_GMAX];
    __shared__ double lrun[ATT_GMAX], alpha[ATT_GMAX];
    const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int z = (int)blockIdx.z, hk = (int)blockIdx.y, x = (int)blockIdx.x;
    const int G = H / Hkv;
    const int64_t t = (int64_t)t0 + z;
    const int64_t lo = tok.lo[z], hi = tok.hi[z];
    const int64_t s0 = lo + (int64_t)x * span;
    if (s0 > hi) return;
    const int64_t s1 = hi < s0 + span - 1 ? hi : s0 + span - 1;
    const int64_t q_pos = q_pos_base + t;
    const float tau = tok.tau[z];
    for (int i = tid; i < G * Dh; i += 256) {
        const int g = i / Dh, d = i - g * Dh;
        qs[g * ATT_DMAX + d] = q[(t * H + (int64_t)hk * G + g) * Dh + d];
    }
    if (tid < G) {
        mrun[tid] = -INFINITY;
        lrun[tid] = 0.0;
    }
    // this thread's outputs o = tid + 256 i: head o / Dh, dim o % Dh
    const int n_out = G * Dh, OPT = (n_out + 255) >> 8;
    double acc[ATT_GMAX * ATT_DMAX / 256];
#pragma unroll
    for (int i = 0; i < ATT_GMAX * ATT_DMAX / 256; i++) acc[i] = 0.0;
    const int l16 = tid & 15, row16 = tid >> 4;
    const int d_a = 4 * l16, d_b = 64 + 4 * l16;
    const float *kh = k + (int64_t)hk * Dh;
    const float *vh = v + (int64_t)hk * Dh;
    const float *rl0 = rel_logits + (t * H + (int64_t)hk * G) * R;
    __syncthreads();
    for (int64_t c0 = s0; c0 <= s1; c0 += ATT_CH) {
        const int n = (int)(s1 - c0 + 1 < ATT_CH ? s1 - c0 + 1 : ATT_CH);
        // scores of rows j = 16 pass + row16
        for (int pass = 0; pass < ATT_CH / 16; pass++) {
            const int j = 16 * pass + row16;
            if (16 * pass >= n) break;
            const int64_t kv = c0 + (j < n ? j : 0);
            const float *kr = kh + kv * kv_dim;
            const float4 ka = d_a < Dh ? *(const float4 *)(kr + d_a) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            const float4 kb = d_b < Dh ? *(const float4 *)(kr + d_b) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            const int64_t dist = q_pos - kv;
            for (int g = 0; g < G; g++) {
                const float *qg = qs + g * ATT_DMAX;
                float s = 0.0f;
                if (d_a < Dh) {
                    s = __builtin_fmaf(qg[d_a], ka.x, s);
                    s = __builtin_fmaf(qg[d_a + 1], ka.y, s);
                    s = __builtin_fmaf(qg[d_a + 2], ka.z, s);
                    s = __builtin_fmaf(qg[d_a + 3], ka.w, s);
                }
                if (d_b < Dh) {
                    s = __builtin_fmaf(qg[d_b], kb.x, s);
                    s = __builtin_fmaf(qg[d_b + 1], kb.y, s);
                    s = __builtin_fmaf(qg[d_b + 2], kb.z, s);
                    s = __builtin_fmaf(qg[d_b + 3], kb.w, s);
                }
                s = att_sum16(s);
                if (l16 == 0 && j < n) {
                    const double bias = dist < R ? (double)rl0[(int64_t)g * R + dist] * (double)tau : 0.0;
                    ps[g * ATT_CH + j] = (float)((double)(s * inv_head_dim) + bias);
                }
            }
        }
        __syncthreads();
        // online softmax, one wave per head
        for (int g = wave; g < G; g += 4) {
            const float sa = lane < n ? ps[g * ATT_CH + lane] : -INFINITY;
            const float sb = lane + 64 < n ? ps[g * ATT_CH + lane + 64] : -INFINITY;
            const float m_old = mrun[g];
            const float m_new = fmaxf(m_old, att_wave_max(fmaxf(sa, sb)));
            const float pa = lane < n ? (float)exp((double)(sa - m_new)) : 0.0f;
            const float pb = lane + 64 < n ? (float)exp((double)(sb - m_new)) : 0.0f;
            ps[g * ATT_CH + lane] = pa;
            ps[g * ATT_CH + lane + 64] = pb;
            double lsum = (double)pa + (double)pb;
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) lsum += __shfl_xor(lsum, o, 64);
            if (lane == 0) {
                const double al = m_old == -INFINITY ? 0.0 : exp((double)(m_old - m_new));
                alpha[g] = al;
                lrun[g] = lrun[g] * al + lsum;
                mrun[g] = m_new;
            }
        }
        __syncthreads();
        // p . v
        for (int i = 0; i < OPT; i++) {
            const int o = tid + 256 * i;
            if (o < n_out) acc[i] *= alpha[o / Dh];
        }
        for (int j = 0; j < n; j++) {
            const float *vr = vh + (c0 + j) * kv_dim;
#pragma unroll
            for (int i = 0; i < ATT_GMAX * ATT_DMAX / 256; i++) {
                const int o = tid + 256 * i;
                if (i < OPT && o < n_out) {
                    const int g = o / Dh, d = o - g * Dh;
                    acc[i] = __builtin_fma((double)ps[g * ATT_CH + j], (double)vr[d], acc[i]);
                }
            }
        }
        __syncthreads();
    }
    const int64_t pbase = ((int64_t)z * H + (int64_t)hk * G) * nsplit + x;
    for (int i = 0; i < OPT; i++) {
        const int o = tid + 256 * i;
        if (o < n_out) {
            const int g = o / Dh, d = o - g * Dh;
            part[(pbase + (int64_t)g * nsplit) * (Dh + 2) + d] = acc[i];
        }
    }
    if (tid < G) {
        part[(pbase + (int64_t)tid * nsplit) * (Dh + 2) + Dh] = (double)mrun[tid];
        part[(pbase + (int64_t)tid * nsplit) * (Dh + 2) + Dh + 1] = lrun[tid];
    }
}

// Fold of token t0 + blockIdx.y, head blockIdx.x: its spans' partials in
// span order, in double, out[t, h, d] = sum_x acc_x[d] e^(m_x - M) /
// sum_x l_x e^(m_x - M) rounded to f32.
extern "C" __global__ __launch_bounds__(128) void sepia_attn_combine(
    const double *__restrict__ part, AttnTok tok, int32_t t0, int32_t H, int32_t Dh, int32_t nsplit, int32_t span,
    float *__restrict__ out) {
    const int z = (int)blockIdx.y, h = (int)blockIdx.x, d = (int)threadIdx.x;
    const int64_t n_kv = (int64_t)tok.hi[z] - tok.lo[z] + 1;
    const int nx = (int)((n_kv + span - 1) / span);
    const double *pb = part + ((int64_t)z * H + h) * nsplit * (Dh + 2);
    double M = -INFINITY;
    for (int x = 0; x < nx; x++) M = fmax(M, pb[(int64_t)x * (Dh + 2) + Dh]);
    double L = 0.0, o = 0.0;
    for (int x = 0; x < nx; x++) {
        const double *px = pb + (int64_t)x * (Dh + 2);
        const double e = exp(px[Dh] - M);
        L = __builtin_fma(px[Dh + 1], e, L);
        if (d < Dh) o = __builtin_fma(px[d], e, o);
    }
    if (d < Dh) out[(((int64_t)t0 + z) * H + h) * Dh + d] = (float)(o / L);
}
