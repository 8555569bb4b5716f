// sepia_kernels.hip -- every gfx950 kernel of the library, compiled into one
// code object (sepia_kernels.hsaco) that sepia_hip.c loads with hipModuleLoad.
// Kernel names are extern "C" so the host finds them with hipModuleGetFunction.
#include "common.h"
#include "decode.h"
#include "matvec.h"

// The device error word's address and the spin-wait bound (common.h): the
// host writes both right after loading this code object.
extern "C" __constant__ uint32_t *sepia_err_word = nullptr;
extern "C" __constant__ uint64_t sepia_wait_ticks = 200000000ull;

// ------------------------------------------------------------------------
// Standalone dequantization (reference metal/matvec_q.metal:578-660): one
// thread per 32-weight part, writing the part's floats. Same decoders as the
// matvec, so this is the bitwise gate for the matvec's unpack.
template <int T>
__device__ void dequant_parts(const uint8_t *__restrict__ raw, float *__restrict__ out, int64_t n_parts) {
    const int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (u >= n_parts) return;
    const int64_t b = u / Fmt<T>::parts;
    const int p = (int)(u % Fmt<T>::parts);
    float w[32];
    decode_part<T>(raw + b * Fmt<T>::bytes, p, w);
    float *o = out + b * Fmt<T>::elems + 32 * p;
#pragma unroll
    for (int i = 0; i < 32; i++) o[i] = w[i];
}

#define SEPIA_DEQUANT_KERNEL(name, T)                                                              \
    extern "C" __global__ __launch_bounds__(256) void sepia_dequant_rows_##name(                 \
        const uint8_t *__restrict__ raw, float *__restrict__ out, int64_t n_parts) {             \
        dequant_parts<T>(raw, out, n_parts);                                                     \
    }
SEPIA_DEQUANT_KERNEL(q8_0, ST_Q8_0)
SEPIA_DEQUANT_KERNEL(q2_k, ST_Q2_K)
SEPIA_DEQUANT_KERNEL(q3_k, ST_Q3_K)
SEPIA_DEQUANT_KERNEL(q4_k, ST_Q4_K)
SEPIA_DEQUANT_KERNEL(q5_k, ST_Q5_K)
SEPIA_DEQUANT_KERNEL(q6_k, ST_Q6_K)
SEPIA_DEQUANT_KERNEL(iq2_xxs, ST_IQ2_XXS)
SEPIA_DEQUANT_KERNEL(iq2_xs, ST_IQ2_XS)
SEPIA_DEQUANT_KERNEL(iq3_xxs, ST_IQ3_XXS)
SEPIA_DEQUANT_KERNEL(iq4_xs, ST_IQ4_XS)

// F16 rows: the integer conversion keeps NaN payloads (src/quants.c:58-77).
extern "C" __global__ __launch_bounds__(256) void sepia_dequant_rows_f16(
    const uint8_t *__restrict__ raw, float *__restrict__ out, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = f16_bits_to_f32_exact(ld_u16(raw + 2 * i));
}

// ------------------------------------------------------------------------
// Generic dequant-fused matvec: one wave per output row (4 rows per
// 256-thread workgroup). Lanes stride over the row's 32-weight parts, decode
// each with the bit-exact decoder and accumulate part . x with FMAs; a
// butterfly shuffle sums the 64 lane partials.
#define SEPIA_MATVEC_GENERIC(name, T)                                                              \
    extern "C" __global__ __launch_bounds__(256) void sepia_matvec_generic_##name(               \
        const uint8_t *__restrict__ w, uint64_t row_bytes, int64_t n_blocks,                     \
        const float *__restrict__ x, float *__restrict__ y, int64_t out_dim) {                   \
        const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);                        \
        if (row >= out_dim) return;                                                              \
        const float acc = row_dot_generic<T>(w + row * row_bytes, n_blocks, x);                  \
        if ((threadIdx.x & 63) == 0) y[row] = acc;                                               \
    }
SEPIA_MATVEC_GENERIC(q8_0, ST_Q8_0)
SEPIA_MATVEC_GENERIC(q2_k, ST_Q2_K)
SEPIA_MATVEC_GENERIC(q3_k, ST_Q3_K)
SEPIA_MATVEC_GENERIC(q4_k, ST_Q4_K)
SEPIA_MATVEC_GENERIC(q5_k, ST_Q5_K)
SEPIA_MATVEC_GENERIC(q6_k, ST_Q6_K)
SEPIA_MATVEC_GENERIC(iq2_xxs, ST_IQ2_XXS)
SEPIA_MATVEC_GENERIC(iq2_xs, ST_IQ2_XS)
SEPIA_MATVEC_GENERIC(iq3_xxs, ST_IQ3_XXS)
SEPIA_MATVEC_GENERIC(iq4_xs, ST_IQ4_XS)

// ------------------------------------------------------------------------
// f32 row ops (reference metal/ops.metal). One wave per row for the
// reductions; elementwise ops one thread per element.

// y[r] = w[r,:] . x with row stride `ld` floats (router logits, f32 matvec).
extern "C" __global__ __launch_bounds__(256) void sepia_matvec_f32(
    const float *__restrict__ w, int64_t ld, const float *__restrict__ x, float *__restrict__ y,
    int64_t out_dim, int64_t in_dim) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= out_dim) return;
    const float acc = row_dot_f32(w + row * ld, x, in_dim);
    if ((threadIdx.x & 63) == 0) y[row] = acc;
}

extern "C" __global__ __launch_bounds__(256) void sepia_silu_mul_f32(
    const float *__restrict__ g, const float *__restrict__ u, float *__restrict__ z, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) z[i] = silu_f32(g[i]) * u[i];
}

extern "C" __global__ __launch_bounds__(256) void sepia_add_f32(
    const float *a, const float *b, float *out, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = a[i] + b[i];
}

extern "C" __global__ __launch_bounds__(256) void sepia_scale_f32(
    const float *x, float *y, int64_t n, float s) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = x[i] * s;
}

extern "C" __global__ __launch_bounds__(256) void sepia_copy_f32(
    const float *in, float *out, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = in[i];
}

extern "C" __global__ __launch_bounds__(256) void sepia_fill_u32(uint32_t *p, int64_t n, uint32_t v) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

// HBM read ceiling of one launch: every workgroup streams a contiguous
// chunk of n16 16-byte words with four loads in flight per lane and nothing
// else (a measurement reference for the weight-streaming kernels). The
// sink is written only if the XOR of the chunk equals a fixed word, which
// keeps the loads.
extern "C" __global__ __launch_bounds__(256) void sepia_read_probe(const uint4 *__restrict__ p, int64_t n16,
                                                                   uint32_t *__restrict__ sink) {
    const int64_t per = (n16 + gridDim.x - 1) / gridDim.x;
    const int64_t b = (int64_t)blockIdx.x * per, e = b + per < n16 ? b + per : n16;
    uint32_t acc = 0;
    for (int64_t i = b + threadIdx.x; i < e; i += 4 * 256) {
        uint4 v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int64_t j = i + (int64_t)u * 256;
            v[u] = j < e ? p[j] : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < 4; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (acc == 0x9E3779B9u) sink[blockIdx.x] = acc;
}

extern "C" __global__ __launch_bounds__(256) void sepia_touch_f32(float *x, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] += 0.0f;
}

// Workgroup-wide sum for 256 threads; every thread receives the total.
__device__ __forceinline__ float block_sum_256(float v, float *lds4) {
    v = wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) lds4[threadIdx.x >> 6] = v;
    __syncthreads();
    return (lds4[0] + lds4[1]) + (lds4[2] + lds4[3]);
}

__device__ __forceinline__ float block_max_256(float v, float *lds4) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, SEPIA_WAVE));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) lds4[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(lds4[0], lds4[1]), fmaxf(lds4[2], lds4[3]));
}

// y[r,i] = w[i] * (x[r,i] * (1 / sqrt(mean(x^2) + eps))): one workgroup per row
// (reference src/sepia.c:719-729 order: x * inv first, then * w).
extern "C" __global__ __launch_bounds__(256) void sepia_rmsnorm_f32(
    const float *w, const float *x, float *y, int64_t n, float eps) {
    __shared__ float red[4];
    const float *xr = x + (int64_t)blockIdx.x * n;
    float *yr = y + (int64_t)blockIdx.x * n;
    float s = 0.0f;
    for (int64_t i = threadIdx.x; i < n; i += 256) s = __builtin_fmaf(xr[i], xr[i], s);
    s = block_sum_256(s, red);
    const float inv = 1.0f / sqrtf(s / (float)n + eps);
    for (int64_t i = threadIdx.x; i < n; i += 256) yr[i] = w[i] * (xr[i] * inv);
}

// Stable softmax per row; y may alias x.
extern "C" __global__ __launch_bounds__(256) void sepia_softmax_f32(
    const float *x, float *y, int64_t n) {
    __shared__ float red[4];
    const float *xr = x + (int64_t)blockIdx.x * n;
    float *yr = y + (int64_t)blockIdx.x * n;
    float m = -INFINITY;
    for (int64_t i = threadIdx.x; i < n; i += 256) m = fmaxf(m, xr[i]);
    m = block_max_256(m, red);
    float s = 0.0f;
    for (int64_t i = threadIdx.x; i < n; i += 256) {
        const float e = expf(xr[i] - m);
        yr[i] = e;
        s += e;
    }
    s = block_sum_256(s, red);
    const float inv = 1.0f / s;
    for (int64_t i = threadIdx.x; i < n; i += 256) yr[i] *= inv;
}

// K-tap depthwise causal conv + residual over window = [hist(K-1) ; in(T)]
// (reference src/sepia.c:801-816): one thread per (t, c).
extern "C" __global__ __launch_bounds__(256) void sepia_sconv_f32(
    const float *w, const float *hist, const float *in, float *out, int32_t C, int32_t K, int32_t T) {
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= (int64_t)C * T) return;
    const int32_t c = (int32_t)(g % C), t = (int32_t)(g / C), km1 = K - 1;
    float acc = 0.0f;
    for (int32_t k = 0; k < K; k++) {
        const int32_t j = t + k;
        const float v = (j < km1) ? hist[(int64_t)j * C + c] : in[(int64_t)(j - km1) * C + c];
        acc = __builtin_fmaf(w[(int64_t)c * K + k], v, acc);
    }
    out[(int64_t)t * C + c] = in[(int64_t)t * C + c] + acc;
}

// New history = last K-1 rows of [hist ; in] (reference src/sepia.c:817),
// one thread per channel; every old value it needs is read before any write.
extern "C" __global__ __launch_bounds__(256) void sepia_sconv_hist_roll_f32(
    float *hist, const float *in, int32_t C, int32_t km1, int32_t T) {
    const int32_t c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= C || km1 <= 0 || km1 > 15) return;
    float keep[15];
    const int32_t nk = (T >= km1) ? 0 : km1 - T;
    for (int32_t j = 0; j < nk; j++) keep[j] = hist[(int64_t)(T + j) * C + c];
    for (int32_t j = 0; j < km1; j++) {
        const float v = (T >= km1) ? in[(int64_t)(T - km1 + j) * C + c]
                                   : (j < nk ? keep[j] : in[(int64_t)(j - nk) * C + c]);
        hist[(int64_t)j * C + c] = v;
    }
}

// ------------------------------------------------------------------------
// Tile kernels with integer dot products (mv.h): the matvec per format, and
// the expert-FFN launches per (routed, shared) format pair; gate/up comes in
// two flavours, x as f32 (converted per workgroup) or as digit planes
// written by the router launch (_xp).
#include "mv.h"
SEPIA_MV_KERNEL(q2_k, ST_Q2_K)
SEPIA_MV_KERNEL(q3_k, ST_Q3_K)
SEPIA_MV_KERNEL(q4_k, ST_Q4_K)

#define SEPIA_FFN_PAIR(a, b, TA, TB)                                                              \
    SEPIA_FFN_GATEUP(a##b, TA, TB, false)                                                         \
    SEPIA_FFN_GATEUP(a##b##_xp, TA, TB, true)                                                     \
    SEPIA_FFN_DOWN(a##b, TA, TB)
SEPIA_FFN_PAIR(2, 2, ST_Q2_K, ST_Q2_K)
SEPIA_FFN_PAIR(2, 3, ST_Q2_K, ST_Q3_K)
SEPIA_FFN_PAIR(2, 4, ST_Q2_K, ST_Q4_K)
SEPIA_FFN_PAIR(3, 2, ST_Q3_K, ST_Q2_K)
SEPIA_FFN_PAIR(3, 3, ST_Q3_K, ST_Q3_K)
SEPIA_FFN_PAIR(3, 4, ST_Q3_K, ST_Q4_K)
SEPIA_FFN_PAIR(4, 2, ST_Q4_K, ST_Q2_K)
SEPIA_FFN_PAIR(4, 3, ST_Q4_K, ST_Q3_K)
SEPIA_FFN_PAIR(4, 4, ST_Q4_K, ST_Q4_K)

#include "mq.h"
#include "moe.h"
#include "prefill.h"
#include "prefill_q.h"
#include "prefill_h.h"
#include "synth.h"
#include "attn.h"

// ------------------------------------------------------------------------
// Matrix-core quantized matvecs and expert FFN (mq.h).
SEPIA_MQ_MV(q2_k, ST_Q2_K)
SEPIA_MQ_MV(q3_k, ST_Q3_K)
SEPIA_MQ_MV(q4_k, ST_Q4_K)
SEPIA_MQ_MV(iq2_xs, ST_IQ2_XS)
SEPIA_MQ_MV(iq3_xxs, ST_IQ3_XXS)
SEPIA_MQ_MV(q5_k, ST_Q5_K)
SEPIA_MQ_MV(q6_k, ST_Q6_K)
SEPIA_MQ_MV(iq4_xs, ST_IQ4_XS)
SEPIA_MQ_MV(q8_0, ST_Q8_0)
SEPIA_MQ_GATEUP()
SEPIA_MQ_DOWN()

// ------------------------------------------------------------------------
// HBM read ceiling through the decode kernels' own staging path: every wave
// streams its steps of KB KB (KB wave-wide 16-byte LDS DMAs) through a
// private ring of S stages, as MqWave does -- wait for the oldest stage,
// read it back (one 16-byte word per lane per KB), refill it -- with no
// decode. Workgroup b reads the contiguous chunk b of the n16 16-byte words;
// its waves take its steps round robin. Lanes past the chunk's end read its
// last word (every DMA is whole and in bounds). LDS: nw * S * KB KB.
template <int KB, int S>
__device__ __forceinline__ void read_probe_dma(const uint4 *__restrict__ p, int64_t n16, uint32_t *__restrict__ sink) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int nw = (int)(blockDim.x >> 6), w = mq_wave_id(), lane = (int)(threadIdx.x & 63);
    const int64_t per = (n16 + gridDim.x - 1) / gridDim.x;
    const int64_t b = (int64_t)blockIdx.x * per, e = b + per < n16 ? b + per : n16;
    if (b >= e) return;
    const int64_t steps = (e - b + 64 * KB - 1) / (64 * KB);
    const int Tn = steps > w ? (int)((steps - w + nw - 1) / nw) : 0;
    uint8_t *ring = smem + (size_t)w * S * KB * 1024;
    const uint32_t rl = mq_lds_addr(ring);
    const uint8_t *pb = (const uint8_t *)(p + b);
    auto issue = [&](int t) {   // step t of this wave into ring slot t % S (32-bit offsets within the chunk)
        const int64_t s = w + (int64_t)t * nw;
        const uint32_t slot = (uint32_t)(t % S) * (uint32_t)(KB * 1024);
#pragma unroll
        for (int d = 0; d < KB; d++) {
            int64_t j = s * 64 * KB + (int64_t)d * 64 + lane;
            j = j < e - b ? j : e - b - 1;
            mq_dma16(pb, (uint32_t)(16 * j), rl + slot + 1024u * (uint32_t)d);
        }
    };
    for (int t = 0; t < S && t < Tn; t++) issue(t);
    uint32_t acc = 0;
    for (int t = 0; t < Tn; t++) {
        const int after = (Tn - 1 - t) < (S - 1) ? (Tn - 1 - t) : (S - 1);
        mq_wait_stages<KB>(after);
        const uint8_t *src = ring + (size_t)(t % S) * (KB * 1024) + 16 * lane;
        uint4 v[KB];
#pragma unroll
        for (int d = 0; d < KB; d++) v[d] = *(const uint4 *)(src + 1024 * d);
        __builtin_amdgcn_s_waitcnt(MQ_WC_LGKM0);
        if (t + S < Tn) issue(t + S);
#pragma unroll
        for (int d = 0; d < KB; d++) acc ^= v[d].x ^ v[d].y ^ v[d].z ^ v[d].w;
    }
    if (acc == 0x9E3779B9u) sink[blockIdx.x] = acc;
}

extern "C" __global__ __launch_bounds__(1024) void sepia_read_probe_dma(const uint4 *__restrict__ p, int64_t n16,
                                                                       uint32_t *__restrict__ sink, int32_t kb,
                                                                       int32_t s) {
    switch (kb * 8 + s) {
    case 7 * 8 + 1: read_probe_dma<7, 1>(p, n16, sink); break;
    case 7 * 8 + 2: read_probe_dma<7, 2>(p, n16, sink); break;
    case 4 * 8 + 1: read_probe_dma<4, 1>(p, n16, sink); break;
    case 4 * 8 + 2: read_probe_dma<4, 2>(p, n16, sink); break;
    case 4 * 8 + 4: read_probe_dma<4, 4>(p, n16, sink); break;
    case 2 * 8 + 4: read_probe_dma<2, 4>(p, n16, sink); break;
    case 1 * 8 + 4: read_probe_dma<1, 4>(p, n16, sink); break;
    default: break;
    }
}
