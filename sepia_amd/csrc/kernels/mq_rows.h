// mq_rows.h -- down of the MoE decode layer with every slot of a row group
// in one workgroup.
//
// mq.h's sepia_mq_down gives each slot its own workgroups, so the slots'
// partial rows meet through agent-scope stores, per-row-group arrival
// counters and a last-arriver sum: several memory round trips at the end of
// every workgroup. Here workgroup b owns row groups [b T / G, (b + 1) T / G)
// (T = hidden / 16) of every slot: the XQ form of every slot's h sits in its
// LDS (DMA'd in place and converted there), waves 0 .. nr - 1 stream the
// routed slots' rows (format TD), waves nr .. nr + ns - 1 the shared slots'
// (format TSD), both at once, and the workgroup sums the slots in slot order
// from LDS: y[r] = sum_s w_s (down_s[r] . h_s), w the routed weights then the
// shared gammas (src/sepia.c:1425, :1441, :3953-3957), deterministic.
#pragma once
#include "mq.h"

// LDS: [zero][XQ of h_0][XQ of h_1]...[routed experts: 64 i32][red][rings]
// (host mirror in sepia_hip.c)
struct MqRowsGeo {
    MqGeo gr, gs;              // routed / shared waves: P and ring bytes per wave
    int32_t nwr, nws;          // routed waves 0 .. nwr - 1, shared waves nwr .. nwr + nws - 1
    uint32_t o_red, o_rings_s; // red area; the shared waves' rings (the routed ones at gr.orings)
};

template <int TD, int TSD>
__device__ __forceinline__ void mq_rows_body(const MqProj &down, const MqProj &s_down, const int32_t *__restrict__ sel_idx,
                                             const float *__restrict__ sel_w, int32_t topk, int32_t n_shared,
                                             int32_t inter, int64_t hidden, const float *__restrict__ h,
                                             float *__restrict__ y, const MqRowsGeo &geo) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int n_slots = topk + n_shared;
    const int64_t T = (hidden + 15) >> 4, G = gridDim.x, b = blockIdx.x;
    const int64_t rg0 = b * T / G, nrg = (b + 1) * T / G - rg0;
    const uint32_t xqb = 4u * (uint32_t)inter;   // XQ bytes of one h vector (= its f32 bytes)
    const int w = mq_wave_id();
    // routed items' partial rows, then the shared items' (each block with its own P)
    float *red = (float *)(smem + geo.o_red);
    float *red_s = red + (int64_t)topk * nrg * geo.gr.P * 16;

    // the routed experts into LDS (the weight issue path reads only LDS);
    // every slot's h into its XQ place (1 KB a wave instruction), ahead of
    // every weight DMA (a bare barrier), then the weights
    int32_t *sel = (int32_t *)(smem + geo.o_red) - 64;
    if (threadIdx.x < (unsigned)topk) sel[threadIdx.x] = sel_idx[threadIdx.x];
    {
        const int nw = (int)(blockDim.x >> 6), nck = inter >> 8;
        const uint32_t lane = threadIdx.x & 63;
        for (int c = w; c < n_slots * nck; c += nw) {
            const int s = c / nck, k = c - s * nck;
            mq_dma16((const uint8_t *)(h + (int64_t)s * inter), (uint32_t)k * 1024u + 16u * lane,
                     mq_lds_addr(smem + MQ_ZERO + (uint32_t)s * xqb + (uint32_t)k * 1024u));
        }
    }
    __builtin_amdgcn_s_waitcnt(MQ_WC_LGKM0);
    __builtin_amdgcn_s_barrier();

    auto ritem = [&](int i) {
        const int s = i / (int)nrg;
        const int64_t e = __builtin_amdgcn_readfirstlane(sel[s]);
        MqItem it;
        it.base = down.base + e * down.stride;
        it.row0 = (rg0 + (i - s * nrg)) * 16;
        it.rows = hidden;
        it.xoff = MQ_ZERO + (uint32_t)s * xqb;
        it.red = i;
        return it;
    };
    auto sitem = [&](int i) {
        const int s = i / (int)nrg;
        MqItem it;
        it.base = s_down.base + (int64_t)s * s_down.stride;
        it.row0 = (rg0 + (i - s * nrg)) * 16;
        it.rows = hidden;
        it.xoff = MQ_ZERO + (uint32_t)(topk + s) * xqb;
        it.red = i;
        return it;
    };
    MqWave<TD, decltype(ritem)> rw(ritem, (int)(topk * nrg), (int)(down.n_blocks >> 2), inter,
                                   (uint32_t)down.row_bytes, geo.gr, smem + geo.gr.orings, 0, geo.nwr);
    MqWave<TSD, decltype(sitem)> swv(sitem, (int)(n_shared * nrg), (int)(s_down.n_blocks >> 2), inter,
                                     (uint32_t)s_down.row_bytes, geo.gs, smem + geo.o_rings_s, geo.nwr, geo.nws);
    const bool is_r = w < geo.nwr, is_s = w >= geo.nwr && w < geo.nwr + geo.nws;
    if (is_r) {
        rw.prologue();
        rw.wait_before_prologue();
    } else if (is_s) {
        swv.prologue();
        swv.wait_before_prologue();
    } else {
        __builtin_amdgcn_s_waitcnt(mq_wc_vm(0));
    }
    // every h has landed: in-place conversion, every float read before any
    // byte is written (up to four segments a thread)
    __syncthreads();
    {
        const int segs = inter >> 4, tot = n_slots * segs, nt = (int)blockDim.x;
        float a[4][16];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int g = (int)threadIdx.x + k * nt;
            if (g < tot) {
                const int s = g / segs, sg = g - s * segs;
                const float4 *x4 = (const float4 *)(smem + MQ_ZERO + (uint32_t)s * xqb) + 4 * sg;
                const float4 v0 = x4[0], v1 = x4[1], v2 = x4[2], v3 = x4[3];
                const float t[16] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w,
                                     v2.x, v2.y, v2.z, v2.w, v3.x, v3.y, v3.z, v3.w};
#pragma unroll
                for (int i = 0; i < 16; i++) a[k][i] = t[i];
            }
        }
        if (threadIdx.x < MQ_ZERO / 16) ((uint4 *)(smem))[threadIdx.x] = make_uint4(0, 0, 0, 0);
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int g = (int)threadIdx.x + k * nt;
            if (g < tot) {
                const int s = g / segs, sg = g - s * segs;
                xq_store(xq_segment(a[k]), smem + MQ_ZERO + (uint32_t)s * xqb, inter, sg);
            }
        }
    }
    __syncthreads();
    if (is_r) rw.run(smem, red);
    else if (is_s) swv.run(smem, red_s);
    __syncthreads();
    // y: the slots in slot order
    for (int64_t i = threadIdx.x; i < nrg * 16; i += blockDim.x) {
        const int64_t g = i >> 4, t = i & 15, r = (rg0 + g) * 16 + t;
        if (r >= hidden) continue;
        float acc = 0.0f;
        for (int s = 0; s < n_slots; s++) {
            const float v = s < topk ? mq_red_sum(red, (int)(s * nrg + g), geo.gr.P, (int)t)
                                     : mq_red_sum(red_s, (int)((s - topk) * nrg + g), geo.gs.P, (int)t);
            acc = __builtin_fmaf(sel_w[s], v, acc);
        }
        y[r] = acc;
    }
}

__device__ __forceinline__ void mq_rows(const MqProj &down, const MqProj &s_down, const int32_t *__restrict__ sel_idx,
                                        const float *__restrict__ sel_w, int32_t topk, int32_t n_shared, int32_t inter,
                                        int64_t hidden, const float *__restrict__ h, float *__restrict__ y,
                                        const MqRowsGeo &geo) {
    const int td = down.type, ts = n_shared > 0 ? s_down.type : down.type;
    if (false) {
    }
#define MQ_ROWS_CASE(A, B) \
    else if (td == A && ts == B) mq_rows_body<A, B>(down, s_down, sel_idx, sel_w, topk, n_shared, inter, hidden, h, y, geo);
    MQ_ROWS_CASE(ST_Q2_K, ST_Q2_K) MQ_ROWS_CASE(ST_Q2_K, ST_Q3_K) MQ_ROWS_CASE(ST_Q2_K, ST_Q4_K)
    MQ_ROWS_CASE(ST_Q3_K, ST_Q2_K) MQ_ROWS_CASE(ST_Q3_K, ST_Q3_K) MQ_ROWS_CASE(ST_Q3_K, ST_Q4_K)
    MQ_ROWS_CASE(ST_Q4_K, ST_Q2_K) MQ_ROWS_CASE(ST_Q4_K, ST_Q3_K) MQ_ROWS_CASE(ST_Q4_K, ST_Q4_K)
#undef MQ_ROWS_CASE
}

#define SEPIA_MQ_ROWS()                                                                                   \
    extern "C" __global__ __launch_bounds__(1024) void sepia_mq_down_rows(                                \
        MqProj down, MqProj s_down, const int32_t *__restrict__ sel_idx, const float *__restrict__ sel_w, \
        int32_t topk, int32_t n_shared, int32_t inter, int64_t hidden, const float *__restrict__ h,       \
        float *__restrict__ y, MqRowsGeo geo) {                                                           \
        mq_rows(down, s_down, sel_idx, sel_w, topk, n_shared, inter, hidden, h, y, geo);                  \
    }
