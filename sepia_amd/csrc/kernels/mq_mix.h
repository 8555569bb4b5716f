// mq_mix.h -- gate/up of the MoE decode layer with the expert selection
// hidden behind weight streaming.
//
// mq.h's sepia_mq_gateup gives each slot its own workgroups: the routed ones
// cannot issue a weight DMA until their wave 0 has selected the experts from
// the router's logits (a few microseconds of one wave's dependent work),
// while only the shared-expert workgroups stream. Here every workgroup takes
// a share of both: wave 0 selects (route.h) and raises an LDS flag; waves
// 1.. convert x and stream the workgroup's shared units, then, once the flag
// is up, its routed units. A unit is 16 rows of one slot's gate and the same
// rows of its up. Output: h[slot][inter] f32, and (workgroup 0) the
// selection for the down launch, as sepia_mq_gateup.
#pragma once
#include "mq.h"

// LDS layout and geometry (host mirror in sepia_hip.c):
// [zero][XQ of x][selection: idx[64], w[64], flag][control words][red][rings]
struct MqMixGeo {
    MqGeo gu;                  // P and ring bytes of each streaming wave
    uint32_t o_sel, o_ctl, o_gred, o_rings;
    int32_t nstream;           // streaming waves 1 .. nstream (P C of them; the rest only convert x)
};

// Routed units before workgroup b of G: with T the total bytes (us shared
// units of ws bytes, ur routed ones of wr), workgroup b takes shared units
// [b us / G, (b + 1) us / G) and routed units so that the bytes before it
// are about T b / G. Monotone in b when T / G >= ws ceil(us / G) (the host
// checks), and ur at b = G.
__device__ __forceinline__ int64_t mq_mix_rbefore(int64_t us, int64_t ws, int64_t ur, int64_t wr, int64_t G,
                                                  int64_t b) {
    const int64_t T = us * ws + ur * wr;
    const int64_t f = T * b / G - (b * us / G) * ws;
    const int64_t r = f <= 0 ? 0 : f / wr;
    return r < ur ? r : ur;
}

template <int TS, int TG>
__device__ __forceinline__ void mq_mix_body(const MqProj &gate, const MqProj &up, const MqProj &s_gate,
                                            const MqProj &s_up, const MqRoute &rt, int32_t topk, int32_t n_shared,
                                            int32_t inter, const float *__restrict__ x, float *__restrict__ h,
                                            const MqMixGeo &geo) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int w = mq_wave_id(), lane = (int)(threadIdx.x & 63);
    const int64_t I = inter, H = 256 * gate.n_blocks, G = gridDim.x, b = blockIdx.x;
    const int64_t tiles_i = I >> 4;
    const int64_t us = (int64_t)n_shared * tiles_i, ur = (int64_t)topk * tiles_i;
    const int64_t ws = 32 * (int64_t)(n_shared > 0 ? s_gate.row_bytes : 0), wr = 32 * (int64_t)gate.row_bytes;
    const int64_t s0 = b * us / G, ns = (b + 1) * us / G - s0;
    const int64_t r0 = mq_mix_rbefore(us, ws, ur, wr, G, b), nr = mq_mix_rbefore(us, ws, ur, wr, G, b + 1) - r0;
    int32_t *si = (int32_t *)(smem + geo.o_sel);
    float *sw = (float *)(si + 64);
    int32_t *flag = si + 128;
    uint32_t *ctl = (uint32_t *)(smem + geo.o_ctl);
    float *gred = (float *)(smem + geo.o_gred);
    uint8_t *rings = smem + geo.o_rings;
    const int nconv = (int)blockDim.x - 64;

    // the flag down and the selection in range before anyone looks; the
    // vector's DMAs go out ahead of every weight DMA
    if (threadIdx.x < 129) si[threadIdx.x] = 0;
    if (threadIdx.x == 129) ctl[0] = 0u;
    if (w > 0) mq_xq_dma_by(x, (int)H, smem, MQ_ZERO, 64, nconv);
    __builtin_amdgcn_s_waitcnt(MQ_WC_LGKM0);
    __builtin_amdgcn_s_barrier();
    if (w == 0) {
        // ---- the selection, while the other waves stream
        route_pick_any<false>(rt.logits, rt.bias, rt.n_routed, rt.n_shared, topk, rt.route_scale, rt.global_scale,
                              si, sw);
        if (b == 0 && lane < topk + n_shared) {
            if (lane < topk) rt.idx_out[lane] = si[lane];
            rt.w_out[lane] = sw[lane];
        }
        __hip_atomic_store(flag, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    } else {
        // ---- x into its XQ place, then the shared units, then the routed ones
        auto sitem = [&](int i) {
            const int64_t u = s0 + (i >> 1), e = u / tiles_i;
            MqItem it;
            it.base = ((i & 1) ? s_up.base : s_gate.base) + e * ((i & 1) ? s_up.stride : s_gate.stride);
            it.row0 = (u - e * tiles_i) * 16;
            it.rows = I;
            it.xoff = MQ_ZERO;
            it.red = i;
            return it;
        };
        MqWave<TS, decltype(sitem)> sp(sitem, (int)(2 * ns), (int)(s_gate.n_blocks >> 2), (int)H,
                                       (uint32_t)s_gate.row_bytes, geo.gu, rings, 1, geo.nstream);
        sp.prologue();
        sp.wait_before_prologue();   // this wave's x DMAs (older than its weights)
        mq_xq_in_place_by((int)H, smem, MQ_ZERO, 64, nconv, ctl, nullptr, true);
        mq_waves_wait(ctl, 3u * (uint32_t)(nconv >> 6), lane, nullptr);
        sp.run(smem, gred);
        if (nr > 0) {
            const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
            while (__hip_atomic_load(flag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) == 0) {
                __builtin_amdgcn_s_sleep(1);
                if (__builtin_amdgcn_s_memrealtime() - t0 > MQ_WAIT_TICKS) break;   // never: wave 0 always ends
            }
            auto ritem = [&](int i) {
                const int64_t u = r0 + (i >> 1);
                const int64_t slot = u / tiles_i;
                int64_t e = __builtin_amdgcn_readfirstlane(si[slot]);
                e = e < 0 ? 0 : (e < rt.n_routed ? e : rt.n_routed - 1);
                MqItem it;
                it.base = ((i & 1) ? up.base : gate.base) + e * ((i & 1) ? up.stride : gate.stride);
                it.row0 = (u - slot * tiles_i) * 16;
                it.rows = I;
                it.xoff = MQ_ZERO;
                it.red = (int32_t)(2 * ns) + i;
                return it;
            };
            MqWave<TG, decltype(ritem)> rp(ritem, (int)(2 * nr), (int)(gate.n_blocks >> 2), (int)H,
                                           (uint32_t)gate.row_bytes, geo.gu, rings, 1, geo.nstream);
            rp.prologue();
            rp.run(smem, gred);
        }
    }
    __syncthreads();
    // h = silu(gate) * up for every unit of the workgroup
    const int P = geo.gu.P;
    for (int64_t i = threadIdx.x; i < (ns + nr) * 16; i += blockDim.x) {
        const int64_t m = i >> 4, t = i & 15;
        const bool sh = m < ns;
        const int64_t u = sh ? s0 + m : r0 + (m - ns);
        const int64_t slot = sh ? topk + u / tiles_i : u / tiles_i;
        const int64_t row = (u % tiles_i) * 16 + t;
        h[slot * I + row] = silu_f32(mq_red_sum(gred, (int)(2 * m), P, (int)t)) *
                            mq_red_sum(gred, (int)(2 * m + 1), P, (int)t);
    }
}

__device__ __forceinline__ void mq_mix(const MqProj &gate, const MqProj &up, const MqProj &s_gate, const MqProj &s_up,
                                       const MqRoute &rt, int32_t topk, int32_t n_shared, int32_t inter,
                                       const float *__restrict__ x, float *__restrict__ h, const MqMixGeo &geo) {
    const int ts = n_shared > 0 ? s_gate.type : gate.type, tg = gate.type;
    if (false) {
    }
#define MQ_MIX_CASE(A, B) \
    else if (ts == A && tg == B) mq_mix_body<A, B>(gate, up, s_gate, s_up, rt, topk, n_shared, inter, x, h, geo);
    MQ_MIX_CASE(ST_Q2_K, ST_Q2_K) MQ_MIX_CASE(ST_Q2_K, ST_Q3_K) MQ_MIX_CASE(ST_Q2_K, ST_Q4_K)
    MQ_MIX_CASE(ST_Q3_K, ST_Q2_K) MQ_MIX_CASE(ST_Q3_K, ST_Q3_K) MQ_MIX_CASE(ST_Q3_K, ST_Q4_K)
    MQ_MIX_CASE(ST_Q4_K, ST_Q2_K) MQ_MIX_CASE(ST_Q4_K, ST_Q3_K) MQ_MIX_CASE(ST_Q4_K, ST_Q4_K)
#undef MQ_MIX_CASE
}

#define SEPIA_MQ_MIX()                                                                                    \
    extern "C" __global__ __launch_bounds__(1024) void sepia_mq_gateup_mix(                               \
        MqProj gate, MqProj up, MqProj s_gate, MqProj s_up, MqRoute rt, int32_t topk, int32_t n_shared,    \
        int32_t inter, const float *__restrict__ x, float *__restrict__ h, MqMixGeo geo) {                \
        mq_mix(gate, up, s_gate, s_up, rt, topk, n_shared, inter, x, h, geo);                             \
    }
