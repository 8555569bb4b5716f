// mq_flow.h -- the SwiGLU FFN of one expert (gate/up, h = silu(g) * u, down)
// in ONE launch, with the down weights streaming from the first instant.
//
// Two launches (mq.h's sepia_mq_gateup then sepia_mq_down) leave the down
// weights idle until the gate/up launch has ended, and pay a kernel
// boundary between them. Here each workgroup (one per CU) splits its waves
// into two roles that never wait for one another at a workgroup barrier
// after the start:
//   gate/up waves  stream the workgroup's units (16 rows of gate and the same
//                  16 rows of up); the last of them to finish forms h for its
//                  units, publishes h's XQ segments (agent-scope stores),
//                  waits for them to complete and adds its unit count to a
//                  global counter;
//   down waves     issue their down weights once x has landed, then wait
//                  for h (one poller per workgroup, bounded in time), fetch
//                  XQ(h) into LDS and run; the last of them to finish sums
//                  the partial rows into y.
// Workgroups without gate/up units give all their waves to down and take
// more down rows, so that every workgroup streams about the same bytes.
//
// Progress does not depend on residency: gate/up waves wait for nothing, so
// every unit of h is published once its workgroup runs. The host still
// launches only when the occupancy query admits the whole grid at once (one
// workgroup per CU), so that no workgroup's down waves hold a CU that a
// later workgroup's gate/up waves need; every wait is bounded anyway (a
// time-out raises the error flag the host reads at batch end, and the
// kernel still ends).
//
// Signals: hcnt counts published units; the wave that adds the last one
// puts it back to zero and raises the flag of every workgroup with down
// rows, each flag in its own 128-byte line, so that no address is polled by
// more than one workgroup (256 pollers on one counter serialize at the
// memory side and delay the very adds they wait for). Each poller lowers
// its own flag once it has seen it, so all are down between launches.
// After a time-out the host zeroes them.
#pragma once
#include "mq_fused.h"

// Geometry of a flow launch (host mirror in sepia_hip.c). Workgroup b of G
// owns gate/up units [b U / G, (b + 1) U / G) (U = inter / 16) and down row
// groups [d0(b), d0(b) + nd(b)): nd = dl for workgroups with units, dh for
// the others, one more for the first drem workgroups.
struct MqFlowGeo {
    MqGeo gu;                   // gate/up waves 0 .. ngu - 1: P and ring bytes per wave
    MqGeo d1;                   // down waves ngu .. ngu + nd1 - 1 of a workgroup with units
    MqGeo d0;                   // down waves 0 .. nd0 - 1 of a workgroup without
    int32_t ngu, nd1, nd0;
    int32_t dl, dh, drem;
    int32_t free_delay;         // s_memrealtime ticks a workgroup without units waits before its down weights
    uint32_t o_xqh, o_gred, o_dred, o_ctl, o_rings;   // LDS offsets (XQ(x) at MQ_ZERO)
};

struct MqFlowIo {
    const float *x;
    float *y;
    int64_t inter, hidden;
    uint8_t *xq_h;              // XQ of h, agent scope
    uint32_t *hcnt, *flags, *err;   // flags: workgroup b's at flags[b * MQ_FL_FSTRIDE]
};
#define MQ_FL_FSTRIDE 32

// Down row groups of workgroup b: count and first (see MqFlowGeo).
__device__ __forceinline__ int mq_flow_nd(const MqFlowGeo &geo, int64_t U, int64_t G, int64_t b) {
    const bool has_u = (b + 1) * U / G > b * U / G;
    return (has_u ? geo.dl : geo.dh) + (b < geo.drem ? 1 : 0);
}

// LDS control words at o_ctl: gate/up waves done, down waves done, XQ(h)
// ready (1) or abandoned (2), arrivals of the waves converting x.
#define MQ_FL_GDONE 0
#define MQ_FL_DDONE 1
#define MQ_FL_HREADY 2
#define MQ_FL_XSYNC 3

// Thread 0 of the poller: wait until the workgroup's flag is up, then lower
// it. Returns 0 after a time-out (error flag raised).
__device__ __forceinline__ bool mq_flow_poll(uint32_t *flag, uint32_t *err) {
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    while (__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u) {
        __builtin_amdgcn_s_sleep(1);
        if (__builtin_amdgcn_s_memrealtime() - t0 > MQ_WAIT_TICKS) {
            __hip_atomic_store(err, 3u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return false;
        }
    }
    __hip_atomic_store(flag, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
}

// One wave-wide DMA as mq_dma16, with agent-scope coherence (sc1, as an
// agent-scope atomic load): reads data other CUs published this launch.
__device__ __forceinline__ void mq_dma16_agent(const uint8_t *base, uint32_t voff, uint32_t lds) {
    const uint64_t b = (uint64_t)(uintptr_t)base;
    const uint64_t bs = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32)) << 32) |
                        (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 sc1" : : "v"(voff), "s"((const uint8_t *)(uintptr_t)bs), "{m0}"(lds) : "memory");
}

// One arrival of the calling wave at an LDS counter (lane 0 adds; release
// of the wave's LDS writes, acquire of the earlier arrivals' ones); returns
// the count before it, the same in every lane.
__device__ __forceinline__ int mq_flow_count(uint32_t *c, int lane) {
    uint32_t prev = 0;
    if (lane == 0) prev = __hip_atomic_fetch_add(c, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
    return __builtin_amdgcn_readfirstlane((int)prev);
}

template <int TG, int TD>
__device__ __forceinline__ void mq_flow_body(const MqProj &gate, const MqProj &up, const MqProj &down, int64_t e,
                                             const MqFlowIo &io, const MqFlowGeo &geo) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int64_t H = io.hidden, I = io.inter;
    const int64_t U = I >> 4, G = gridDim.x, b = blockIdx.x;
    const int w = mq_wave_id();
    const int lane = (int)(threadIdx.x & 63);
    uint32_t *ctl = (uint32_t *)(smem + geo.o_ctl);
    float *gred = (float *)(smem + geo.o_gred), *dred = (float *)(smem + geo.o_dred);
    uint8_t *rings = smem + geo.o_rings;

    // this workgroup's units and down row groups
    const int64_t u0 = b * U / G, u1 = (b + 1) * U / G;
    const int nu = (int)(u1 - u0);
    const int64_t nub = U >= G ? b : u0;   // workgroups before b with units
    const int64_t dstart = nub * geo.dl + (b - nub) * geo.dh + (b < geo.drem ? b : geo.drem);
    const int nd = mq_flow_nd(geo, U, G, b);
    const int ngu = nu > 0 ? geo.ngu : 0;
    const int ndw = nd > 0 ? (nu > 0 ? geo.nd1 : geo.nd0) : 0;
    const MqGeo &dg = nu > 0 ? geo.d1 : geo.d0;

    const uint8_t *wg = gate.base + e * gate.stride, *wu = up.base + e * up.stride, *wd = down.base + e * down.stride;
    auto gitem = [&](int i) {
        MqItem it;
        it.base = (i & 1) ? wu : wg;
        it.row0 = (u0 + (i >> 1)) * 16;
        it.rows = I;
        it.xoff = MQ_ZERO;
        it.red = i;
        return it;
    };
    auto ditem = [&](int i) {
        MqItem it;
        it.base = wd;
        it.row0 = (dstart + i) * 16;
        it.rows = H;
        it.xoff = geo.o_xqh;
        it.red = i;
        return it;
    };
    MqWave<TG, decltype(gitem)> gw(gitem, 2 * nu, (int)(gate.n_blocks >> 2), (int)H, (uint32_t)gate.row_bytes,
                                   geo.gu, rings, 0, ngu);
    MqWave<TD, decltype(ditem)> dw(ditem, nd, (int)(down.n_blocks >> 2), (int)I, (uint32_t)down.row_bytes, dg,
                                   rings + (size_t)ngu * geo.gu.ring, ngu, ndw);
    const bool is_g = w < ngu, is_d = w >= ngu && w < ngu + ndw;

    // ---- start: x by LDS DMA ahead of the gate/up weights; the down
    // weights, needed only once h is complete, queue up after x has landed
    if (threadIdx.x < 8) ctl[threadIdx.x] = 0u;
    // The waves past the gate/up ones DMA x and turn it into XQ on their own
    // (an LDS counter orders them); the gate/up waves issue their weights
    // right after the x DMAs (one bare barrier), decode their first step as
    // soon as it lands and wait only for the XQ vector to finish it.
    if (nu > 0) {
        const int nconv = (int)blockDim.x - 64 * ngu;
        if (!is_g) mq_xq_dma_by(io.x, (int)H, smem, MQ_ZERO, 64 * ngu, nconv);
        // a bare barrier (no wait for the x DMAs): the control words are zero
        // and x is queued ahead of every weight
        __builtin_amdgcn_s_waitcnt(MQ_WC_LGKM0);
        __builtin_amdgcn_s_barrier();
        if (is_g) {
            gw.prologue();
            if (gw.Tn > 0) {
                const typename MQ<TG>::Pre gpr = gw.pre_first();
                mq_waves_wait(&ctl[MQ_FL_XSYNC], 3u * (uint32_t)(nconv >> 6), lane, io.err);
                gw.run_after(smem, gred, gpr);
            }
        } else {
            mq_xq_in_place_by((int)H, smem, MQ_ZERO, 64 * ngu, nconv, &ctl[MQ_FL_XSYNC], io.err);
            if (is_d) dw.prologue();
        }
    } else {
        // no x here: hold the down weights back a while, so that they do not
        // queue ahead of the other workgroups' x (bounded: a fixed time)
        if (is_d) {
            const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
            while (__builtin_amdgcn_s_memrealtime() - t0 < (uint64_t)geo.free_delay) __builtin_amdgcn_s_sleep(2);
            dw.prologue();
        }
        if (threadIdx.x < MQ_ZERO / 16) ((uint4 *)(smem))[threadIdx.x] = make_uint4(0, 0, 0, 0);
        __syncthreads();
    }

    if (is_g) {
        // ---- gate/up (run above); the last wave to finish publishes h
        if (mq_flow_count(&ctl[MQ_FL_GDONE], lane) != ngu - 1) return;
        // h = silu(g) * u and its XQ segments, four lanes per unit (lane j
        // of a quad: rows 4j .. 4j + 3), published with agent-scope stores
        __builtin_amdgcn_s_setprio(3);
        const int P = geo.gu.P, j = lane & 3;
        for (int m = lane >> 2; m < ((nu + 15) & ~15); m += 16) {
            const bool on = m < nu;
            const int mm = on ? m : nu - 1;
            float a[4];
#pragma unroll
            for (int i = 0; i < 4; i++)
                a[i] = silu_f32(mq_red_sum(gred, 2 * mm, P, 4 * j + i)) * mq_red_sum(gred, 2 * mm + 1, P, 4 * j + i);
            const XqQuad r = mq_xq_quad(a);
            if (on) {
                const int64_t seg = u0 + m;
                uint32_t *pl = (uint32_t *)(io.xq_h + (seg >> 4) * MQ_BREC + (seg & 15) * 48) + j;
                __hip_atomic_store(pl, r.p0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(pl + 4, r.p1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(pl + 8, r.p2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (j == 0) {
                    float *xs = (float *)(io.xq_h + mq_xq_planes(I));
                    __hip_atomic_store(&xs[seg], r.xs, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(&xs[I / 16 + seg], r.gs, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(&xs[I / 8 + seg], r.gq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        }
        // every lane's h stores have completed before the count goes up; no
        // release fence: it would write back the whole L2, and the stores
        // are agent-scope already
        __builtin_amdgcn_s_waitcnt(0);
        uint32_t old = 0;
        if (lane == 0) old = __hip_atomic_fetch_add(io.hcnt, (uint32_t)nu, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        old = (uint32_t)__builtin_amdgcn_readfirstlane((int)old);
        if (old + (uint32_t)nu == (uint32_t)U) {
            // h is complete (every other unit's stores completed before its
            // add): zero the count for the next launch, release the down rows
            if (lane == 0) __hip_atomic_store(io.hcnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            for (int64_t bb = lane; bb < G; bb += 64)
                if (mq_flow_nd(geo, U, G, bb) > 0)
                    __hip_atomic_store(&io.flags[bb * MQ_FL_FSTRIDE], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return;
    }
    if (!is_d) return;

    // ---- down: each wave decodes its first step while h is pending; the
    // first down wave waits for h and fetches XQ(h) into LDS
    typename MQ<TD>::Pre pr;
    if (dw.Tn > 0) pr = dw.pre_first();
    if (w == ngu) {
        bool ok = true;
        if (lane == 0) ok = mq_flow_poll(&io.flags[b * MQ_FL_FSTRIDE], io.err);
        ok = __builtin_amdgcn_readfirstlane((int)ok) != 0;
        if (ok) {
            // XQ(h) (4 I bytes, a multiple of 1 KB) by agent-scope LDS DMA,
            // issued after the flag load returned; no acquire fence (it
            // would invalidate the whole L2)
            const uint32_t xq = mq_lds_addr(smem + geo.o_xqh);
            for (int c = 0; c < (int)(I >> 8); c++)
                mq_dma16_agent(io.xq_h, (uint32_t)c * 1024u + 16u * (uint32_t)lane, xq + (uint32_t)c * 1024u);
            __builtin_amdgcn_s_waitcnt(mq_wc_vm(0));
        }
        __hip_atomic_store(&ctl[MQ_FL_HREADY], ok ? 1u : 2u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    {
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        uint32_t st;
        while ((st = __hip_atomic_load(&ctl[MQ_FL_HREADY], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP)) == 0u) {
            __builtin_amdgcn_s_sleep(1);
            if (__builtin_amdgcn_s_memrealtime() - t0 > 2 * MQ_WAIT_TICKS) {
                if (lane == 0) __hip_atomic_store(io.err, 4u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                st = 2u;
                break;
            }
        }
        if (st != 1u) return;
    }
    if (dw.Tn > 0) dw.run_after(smem, dred, pr);
    if (mq_flow_count(&ctl[MQ_FL_DDONE], lane) != ndw - 1) return;
    for (int i = lane; i < nd * 16; i += 64) {
        const int64_t r = (dstart + (i >> 4)) * 16 + (i & 15);
        if (r < H) io.y[r] = mq_red_sum(dred, i >> 4, dg.P, i & 15);
    }
}

__device__ __forceinline__ void mq_flow(const MqProj &gate, const MqProj &up, const MqProj &down, int32_t expert,
                                        const MqFlowIo &io, const MqFlowGeo &geo) {
    const int64_t e = expert;
    const int tg = gate.type, td = down.type;
    if (false) {
    }
#define MQ_FLOW_CASE(A, B) \
    else if (tg == A && td == B) mq_flow_body<A, B>(gate, up, down, e, io, geo);
    MQ_FLOW_CASE(ST_Q2_K, ST_Q2_K) MQ_FLOW_CASE(ST_Q2_K, ST_Q3_K) MQ_FLOW_CASE(ST_Q2_K, ST_Q4_K)
    MQ_FLOW_CASE(ST_Q3_K, ST_Q2_K) MQ_FLOW_CASE(ST_Q3_K, ST_Q3_K) MQ_FLOW_CASE(ST_Q3_K, ST_Q4_K)
    MQ_FLOW_CASE(ST_Q4_K, ST_Q2_K) MQ_FLOW_CASE(ST_Q4_K, ST_Q3_K) MQ_FLOW_CASE(ST_Q4_K, ST_Q4_K)
#undef MQ_FLOW_CASE
}

#define SEPIA_MQ_FLOW()                                                                                   \
    extern "C" __global__ __launch_bounds__(1024) void sepia_mq_ffn(MqProj gate, MqProj up, MqProj down,  \
                                                                    int32_t expert, MqFlowIo io,          \
                                                                    MqFlowGeo geo) {                      \
        mq_flow(gate, up, down, expert, io, geo);                                                         \
    }
