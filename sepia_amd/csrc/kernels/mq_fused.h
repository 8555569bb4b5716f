// mq_fused.h -- the whole MoE layer for one token (router, selection, gate/up,
// down, slot sum) in ONE launch of the matrix-core pipelines of mq.h, and the
// single expert FFN the same way.
//
// Three launches pay three ramps (dispatch, first weight bytes, tail) and
// serialize the phases; here one persistent grid of exactly one workgroup
// per CU runs
//   X   XQ(x) into LDS, the router rows (agent-scope stores of the logits);
//   GU  wave 0 is the control wave: it waits at grid barrier 1 (every logit
//       published), runs the selection (route.h) into LDS and raises an LDS
//       flag. The other waves meanwhile stream the shared experts' gate/up
//       rows, which need no selection, then wait for the flag and stream the
//       routed experts' rows. (Without a router, the expert FFN, wave 0
//       streams as well.) The gate/up work of all slots is cut into
//       units of 16 rows (gate and up) and dealt to the workgroups in
//       contiguous runs of equal weight bytes, shared units first.
//       h = silu(g) * u leaves as XQ segments of 16 rows (agent-scope stores);
//   D   grid barrier 2; down of the workgroup's slot and rows from the slot's
//       XQ(h), the slot sum through per-row-group arrival counters (as
//       mq_down). Down weights start streaming while barrier 2 is pending.
//
// Grid barriers. The host launches this kernel only with gridDim.x (a power
// of two) workgroups that are all resident at once (one per CU, LDS-bound),
// on the library's single stream. Arrivals add to a counter that is never
// reset. Each workgroup reads the counter when it starts, before its own
// first arrival: barrier 1 cannot have completed by then, so the count is
// c0 + k with c0 a multiple of gridDim.x and k < gridDim.x, and barrier j of
// the launch completes when the counter reaches c0 + j * gridDim.x (the wrap
// at 2^32 lands on a multiple too). Arrivals thus need no returned value.
// Every wait is bounded in time; a wait that runs out raises an error flag
// (the host then fails the batch and zeroes counter and flag), every index
// used afterwards is still in range, and the kernel still ends.
#pragma once
#include "mq.h"


// Thread 0: wait until the barrier counter reaches target.
__device__ __forceinline__ void mq_grid_wait(const uint32_t *bar, uint32_t target, uint32_t *err) {
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    while ((int32_t)(__hip_atomic_load(bar, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - target) < 0) {
        __builtin_amdgcn_s_sleep(1);
        if (__builtin_amdgcn_s_memrealtime() - t0 > MQ_WAIT_TICKS) {
            __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
    }
}
__device__ __forceinline__ void mq_grid_arrive(uint32_t *bar) {
    __hip_atomic_fetch_add(bar, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Geometry and LDS layout of a fused launch (host mirror in sepia_hip.c).
struct MqFuseGeo {
    MqGeo gu, dn;                      // parts and ring bytes per phase
    int32_t dn_wps_r, dn_wps_s;        // down: workgroups per routed / shared slot
    uint32_t o_sel, o_gred, o_xqh, o_dred, o_flag, o_rings;   // LDS offsets (XQ(x) at MQ_ZERO)
};

// Buffers and layer constants of a fused launch. rw NULL: no router, the
// routed slots are experts fixed + slot (the expert FFN).
struct MqFuseIo {
    const float *rw;
    int64_t ld;
    const float *bias;
    const float *x;
    int32_t n_routed, n_shared, topk, fixed;
    float route_scale, global_scale;
    int64_t inter, hidden;
    float *logits;
    int32_t *sel_idx;
    float *sel_w;
    uint8_t *xq_h;                     // [n_slots][XQ of inter], agent-scope
    float *ypart;                      // [n_slots][hidden]
    uint32_t *cnt, *bar, *err;
    float *y;
};

// The selection region (o_sel, MQ_FSEL_BYTES): idx[64], w[64], the flag.
#define MQ_SEL_FLAG 128
#define MQ_FSEL_BYTES 1024

// XQ segment r of a vector published with agent-scope stores (layout of
// xq_store).
__device__ __forceinline__ void xq_store_agent(const XqSeg &r, uint8_t *xq, int64_t n, int64_t seg) {
    uint32_t *pl = (uint32_t *)(xq + (seg >> 4) * MQ_BREC + (seg & 15) * 48);
    const uint32_t v[12] = {r.p0.x, r.p0.y, r.p0.z, r.p0.w, r.p1.x, r.p1.y, r.p1.z, r.p1.w,
                            r.p2.x, r.p2.y, r.p2.z, r.p2.w};
#pragma unroll
    for (int i = 0; i < 12; i++) __hip_atomic_store(&pl[i], v[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    float *xs = (float *)(xq + mq_xq_planes(n));
    __hip_atomic_store(&xs[seg], r.xs, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&xs[n / 16 + seg], r.gs, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&xs[n / 8 + seg], r.gq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Gate/up units of a workgroup: a unit is 16 rows of one slot's gate and up;
// the us shared units (ws weight bytes each) come first, then the ur routed
// ones (wr bytes each). Workgroup b of G takes the units whose first byte
// lies in [b T / G, (b + 1) T / G), T the total: shared units [s0, s0 + ns)
// and routed units [r0, r0 + nr). (Host mirror: mq_gu_range in sepia_hip.c.)
struct MqGuRange {
    int32_t s0, ns, r0, nr;
};
__device__ __forceinline__ int64_t mq_cdiv_pos(int64_t a, int64_t d) { return a <= 0 ? 0 : (a + d - 1) / d; }
__device__ __forceinline__ MqGuRange mq_gu_range(int64_t us, int64_t ws, int64_t ur, int64_t wr, int64_t G,
                                                 int64_t b) {
    const int64_t S = us * ws, T = S + ur * wr;
    const int64_t lo = T * b / G, hi = T * (b + 1) / G;
    int64_t a0 = 0, a1 = 0;
    if (us > 0) {
        a0 = mq_cdiv_pos(lo, ws);
        a1 = mq_cdiv_pos(hi, ws);
        a0 = a0 < us ? a0 : us;
        a1 = a1 < us ? a1 : us;
    }
    int64_t b0 = mq_cdiv_pos(lo - S, wr), b1 = mq_cdiv_pos(hi - S, wr);
    b0 = b0 < ur ? b0 : ur;
    b1 = b1 < ur ? b1 : ur;
    MqGuRange g;
    g.s0 = (int32_t)a0;
    g.ns = (int32_t)(a1 - a0);
    g.r0 = (int32_t)b0;
    g.nr = (int32_t)(b1 - b0);
    return g;
}

// Down slot and row-group stride of a workgroup for a split of wps_r
// workgroups per routed slot and wps_s per shared one. Workgroups past
// topk * wps_r + n_shared * wps_s idle in the phase (slot 0, no row groups)
// but still arrive at barrier 2.
struct MqSlotMap {
    int32_t slot, j0, jstep;
    bool routed;
};
__device__ __forceinline__ MqSlotMap mq_slot_map(int32_t topk, int32_t n_shared, int32_t wps_r, int32_t wps_s,
                                                 int32_t tiles) {
    MqSlotMap m;
    const int32_t bid = (int32_t)blockIdx.x;
    m.routed = bid < topk * wps_r;
    m.jstep = m.routed ? wps_r : wps_s;
    const int32_t k0 = m.routed ? bid : bid - topk * wps_r;
    m.slot = (m.routed ? 0 : topk) + k0 / m.jstep;
    m.j0 = k0 % m.jstep;
    if (m.slot >= topk + n_shared) {
        m.routed = topk > 0;
        m.slot = 0;
        m.j0 = tiles;
        m.jstep = 1;
    }
    return m;
}

// The router rows r = b, b + G, ... of workgroup b; rows r and r + G go
// together so that the workgroups with a second row end with the others, and
// every load of a batch of 4 chunks per thread is in flight at once. part:
// 2 x waves floats of LDS.
__device__ __forceinline__ void mq_fz_router(const MqFuseIo &io, float *part) {
    const int64_t n_tot = io.n_routed + io.n_shared, H = io.hidden;
    const int nt = (int)blockDim.x, nwv = nt >> 6, w = mq_wave_id();
    const bool vec = ((((uintptr_t)io.rw | (uintptr_t)io.x) & 15) == 0) && (io.ld & 3) == 0 && (H & 3) == 0;
    for (int64_t r = blockIdx.x; r < n_tot; r += 2 * (int64_t)gridDim.x) {
        const int64_t r2 = r + gridDim.x;
        const bool two = r2 < n_tot;
        const float *row0 = io.rw + r * io.ld, *row1 = io.rw + (two ? r2 : r) * io.ld;
        float a0 = 0.0f, a1 = 0.0f;
        if (vec) {
            const int n4 = (int)(H >> 2);
            const float4 *x4 = (const float4 *)io.x, *w0 = (const float4 *)row0, *w1 = (const float4 *)row1;
            for (int c0 = threadIdx.x; c0 < n4; c0 += 4 * nt) {
                float4 xv[4], v0[4], v1[4];
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const int c = c0 + u * nt;
                    if (c < n4) {
                        xv[u] = x4[c];
                        v0[u] = w0[c];
                        v1[u] = w1[c];
                    }
                }
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    if (c0 + u * nt < n4) {
                        a0 = __builtin_fmaf(v0[u].x, xv[u].x, a0);
                        a0 = __builtin_fmaf(v0[u].y, xv[u].y, a0);
                        a0 = __builtin_fmaf(v0[u].z, xv[u].z, a0);
                        a0 = __builtin_fmaf(v0[u].w, xv[u].w, a0);
                        a1 = __builtin_fmaf(v1[u].x, xv[u].x, a1);
                        a1 = __builtin_fmaf(v1[u].y, xv[u].y, a1);
                        a1 = __builtin_fmaf(v1[u].z, xv[u].z, a1);
                        a1 = __builtin_fmaf(v1[u].w, xv[u].w, a1);
                    }
                }
            }
        } else {
            for (int64_t c = threadIdx.x; c < H; c += nt) {
                const float xv = io.x[c];
                a0 = __builtin_fmaf(row0[c], xv, a0);
                a1 = __builtin_fmaf(row1[c], xv, a1);
            }
        }
        a0 = wave_sum(a0);
        a1 = wave_sum(a1);
        if ((threadIdx.x & 63) == 0) {
            part[w] = a0;
            part[nwv + w] = a1;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            float v0 = 0.0f, v1 = 0.0f;
            for (int k = 0; k < nwv; k++) {
                v0 += part[k];
                v1 += part[nwv + k];
            }
            __hip_atomic_store(&io.logits[r], v0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (two) __hip_atomic_store(&io.logits[r2], v1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
    }
}

// ---- phase GU: the shared units (format TS) then the routed ones (TG) on
// waves 1.., while wave 0 runs barrier 1 and the selection. Partial sums of
// unit m land in red slots 2 m (gate) and 2 m + 1 (up), shared units first.
template <int TS, int TG>
__device__ __forceinline__ void mq_fz_gu(const MqProj &gate, const MqProj &up, const MqProj &s_gate,
                                         const MqProj &s_up, const MqFuseIo &io, const MqFuseGeo &geo,
                                         const MqGuRange &gr, uint32_t target1, int32_t *si, float *sw) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int w = mq_wave_id();
    const int64_t I = io.inter;
    const int tiles_i = (int)((I + 15) >> 4);
    uint8_t *rings = smem + geo.o_rings;
    float *gred = (float *)(smem + geo.o_gred);
    int32_t *flag = si + MQ_SEL_FLAG;
    const int first = io.rw ? 1 : 0;   // without a router wave 0 streams too
    if (w == 0) {
        if (io.rw) {
            if (threadIdx.x == 0) mq_grid_wait(io.bar, target1, io.err);
            route_pick_any<true>(io.logits, io.bias, io.n_routed, io.n_shared, io.topk, io.route_scale,
                                 io.global_scale, si, sw);
            // workgroup 0 also hands the selection to the host
            if (blockIdx.x == 0 && (int)threadIdx.x < io.topk + io.n_shared) {
                if ((int)threadIdx.x < io.topk) io.sel_idx[threadIdx.x] = si[threadIdx.x];
                io.sel_w[threadIdx.x] = sw[threadIdx.x];
            }
        } else if (threadIdx.x < (unsigned)io.topk) {
            si[threadIdx.x] = io.fixed + (int32_t)threadIdx.x;
        }
        if (threadIdx.x == 0) __hip_atomic_store(flag, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (first) return;
    }
    // shared unit u: slot topk + u / tiles_i, expert u / tiles_i
    auto sitem = [&](int i) {
        const int32_t u = gr.s0 + (i >> 1);
        const int32_t e = u / tiles_i;
        MqItem it;
        it.base = ((i & 1) ? s_up.base : s_gate.base) + (int64_t)e * ((i & 1) ? s_up.stride : s_gate.stride);
        it.row0 = (int64_t)(u - e * tiles_i) * 16;
        it.rows = I;
        it.xoff = MQ_ZERO;
        it.red = i;
        return it;
    };
    {
        MqWave<TS, decltype(sitem)> sp(sitem, 2 * gr.ns, (int)(s_gate.n_blocks >> 2), (int)(256 * s_gate.n_blocks),
                                       (uint32_t)s_gate.row_bytes, geo.gu, rings, first);
        sp.prologue();
        sp.run(smem, gred);
    }
    if (gr.nr == 0) return;
    // the routed units need the selection
    {
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        while (__hip_atomic_load(flag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) == 0) {
            __builtin_amdgcn_s_sleep(1);
            if (__builtin_amdgcn_s_memrealtime() - t0 > 2 * MQ_WAIT_TICKS) {
                if ((threadIdx.x & 63) == 0) __hip_atomic_store(io.err, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                return;
            }
        }
    }
    const int32_t nbh = (int32_t)gate.n_blocks;
    auto ritem = [&](int i) {
        const int32_t u = gr.r0 + (i >> 1);
        const int32_t slot = u / tiles_i;
        const int64_t e = __builtin_amdgcn_readfirstlane(si[slot]);
        MqItem it;
        it.base = ((i & 1) ? up.base : gate.base) + e * ((i & 1) ? up.stride : gate.stride);
        it.row0 = (int64_t)(u - slot * tiles_i) * 16;
        it.rows = I;
        it.xoff = MQ_ZERO;
        it.red = 2 * gr.ns + i;
        return it;
    };
    MqWave<TG, decltype(ritem)> rp(ritem, 2 * gr.nr, nbh >> 2, (int)(256 * nbh), (uint32_t)gate.row_bytes, geo.gu,
                                   rings, first);
    rp.prologue();
    rp.run(smem, gred);
}

// ---- phase D for a workgroup whose down slot has format TD.
template <int TD>
__device__ __forceinline__ void mq_fz_dn(const MqProj &down, const MqProj &s_down, const MqFuseIo &io,
                                         const MqFuseGeo &geo, const MqSlotMap &dm, uint32_t target2,
                                         const int32_t *si, const float *sw) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int w = mq_wave_id();
    const int n_slots = io.topk + io.n_shared;
    const int64_t H = io.hidden, I = io.inter;
    uint8_t *rings = smem + geo.o_rings;
    float *dred = (float *)(smem + geo.o_dred);
    int32_t *dflag = (int32_t *)(smem + geo.o_flag);
    const uint32_t xqb = (uint32_t)mq_xq_bytes(I);
    const MqProj &D = dm.routed ? down : s_down;
    const int64_t de = dm.routed ? (int64_t)__builtin_amdgcn_readfirstlane(si[dm.slot]) : (int64_t)(dm.slot - io.topk);
    const uint8_t *wd = D.base + de * D.stride;
    const int tiles_h = (int)((H + 15) >> 4);
    const int dnk = dm.j0 < tiles_h ? (tiles_h - dm.j0 + dm.jstep - 1) / dm.jstep : 0;
    auto ditem = [&](int i) {
        MqItem it;
        it.base = wd;
        it.row0 = ((int64_t)dm.j0 + (int64_t)i * dm.jstep) * 16;
        it.rows = H;
        it.xoff = geo.o_xqh;
        it.red = i;
        return it;
    };
    MqWave<TD, decltype(ditem)> dw(ditem, dnk, (int)(D.n_blocks >> 2), (int)I, (uint32_t)D.row_bytes, geo.dn, rings);
    // barrier 2: arrive (before this workgroup's down weights queue up ahead
    // of the arrival), let the other waves start their down weights, wait
    if (threadIdx.x == 0) mq_grid_arrive(io.bar);
    if (dnk == 0) return;              // nothing to read: no need to wait
    __builtin_amdgcn_s_barrier();
    if (w > 0) dw.prologue();
    if (threadIdx.x == 0) mq_grid_wait(io.bar, target2, io.err);
    __syncthreads();
    if (w == 0) dw.prologue();

    // the slot's XQ(h) (agent-scope loads, 4 per thread in flight), then the rows
    {
        const uint32_t *src = (const uint32_t *)(io.xq_h + (size_t)dm.slot * xqb);
        uint32_t *dst = (uint32_t *)(smem + geo.o_xqh);
        const uint32_t nwd = xqb / 4, nt = blockDim.x;
        for (uint32_t i0 = threadIdx.x; i0 < nwd; i0 += 4 * nt) {
            uint32_t v[4];
#pragma unroll
            for (int u = 0; u < 4; u++)
                if (i0 + u * nt < nwd)
                    v[u] = __hip_atomic_load(&src[i0 + u * nt], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int u = 0; u < 4; u++)
                if (i0 + u * nt < nwd) dst[i0 + u * nt] = v[u];
        }
    }
    __syncthreads();
    dw.run(smem, dred);
    __syncthreads();
    if (n_slots == 1) {
        const float wv = io.rw ? sw[0] : 1.0f;
        for (int i = threadIdx.x; i < dnk * 16; i += blockDim.x) {
            const int64_t r = ((int64_t)dm.j0 + (int64_t)(i >> 4) * dm.jstep) * 16 + (i & 15);
            if (r < H) io.y[r] = wv * mq_red_sum(dred, i >> 4, geo.dn.P, i & 15);
        }
        return;
    }
    for (int i = threadIdx.x; i < dnk * 16; i += blockDim.x) {
        const int64_t r = ((int64_t)dm.j0 + (int64_t)(i >> 4) * dm.jstep) * 16 + (i & 15);
        if (r < H)
            __hip_atomic_store(&io.ypart[(int64_t)dm.slot * H + r], mq_red_sum(dred, i >> 4, geo.dn.P, i & 15),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (int k = threadIdx.x; k < dnk; k += blockDim.x) {
        const uint32_t prev = __hip_atomic_fetch_add(&io.cnt[dm.j0 + k * dm.jstep], 1u, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        dflag[k] = prev == (uint32_t)(n_slots - 1);
    }
    __syncthreads();
    // the last slot of a row group to arrive sums the slots in slot order
    // (up to 8 loads per row in flight)
    for (int i = threadIdx.x; i < dnk * 16; i += blockDim.x) {
        if (!dflag[i >> 4]) continue;
        const int64_t r = ((int64_t)dm.j0 + (int64_t)(i >> 4) * dm.jstep) * 16 + (i & 15);
        if (r >= H) continue;
        float acc = 0.0f;
        for (int s0 = 0; s0 < n_slots; s0 += 8) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; u++)
                v[u] = s0 + u < n_slots ? __hip_atomic_load(&io.ypart[(int64_t)(s0 + u) * H + r], __ATOMIC_RELAXED,
                                                            __HIP_MEMORY_SCOPE_AGENT)
                                        : 0.0f;
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (s0 + u < n_slots) acc = __builtin_fmaf(io.rw ? sw[s0 + u] : 1.0f, v[u], acc);
        }
        io.y[r] = acc;
    }
    for (int k = threadIdx.x; k < dnk; k += blockDim.x)
        if (dflag[k]) __hip_atomic_store(&io.cnt[dm.j0 + k * dm.jstep], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void mq_fused(const MqProj &gate, const MqProj &up, const MqProj &down,
                                         const MqProj &s_gate, const MqProj &s_up, const MqProj &s_down,
                                         const MqFuseIo &io, const MqFuseGeo &geo) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    int32_t *si = (int32_t *)(smem + geo.o_sel);
    float *sw = (float *)(si + 64);
    const int64_t I = io.inter, H = io.hidden;
    const int tiles_i = (int)((I + 15) >> 4);
    const uint32_t G = gridDim.x;

    // the barrier base (see the header); the selection starts in range and
    // its flag down
    uint32_t c0 = 0;
    if (threadIdx.x == 0) {
        c0 = __hip_atomic_load(io.bar, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        c0 -= c0 % G;
    }
    for (int i = threadIdx.x; i <= MQ_SEL_FLAG; i += blockDim.x) si[i] = 0;
    const uint32_t target1 = c0 + G, target2 = c0 + (io.rw ? 2u : 1u) * G;

    // ---- phase X (mq_stage_xq ends with a barrier)
    mq_stage_xq(io.x, 0, 1, (int)(256 * gate.n_blocks), smem, MQ_ZERO, 0u);
    if (io.rw) {
        mq_fz_router(io, (float *)(smem + geo.o_gred));
        if (threadIdx.x == 0) {
            __builtin_amdgcn_s_waitcnt(0);   // the logit stores have completed
            mq_grid_arrive(io.bar);
        }
        __builtin_amdgcn_s_barrier();        // the arrival leaves before any weight DMA
    }

    // ---- phase GU
    const MqGuRange gr = mq_gu_range(io.n_shared * (int64_t)tiles_i, 32 * (int64_t)s_gate.row_bytes,
                                     io.topk * (int64_t)tiles_i, 32 * (int64_t)gate.row_bytes, G, blockIdx.x);
    const int ts = io.n_shared > 0 ? s_gate.type : gate.type, tg = gate.type;
    if (false) {
    }
#define MQ_FG(A, B) \
    else if (ts == A && tg == B) mq_fz_gu<A, B>(gate, up, s_gate, s_up, io, geo, gr, target1, si, sw);
    MQ_FG(ST_Q2_K, ST_Q2_K) MQ_FG(ST_Q2_K, ST_Q3_K) MQ_FG(ST_Q2_K, ST_Q4_K)
    MQ_FG(ST_Q3_K, ST_Q2_K) MQ_FG(ST_Q3_K, ST_Q3_K) MQ_FG(ST_Q3_K, ST_Q4_K)
    MQ_FG(ST_Q4_K, ST_Q2_K) MQ_FG(ST_Q4_K, ST_Q3_K) MQ_FG(ST_Q4_K, ST_Q4_K)
#undef MQ_FG
    __syncthreads();

    // h = silu(gate) * up, one element per thread, written over part 0 of
    // the gate sums (only this thread reads that element); then one thread
    // per unit publishes its XQ segment
    float *gred = (float *)(smem + geo.o_gred);
    const int P = geo.gu.P, nu = gr.ns + gr.nr;
    for (int i = threadIdx.x; i < nu * 16; i += blockDim.x) {
        const int m = i >> 4, t = i & 15;
        const float hv = silu_f32(mq_red_sum(gred, 2 * m, P, t)) * mq_red_sum(gred, 2 * m + 1, P, t);
        gred[(2 * m * P) * 16 + t] = hv;
    }
    __syncthreads();
    const uint32_t xqb = (uint32_t)mq_xq_bytes(I);
    for (int m = threadIdx.x; m < nu; m += blockDim.x) {
        const bool sh = m < gr.ns;
        const int32_t u = sh ? gr.s0 + m : gr.r0 + (m - gr.ns);
        const int32_t slot = sh ? io.topk + u / tiles_i : u / tiles_i;
        float hv[16];
#pragma unroll
        for (int t = 0; t < 16; t++) hv[t] = gred[(2 * m * P) * 16 + t];
        xq_store_agent(xq_segment(hv), io.xq_h + (size_t)slot * xqb, I, u % tiles_i);
    }
    __builtin_amdgcn_s_waitcnt(0);   // this thread's h stores completed (no DMAs in flight)
    __syncthreads();

    // ---- phase D
    const MqSlotMap dm = mq_slot_map(io.topk, io.n_shared, geo.dn_wps_r, geo.dn_wps_s, (int32_t)((H + 15) >> 4));
    const int td = dm.routed ? down.type : s_down.type;
    if (td == ST_Q2_K) mq_fz_dn<ST_Q2_K>(down, s_down, io, geo, dm, target2, si, sw);
    else if (td == ST_Q3_K) mq_fz_dn<ST_Q3_K>(down, s_down, io, geo, dm, target2, si, sw);
    else mq_fz_dn<ST_Q4_K>(down, s_down, io, geo, dm, target2, si, sw);
}

#define SEPIA_MQ_FUSED()                                                                                 \
    extern "C" __global__ __launch_bounds__(1024) void sepia_mq_moe(MqProj gate, MqProj up, MqProj down, \
                                                                    MqProj s_gate, MqProj s_up,          \
                                                                    MqProj s_down, MqFuseIo io,          \
                                                                    MqFuseGeo geo) {                     \
        mq_fused(gate, up, down, s_gate, s_up, s_down, io, geo);                                         \
    }
