// mv.h -- split-K tile matvec for quantized rows (decode, batch 1).
//
// A 256-thread workgroup owns a tile: R = 16 * J rows x one column slice of
// NBC blocks (NBC * 256 columns). It
//   1. stages its slice of x in LDS as three int8 digit planes, a power-of-two
//      scale per block and f32 sums per 16 columns (one wave per block);
//   2. gives each lane one 64-weight unit of the slice (lane % 16 -> unit,
//      NBC = 4 gives 16 units per row slice): the lane keeps that unit's x
//      planes in registers and walks J rows, 4 rows per wave step, so 16
//      consecutive lanes cover one row and 64 lanes four consecutive rows;
//   3. sums the 16 lane partials of each row with butterfly shuffles.
// With KS = n_blocks / NBC > 1 slices, partial row sums go to a scratch array
// and the last workgroup to finish a row tile (an atomic arrival counter, no
// waiting) adds the KS partials in slice order -- deterministic, and it
// leaves the counter at zero for the next launch.
#pragma once
#include "common.h"
#include "qdot.h"

#define MV_THREADS 256
#define MV_NBC 4
#define MV_UC (4 * MV_NBC)           // units per row slice
#define MV_RW (SEPIA_WAVE / MV_UC)   // rows per wave step
#define MV_RS (4 * MV_RW)            // rows per workgroup step

struct __attribute__((aligned(16))) MvLds {
    int32_t planes[3][MV_NBC * 256 / 4];  // plane k, columns 4i..4i+3 in word i
    float scale[MV_NBC];
    float gsum[MV_NBC * 16];
    uint32_t last;
};

// Stage x[c0 .. c0 + NBC*256) (f32) into LDS. Thread t handles columns 4t..4t+3;
// wave w covers block w, so the block max is a wave reduction.
__device__ __forceinline__ void mv_stage_x(const float *__restrict__ x, int64_t c0, MvLds &L) {
    const int t = threadIdx.x;
    const float4 v = *(const float4 *)(x + c0 + 4 * t);
    float m = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, SEPIA_WAVE));
    // |x| * inv <= 8355000 < 127 * (65536 + 256 + 1): three balanced int8 digits
    const float inv = (m > 0.0f) ? 8355000.0f / m : 0.0f;
    const float vals[4] = {v.x, v.y, v.z, v.w};
    uint32_t w0 = 0, w1 = 0, w2 = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int32_t q = (int32_t)__builtin_rintf(vals[i] * inv);
        const int32_t lo = (int32_t)(int8_t)q;       // balanced base-256 digits
        const int32_t r1 = (q - lo) >> 8;
        const int32_t mid = (int32_t)(int8_t)r1;
        const int32_t hi = (r1 - mid) >> 8;
        w0 |= ((uint32_t)hi & 0xFFu) << (8 * i);
        w1 |= ((uint32_t)mid & 0xFFu) << (8 * i);
        w2 |= ((uint32_t)lo & 0xFFu) << (8 * i);
    }
    L.planes[0][t] = (int32_t)w0;
    L.planes[1][t] = (int32_t)w1;
    L.planes[2][t] = (int32_t)w2;
    float s = (v.x + v.y) + (v.z + v.w);
    s += __shfl_xor(s, 1, SEPIA_WAVE);
    s += __shfl_xor(s, 2, SEPIA_WAVE);
    if ((t & 3) == 0) L.gsum[t >> 2] = s;
    if ((t & 63) == 0) L.scale[t >> 6] = (m > 0.0f) ? 1.0f / inv : 0.0f;
}

template <int T>
__device__ __forceinline__ void mv_load_xu(const MvLds &L, int unit, XU &X) {
    const int bl = unit >> 2, k = unit & 3;
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const int col = 256 * bl + QU<T>::seg_col(k, s);
#pragma unroll
        for (int p = 0; p < 3; p++) {
            const int4 v = *(const int4 *)&L.planes[p][col >> 2];
            X.p[p][4 * s + 0] = v.x;
            X.p[p][4 * s + 1] = v.y;
            X.p[p][4 * s + 2] = v.z;
            X.p[p][4 * s + 3] = v.w;
        }
        X.gsum[s] = L.gsum[col >> 4];
    }
    X.xs = L.scale[bl];
}

// Row handled by this thread at step j of a tile starting at r0.
__device__ __forceinline__ int64_t mv_row(int64_t r0, int j) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    return r0 + (int64_t)j * MV_RS + wave * MV_RW + lane / MV_UC;
}

// Issue the loads of this thread's unit for J rows of matrix W (rows x
// n_blocks blocks, row stride row_bytes) in column slice ks. Rows past `rows`
// read row rows-1 (in bounds) and are discarded by the caller. Loads are
// issued before x is staged so their latency overlaps the staging.
template <int T, int J>
__device__ __forceinline__ void mv_issue(const uint8_t *__restrict__ W, uint64_t row_bytes, int64_t rows,
                                         int64_t r0, int ks, typename QU<T>::Data (&d)[J]) {
    const int unit = threadIdx.x & (MV_UC - 1);
    const int bl = unit >> 2, k = unit & 3;
    const uint64_t col_off = (uint64_t)(ks * MV_NBC + bl) * QU<T>::bytes;
#pragma unroll
    for (int j = 0; j < J; j++) {
        int64_t r = mv_row(r0, j);
        r = r < rows ? r : rows - 1;
        d[j] = QU<T>::load(W + (uint64_t)r * row_bytes + col_off, k);
    }
}

// Row sums of the issued units: each 16-lane group adds its unit partials.
template <int T, int J>
__device__ __forceinline__ void mv_finish(const typename QU<T>::Data (&d)[J], const XU &X, float (&acc)[J]) {
    const int k = threadIdx.x & 3;
#pragma unroll
    for (int j = 0; j < J; j++) {
        float a = QU<T>::dot(d[j], k, X);
#pragma unroll
        for (int off = MV_UC / 2; off >= 1; off >>= 1) a += __shfl_xor(a, off, SEPIA_WAVE);
        acc[j] = a;
    }
}

// Partial sums cross workgroups (and XCDs, whose L2s are not coherent with
// each other) as agent-scope atomic stores and loads, which go to the
// coherent level directly; no L2 writeback or invalidate is needed.
__device__ __forceinline__ void part_store(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float part_load(const float *p) {
    return __hip_atomic_load((float *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// After every thread stored its partials with part_store: returns true in the
// workgroup that arrives last at counter *cnt (of `expect` arrivals), which
// then resets the counter. Each wave waits for its stores to be acknowledged
// (vmcnt 0) before the barrier, so every partial is in place before the
// workgroup's arrival is counted; nothing ever waits on another workgroup.
__device__ __forceinline__ bool mv_last_arrival(uint32_t *cnt, uint32_t expect, MvLds &L) {
    __builtin_amdgcn_s_waitcnt(0x0F70);   // gfx9 encoding: vmcnt(0), expcnt/lgkmcnt untouched
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t last = (old == expect - 1) ? 1u : 0u;
        if (last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        L.last = last;
    }
    __syncthreads();
    return L.last != 0;
}

// y = W x for one quantized matrix. grid = n_tiles * KS; tile = blockIdx / KS.
template <int T, int J>
__device__ __forceinline__ void mv_kernel_body(const uint8_t *__restrict__ W, uint64_t row_bytes, int64_t rows,
                                               int32_t n_ks, const float *__restrict__ x, float *__restrict__ y,
                                               float *__restrict__ part, uint32_t *__restrict__ cnt) {
    __shared__ MvLds L;
    const int64_t tile = blockIdx.x / n_ks;
    const int ks = (int)(blockIdx.x % n_ks);
    const int64_t r0 = tile * (MV_RS * J);
    typename QU<T>::Data d[J];
    mv_issue<T, J>(W, row_bytes, rows, r0, ks, d);
    mv_stage_x(x, (int64_t)ks * MV_NBC * 256, L);
    __syncthreads();
    XU X;
    mv_load_xu<T>(L, threadIdx.x & (MV_UC - 1), X);
    float acc[J];
    mv_finish<T, J>(d, X, acc);
    const bool writer = (threadIdx.x & (MV_UC - 1)) == 0;
    if (n_ks == 1) {
#pragma unroll
        for (int j = 0; j < J; j++) {
            const int64_t r = mv_row(r0, j);
            if (writer && r < rows) y[r] = acc[j];
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < J; j++) {
        const int64_t r = mv_row(r0, j);
        if (writer && r < rows) part_store(&part[(int64_t)ks * rows + r], acc[j]);
    }
    if (!mv_last_arrival(&cnt[tile], (uint32_t)n_ks, L)) return;
    for (int i = threadIdx.x; i < MV_RS * J; i += MV_THREADS) {
        const int64_t r = r0 + i;
        if (r >= rows) break;
        float s = 0.0f;
        for (int p = 0; p < n_ks; p++) s += part_load(&part[(int64_t)p * rows + r]);
        y[r] = s;
    }
}

#define SEPIA_MV_KERNEL(name, T, J)                                                                 \
    extern "C" __global__ __launch_bounds__(MV_THREADS) void sepia_mv_##name##_j##J(              \
        const uint8_t *__restrict__ W, uint64_t row_bytes, int64_t rows, int32_t n_ks,            \
        const float *__restrict__ x, float *__restrict__ y, float *__restrict__ part,             \
        uint32_t *__restrict__ cnt) {                                                             \
        mv_kernel_body<T, J>(W, row_bytes, rows, n_ks, x, y, part, cnt);                          \
    }
