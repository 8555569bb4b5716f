#!/usr/bin/env python3
"""Benchmark of SEPIA's quantized-weight decode path on one MI355X.

Headline workload ("C3"): the full MoE decode layer
at batch 1 through the library's C ABI (sepia_gpu_moe_decode): f32 router
[258, 6144], sigmoid selection with a selection-only bias, top-6 of 256
routed experts (gate/up Q2_K [3072x6144], down Q3_K [6144x3072]) plus 2
shared Q4_K experts, SwiGLU, weighted sum. A step is one token through one
layer. 8 such layers (42 GB) are resident in HBM and the steps rotate over
them and over 64 input vectors, so every step's router, shared experts and
selected experts come from HBM rather than the 256 MB Infinity Cache.

value  = algorithmic bytes per token-layer (router + 6 routed + 2 shared
         experts' packed weights) / time per step, with the K timed steps
         replayed from one HIP graph (inputs resident in HBM, host issue
         overhead out of the timed region); us_per_token is the same time.
roofline.achieved = algorithmic bytes of the dominant kernel (the gate/up
         launch) per launch / its average launch duration, from HIP events
         recorded around each launch on the library's stream
         (sepia_hip_profile_*).
cpu_baseline = the C oracle's scalar MoE layer (the reference's
         mlp_moe_forward: qlinear per-row dequant + double accumulate) on one
         host core, on the same token and experts, over a bounded sample.
extra  = the other BASELINE configurations (C1 Q4_K matvec, C2 one expert
         FFN, C4 IQ matvecs, C5 512-token prefill MoE layer) measured the same
         way, and the C3 layer in the real checkpoint's formats (IQ2_XS
         gate/up, IQ3_XXS down, Q5_K/Q6_K shared experts).
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "quantized-weight GB/s (% of HBM peak); MoE layer µs/token at decode batch 1"
SCALE_LO, SCALE_HI = 2.0 ** -10, 2.0 ** -6
Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ2_XXS, IQ2_XS, IQ3_XXS, IQ4_XS = 8, 10, 11, 12, 13, 14, 16, 17, 18, 23
GEOM = {8: (32, 34), 10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210),
        16: (256, 66), 17: (256, 74), 18: (256, 98), 23: (256, 136)}
# Formats of a MoE layer: (routed gate/up, routed down, shared gate/up, shared down).
C3_TYPES = (Q2_K, Q3_K, Q4_K, Q4_K)
# The real checkpoint's most common layer (reference docs/gguf-inventory-ud-q2_k_xl.md:72-111):
# IQ2_XS gate/up, IQ3_XXS down; shared experts Q5_K gate/up, Q6_K down.
REAL_TYPES = (IQ2_XS, IQ3_XXS, Q5_K, Q6_K)


def log(*a):
    print("bench:", *a, file=sys.stderr, flush=True)


def mat_bytes(t, rows, cols):
    be, bb = GEOM[t]
    return rows * (cols // be) * bb


class HipRT:
    """The few HIP runtime calls the benchmark needs (events, stream capture)."""

    def __init__(self):
        self.L = ctypes.CDLL("libamdhip64.so")

    def ok(self, e, what):
        if e != 0:
            raise RuntimeError("%s failed with hipError %d" % (what, e))

    def event(self):
        ev = ctypes.c_void_p()
        self.ok(self.L.hipEventCreate(ctypes.byref(ev)), "hipEventCreate")
        return ev

    def record(self, ev, stream):
        self.ok(self.L.hipEventRecord(ev, ctypes.c_void_p(stream)), "hipEventRecord")

    def elapsed_ms(self, a, b):
        self.ok(self.L.hipEventSynchronize(b), "hipEventSynchronize")
        ms = ctypes.c_float()
        self.ok(self.L.hipEventElapsedTime(ctypes.byref(ms), a, b), "hipEventElapsedTime")
        return ms.value

    def sync(self, stream):
        self.ok(self.L.hipStreamSynchronize(ctypes.c_void_p(stream)), "hipStreamSynchronize")

    def capture(self, stream, issue):
        """Capture everything issue() launches on `stream` into an executable graph."""
        self.ok(self.L.hipStreamBeginCapture(ctypes.c_void_p(stream), 1), "hipStreamBeginCapture")
        try:
            issue()
        finally:
            graph = ctypes.c_void_p()
            e = self.L.hipStreamEndCapture(ctypes.c_void_p(stream), ctypes.byref(graph))
        self.ok(e, "hipStreamEndCapture")
        exe = ctypes.c_void_p()
        self.ok(self.L.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, ctypes.c_size_t(0)),
                "hipGraphInstantiate")
        self.L.hipGraphDestroy(graph)
        return exe

    def launch_graph(self, exe, stream):
        self.ok(self.L.hipGraphLaunch(exe, ctypes.c_void_p(stream)), "hipGraphLaunch")

    def destroy_graph(self, exe):
        self.L.hipGraphExecDestroy(exe)


TIMING = "graph"


class Bench:
    def __init__(self, dev):
        from sepia_amd import hip
        self.hip = hip
        self.dev = dev
        self.L = dev.L
        self.rt = HipRT()
        self.stream = dev.stream()

    def private(self, nbytes):
        return self.dev.alloc(nbytes, private=True)

    def synth(self, t, buf, n_blocks, seed):
        self.dev.run(self.L.sepia_hip_synth_blocks, t, buf, 0, n_blocks, seed, SCALE_LO, SCALE_HI)

    def vectors(self, n, count, seed, scale=1.0):
        """count private f32 [n] buffers holding N(0, scale^2) vectors (host copies returned)."""
        rng = np.random.default_rng(seed)
        host, bufs = [], []
        for _ in range(count):
            v = (rng.standard_normal(n) * scale).astype(np.float32)
            sb = self.dev.shared_from(v)
            pb = self.private(n * 4)
            self.dev.run(self.L.sepia_gpu_copy, sb, 0, pb, 0, n)
            self.dev.free(sb)
            host.append(v)
            bufs.append(pb)
        return host, bufs

    def fetch(self, buf, off, nbytes):
        """Bytes [off, off + nbytes) of a private buffer (nbytes and off multiples of 4)."""
        sb = self.dev.alloc(nbytes)
        self.dev.run(self.L.sepia_gpu_copy, buf, off, sb, 0, nbytes // 4)
        out = self.dev.download(sb, nbytes, dtype=np.uint8)
        self.dev.free(sb)
        return out

    def timed_steps(self, step, warmup, steps):
        """W untimed warmup steps, then exactly `steps` steps between two events on the
        library's stream; returns ms per step. TIMING selects how the timed steps are issued:
        "graph" (default) replays all steps from one captured graph, "step-graphs" captures
        each step as its own HIP graph and launches the graphs back to back, "eager" issues
        them through the C ABI directly. Every mode first runs the exact timed
        sequence once untimed (graph upload, caches)."""
        dev = self.dev
        dev.begin()
        for i in range(warmup):
            dev.check(step(i), "warmup step")
        dev.end()
        e0, e1 = self.rt.event(), self.rt.event()
        if TIMING == "eager":
            for rep in range(2):
                dev.begin()
                self.rt.record(e0, self.stream)
                for i in range(steps):
                    dev.check(step(warmup + i), "timed step")
                self.rt.record(e1, self.stream)
                dev.end()
            return self.rt.elapsed_ms(e0, e1) / steps
        dev.begin()
        if TIMING == "graph":
            graphs = [self.rt.capture(self.stream, lambda: [dev.check(step(warmup + i), "captured step")
                                                            for i in range(steps)])]
        else:
            graphs = [self.rt.capture(self.stream, lambda i=i: dev.check(step(warmup + i), "captured step"))
                      for i in range(steps)]
        dev.end()
        for g in graphs:                               # first launch of each: graph upload, untimed
            self.rt.launch_graph(g, self.stream)
        self.rt.sync(self.stream)
        self.rt.record(e0, self.stream)
        for g in graphs:
            self.rt.launch_graph(g, self.stream)
        self.rt.record(e1, self.stream)
        ms = self.rt.elapsed_ms(e0, e1)
        for g in graphs:
            self.rt.destroy_graph(g)
        return ms / steps

    def kernel_used(self, step, n, candidates):
        """(name, average ms) of the candidate kernel that the steps launch."""
        st = self.kernel_stats(step, n, candidates, strict=False)
        for k in candidates:
            if st[k][0]:
                return k, st[k][1]
        raise RuntimeError("none of %s ran" % candidates)

    def kernel_ms(self, step, n, kernels):
        """Average per-launch duration of each named kernel over n eager steps
        (kernels that did not run are left out)."""
        return {k: ms for k, (cnt, ms) in self.kernel_stats(step, n, kernels).items() if cnt}

    def kernel_stats(self, step, n, kernels, chunks=4, strict=True):
        """(launches, average ms per launch) of each named kernel over n eager steps:
        the median over `chunks` consecutive runs of about n / chunks steps of each
        run's average, so that one stray slow launch does not move the figure.
        strict False: names the library does not know count as not launched."""
        dev = self.dev
        per = max(1, n // chunks)
        runs = {k: [] for k in kernels}
        cnts = {k: 0 for k in kernels}
        for c in range(chunks if n >= chunks else 1):
            self.L.sepia_hip_profile_reset()
            dev.begin()
            dev.check(self.L.sepia_hip_profile_start(), "profile_start")
            for i in range(c * per, (c + 1) * per if n >= chunks else n):
                dev.check(step(i), "profiled step")
            dev.check(self.L.sepia_hip_profile_stop(), "profile_stop")
            dev.end()
            for k in kernels:
                cnt, tot = ctypes.c_int64(), ctypes.c_double()
                ok = self.L.sepia_hip_profile_query(k.encode(), ctypes.byref(cnt), ctypes.byref(tot))
                if strict:
                    dev.check(ok, "query")
                if ok and cnt.value:
                    runs[k].append(tot.value / cnt.value)
                    cnts[k] += cnt.value
        return {k: (cnts[k], float(np.median(runs[k])) if runs[k] else 0.0) for k in kernels}


# HBM bytes per launch, measured with rocprofv3's FETCH_SIZE and WRITE_SIZE counters (each in its
# own run) and scaled by what the same counters read for the copy kernel of known size
# (profiles/*_hbm_traffic.md). Reported as roofline.traffic for the dominant kernel; None until
# measured for the current build.
MEASURED_TRAFFIC_C2 = {"sepia_mq_gateup": 13001871, "sepia_mq_down": 8582520}
MEASURED_TRAFFIC_C3 = {"sepia_moe_route": 6612357, "sepia_mq_gateup": 122283851, "sepia_mq_down": 72124327}
MEASURED_TRAFFIC_REAL = {"sepia_moe_route": 6612386, "sepia_mq_gateup": 118571552, "sepia_mq_down": 76561443}
MEASURED_TRAFFIC_C5 = {"sepia_pf_gateup_q": 2999146132, "sepia_pf_down_q": 1900014470}
MEASURED_TRAFFIC_C5_REAL = {"sepia_ph_gateup": 3364945920, "sepia_ph_down": 2298700800}   # moe_prefill_c5_real_counters.md


def cpu_sample(fn, min_seconds, max_calls):
    """Run fn until min_seconds have passed (at least once, at most max_calls); mean s/call."""
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        el = time.perf_counter() - t0
        if el >= min_seconds or n >= max_calls:
            return el / n, n


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# ------------------------------------------------------------------ configs
def run_c2(B, warmup, steps, cpu_seconds):
    """one routed expert FFN, Q2_K gate/up, Q3_K down."""
    hip, L = B.hip, B.L
    H, I, NE = 6144, 3072, 40
    gb, ub, db = mat_bytes(Q2_K, I, H), mat_bytes(Q2_K, I, H), mat_bytes(Q3_K, H, I)
    bufs = [B.private(NE * gb), B.private(NE * ub), B.private(NE * db)]
    B.synth(Q2_K, bufs[0], NE * I * H // 256, 11)
    B.synth(Q2_K, bufs[1], NE * I * H // 256, 12)
    B.synth(Q3_K, bufs[2], NE * H * I // 256, 13)
    xs_host, xs = B.vectors(H, 1, 21)
    y = B.private(H * 4)
    tg, tu, td = hip.ExpertTensor(bufs[0], 0, gb, Q2_K), hip.ExpertTensor(bufs[1], 0, ub, Q2_K), \
        hip.ExpertTensor(bufs[2], 0, db, Q3_K)
    ref = (ctypes.byref(tg), ctypes.byref(tu), ctypes.byref(td))

    def step(i):
        return L.sepia_gpu_expert_ffn(*ref, NE, i % NE, H, I, xs[0], y)

    ms = B.timed_steps(step, warmup, steps)
    # graph replay == eager result (the last captured step used expert (warmup+steps-1) % NE)
    e_last = (warmup + steps - 1) % NE
    y_graph = B.fetch(y, 0, H * 4).view(np.float32)
    step_bytes = gb + ub + db + H * 4 + I * 4 + H * 4
    K_GU, K_DN = "sepia_mq_gateup", "sepia_mq_down"
    kms = B.kernel_ms(step, min(steps, 4 * NE), [K_GU, K_DN])
    gu_bytes = gb + ub + H * 4 + I * 4
    dn_bytes = db + I * 4 + H * 4
    B.dev.run(L.sepia_gpu_expert_ffn, *ref, NE, e_last, H, I, xs[0], y)
    y_eager = B.fetch(y, 0, H * 4).view(np.float32)
    if not np.array_equal(y_graph.view(np.uint32), y_eager.view(np.uint32)):
        raise RuntimeError("graph replay differs from the eager result")

    # CPU baseline on the same expert's bytes; parity check of the GPU result
    import oracle
    wg = B.fetch(bufs[0], e_last * gb, gb)
    wu = B.fetch(bufs[1], e_last * ub, ub)
    wd = B.fetch(bufs[2], e_last * db, db)
    want = oracle.expert_ffn(Q2_K, wg, Q2_K, wu, Q3_K, wd, H, I, xs_host[0], threads=min(16, os.cpu_count() or 1))
    err = float(np.max(np.abs(y_eager - want)))
    scale = float(np.max(np.abs(want)))
    if err > 1e-4 * scale:
        raise RuntimeError("C2 parity: max|diff| %g > 1e-4 * %g" % (err, scale))
    s1, n1 = cpu_sample(lambda: oracle.expert_ffn(Q2_K, wg, Q2_K, wu, Q3_K, wd, H, I, xs_host[0], threads=1),
                        cpu_seconds, 1000)
    nthr = min(16, os.cpu_count() or 1)
    sN, nN = cpu_sample(lambda: oracle.expert_ffn(Q2_K, wg, Q2_K, wu, Q3_K, wd, H, I, xs_host[0], threads=nthr),
                        cpu_seconds / 4, 1000)
    for b in bufs + xs + [y]:
        B.dev.free(b)
    roof = dict(bound="hbm", kernel=K_GU, achieved=gu_bytes / (kms[K_GU] * 1e-3) / 1e9, peak=HBM_PEAK_GBS,
                unit="GB/s", frac=gu_bytes / (kms[K_GU] * 1e-3) / 1e9 / HBM_PEAK_GBS, bytes_per_launch=gu_bytes,
                avg_launch_us=kms[K_GU] * 1e3, traffic=MEASURED_TRAFFIC_C2.get(K_GU),
                other_kernels={K_DN: dict(bytes_per_launch=dn_bytes, avg_launch_us=kms[K_DN] * 1e3,
                                          achieved=dn_bytes / (kms[K_DN] * 1e-3) / 1e9,
                                          traffic=MEASURED_TRAFFIC_C2.get(K_DN))})
    return dict(
        ms=ms, us_per_step=ms * 1e3, step_bytes=step_bytes, gbs=step_bytes / (ms * 1e-3) / 1e9,
        hbm_frac=step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        parity=dict(max_abs_diff=err, y_inf=scale, bound="1e-4*||y||_inf"),
        roofline=roof, cpu=dict(s1=s1, n1=n1, sN=sN, nN=nN, threads=nthr))


def run_matvec_rotation(B, name, t, rows, cols, warmup, steps, cpu_seconds, seed):
    """One quantized matvec per step, rotating over >= 512 MB of weight copies."""
    L = B.L
    mb = mat_bytes(t, rows, cols)
    ncopy = max(2, -(-512 * 2 ** 20 // mb))
    w = B.private(ncopy * mb)
    B.synth(t, w, ncopy * rows * cols // 256, seed)
    xh, xs = B.vectors(cols, 1, seed + 1)
    y = B.private(rows * 4)

    def step(i):
        return L.sepia_gpu_matvec_q(t, w, (i % ncopy) * mb, xs[0], y, rows, cols)

    ms = B.timed_steps(step, warmup, steps)
    tname = {10: "q2_k", 11: "q3_k", 12: "q4_k", 17: "iq2_xs", 18: "iq3_xxs", 16: "iq2_xxs"}[t]
    cands = ["sepia_mq_mv_%s" % tname] + (["sepia_mv_%s" % tname] if t in (10, 11, 12) else []) + \
        ["sepia_matvec_generic_%s" % tname]   # the tile kernels exist for Q2_K, Q3_K, Q4_K
    kname, kms = B.kernel_used(step, min(steps, 2 * ncopy), cands)
    nbytes = mb + cols * 4 + rows * 4
    import oracle
    wh = B.fetch(w, 0, mb)
    s1, n1 = cpu_sample(lambda: oracle.qlinear(t, wh, rows, cols, xh[0], threads=1), cpu_seconds, 1000)
    B.dev.free(w)
    B.dev.free(xs[0])
    B.dev.free(y)
    return dict(name=name, ms_per_step=ms, bytes_per_step=nbytes, gbs=nbytes / (ms * 1e-3) / 1e9,
                hbm_frac=nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, copies_rotated=ncopy,
                kernel=kname, kernel_avg_us=kms * 1e3, kernel_gbs=nbytes / (kms * 1e-3) / 1e9,
                cpu_1core_ms=s1 * 1e3, cpu_1core_gbs=mb / s1 / 1e9)


def run_store(B, n_routed=32, reps=3):
    """The on-disk stores into HBM: a C3-shaped MoE layer (n_routed routed Q2_K/Q3_K experts, 2 shared
    Q4_K, f32 router) written in the reference's formats (GGUF part, sepia-index sidecar, resident.bin +
    manifest) under a temporary directory, then uploaded through the C ABI: resident.bin whole, the
    layer's experts into one buffer. GB/s of each upload from the page cache (the files were just
    written; the best of `reps` calls, with the first call's times beside them, as that one also
    allocates the library's pinned staging buffers), and the assembled layer's decode against the
    oracle."""
    import shutil
    import tempfile
    import time
    import oracle
    from sepia_amd import store_synth
    L, hip = B.L, B.hip
    H, I, NS = 6144, 3072, 2
    tmp = tempfile.mkdtemp(prefix="sepia-store-")
    try:
        t0 = time.time()
        paths, host = store_synth.write_layer_store(tmp, np.random.default_rng(71), layer=2, hidden=H, inter=I,
                                                    n_routed=n_routed, n_shared=NS, types=C3_TYPES,
                                                    n_parts=1)
        write_s = time.time() - t0
        t = L.sepia_hip_manifest_load(paths["manifest"].encode(), paths["bin"].encode())
        idx = L.sepia_hip_index_load(paths["index"].encode())
        if not t or not idx:
            raise RuntimeError("store: the sidecars did not parse")
        res_bytes = os.path.getsize(paths["bin"])
        up_s, lay_s = [], []
        for _ in range(reps):
            t1 = time.perf_counter()
            rbuf = L.sepia_hip_manifest_upload(t)
            t2 = time.perf_counter()
            ex = (hip.ExpertTensor * 3)()
            ebuf = L.sepia_hip_index_upload_layer(idx, None, 2, ex)
            t3 = time.perf_counter()
            if not rbuf or not ebuf:
                raise RuntimeError("store: upload failed")
            up_s.append(t2 - t1)
            lay_s.append(t3 - t2)
            last = (rbuf, ebuf, ex)
            if _ + 1 < reps:
                B.dev.free(rbuf)
                B.dev.free(ebuf)
        rbuf, ebuf, ex = last
        layer_bytes = 3 * n_routed * ex[0].stride
        desc = hip.MoeLayerDesc()
        if L.sepia_hip_moe_layer_from_stores(t, rbuf, 2, ex, n_routed, 6, 8.0, ctypes.byref(desc)) != 1:
            raise RuntimeError("store: layer descriptor failed")
        x = np.random.default_rng(72).standard_normal(H).astype(np.float32)
        xb, yb, rb = B.dev.shared_from(x), B.dev.alloc(H * 4), B.dev.alloc(64 * 4)
        B.dev.run(L.sepia_gpu_moe_decode, ctypes.byref(desc), xb, yb, rb)
        y = B.dev.download(yb, H)
        sel = B.dev.download(rb, 6, dtype=np.int32)
        spec = dict(host[2], topk=6, route_scale=8.0, global_scale=1.0)
        logits = oracle.linear_f32(spec["router_w"], x)
        chosen = check_selection(oracle, logits, spec["router_bias"], n_routed, NS, 6, sel, "store layer")
        want, _, _, _ = oracle.moe_layer(spec, x, force_idx=chosen, threads=min(16, os.cpu_count() or 1))
        err, scale = float(np.max(np.abs(y - want))), float(np.max(np.abs(want)))
        if err > 1e-4 * scale:
            raise RuntimeError("store layer parity: max|diff| %g > 1e-4 * %g" % (err, scale))
        for b in (xb, yb, rb, rbuf, ebuf):
            B.dev.free(b)
        L.sepia_hip_manifest_free(t)
        L.sepia_hip_index_free(idx)
        return dict(n_routed=n_routed, write_s=write_s, resident_bytes=res_bytes, layer_bytes=layer_bytes,
                    resident_upload_ms=1e3 * min(up_s), layer_upload_ms=1e3 * min(lay_s),
                    first_resident_upload_ms=1e3 * up_s[0], first_layer_upload_ms=1e3 * lay_s[0],
                    resident_gbs=res_bytes / min(up_s) / 1e9, layer_gbs=layer_bytes / min(lay_s) / 1e9,
                    source="page cache (files just written)",
                    parity=dict(max_abs_diff=err, y_inf=scale, bound="1e-4*||y||_inf",
                                selection=[int(v) for v in sel]))
    finally:
        shutil.rmtree(tmp, ignore_errors=True)


def run_copy(B, steps):
    """sepia_copy_f32 over 256 MiB (read 256 MiB, write 256 MiB) per launch: the known-size
    kernel against which rocprofv3's FETCH_SIZE and WRITE_SIZE counters are scaled."""
    L = B.L
    n = 64 * 2 ** 20
    src, dst = B.private(4 * n), B.private(4 * n)

    def step(i):
        return L.sepia_gpu_copy(src, 0, dst, 0, n)

    kms = B.kernel_ms(step, min(steps, 10), ["sepia_copy_f32"])
    B.dev.free(src)
    B.dev.free(dst)
    return dict(bytes_read=4 * n, bytes_written=4 * n, launches=min(steps, 10),
                avg_launch_us=kms["sepia_copy_f32"] * 1e3, gbs=8 * n / (kms["sepia_copy_f32"] * 1e-3) / 1e9)


def ceiling_sizes():
    """(label, bytes) of the single launches the HBM read ceiling is measured at: each kernel's
    algorithmic weight bytes per launch (and the C3 layer's as one stream)."""
    return [("C3_router_f32", (256 + 2) * 6144 * 4),
            ("C1_q4_k_4096x4096", mat_bytes(Q4_K, 4096, 4096)),
            ("C2_down_q3_k", mat_bytes(Q3_K, 6144, 3072)),
            ("C4_iq2_xs_6144x6144", mat_bytes(IQ2_XS, 6144, 6144)),
            ("C2_gateup_q2_k", 2 * mat_bytes(Q2_K, 3072, 6144)),
            ("C4_iq3_xxs_6144x6144", mat_bytes(IQ3_XXS, 6144, 6144)),
            ("C3_down", 6 * mat_bytes(Q3_K, 6144, 3072) + 2 * mat_bytes(Q4_K, 6144, 3072)),
            ("C3_gateup", 12 * mat_bytes(Q2_K, 3072, 6144) + 4 * mat_bytes(Q4_K, 3072, 6144)),
            ("C3_layer_one_stream", (256 + 2) * 6144 * 4 + 12 * mat_bytes(Q2_K, 3072, 6144) + 4 * mat_bytes(Q4_K, 3072, 6144)
             + 6 * mat_bytes(Q3_K, 6144, 3072) + 2 * mat_bytes(Q4_K, 6144, 3072))]


def run_ceiling(B):
    """The HBM read ceiling of one launch at each size of ceiling_sizes(): the library's read probe
    (plain 16-byte streaming loads, nothing else) over copies rotated through 1.6 GB so the 256 MB
    Infinity Cache cannot serve them; per size the fastest of six grid shapes, average per-launch
    HIP-event time."""
    L = B.L
    total = 1600 << 20
    buf = B.private(total)
    out = {}
    for label, nbytes in ceiling_sizes():
        span = (nbytes + 4095) & ~4095
        ncopy = max(1, min(total // span, 64))
        n = max(24, 3 * ncopy)
        best = None
        for grid in (256, 512, 1024, 2048, 4096, 8192):
            def step(i, grid=grid):
                return L.sepia_hip_read_probe(buf, (i % ncopy) * span, nbytes, grid)
            us = B.kernel_ms(step, n, ["sepia_read_probe"])["sepia_read_probe"] * 1e3
            if best is None or us < best[0]:
                best = (us, grid)
        out[label] = dict(bytes=nbytes, us=round(best[0], 3), gbs=round(nbytes / (best[0] * 1e-6) / 1e9, 1),
                          grid=best[1], copies=ncopy)
    B.dev.free(buf)
    return out


def run_ceiling_dma(B):
    """The read of run_ceiling through the decode kernels' staging path (sepia_hip_read_probe_dma:
    per-wave LDS-DMA rings, each stage waited for, read back and refilled, no compute) at the C3
    down and gate/up sizes and C1's, for several grid / wave / ring shapes, with the plain probe at
    three grids beside it. Per shape: average per-launch HIP-event time over copies rotated
    through 1.6 GB."""
    L = B.L
    total = 1600 << 20
    buf = B.private(total)
    out = []
    for label, nbytes in (("C3_down", 69894144), ("C3_gateup", 116785152), ("C1", 9437184)):
        span = (nbytes + 4095) & ~4095
        ncopy = max(1, min(total // span, 64))
        n = max(24, 3 * ncopy)
        for grid in (256, 1024, 8192):
            us = B.kernel_ms(lambda i, g=grid: L.sepia_hip_read_probe(buf, (i % ncopy) * span, nbytes, g), n,
                             ["sepia_read_probe"])["sepia_read_probe"] * 1e3
            out.append(dict(size=label, probe="plain", grid=grid, threads=256, us=round(us, 2),
                            tbs=round(nbytes / us / 1e6, 2)))
        for grid, thr, kb, st in ((256, 1024, 7, 1), (256, 512, 7, 2), (256, 1024, 4, 1), (256, 1024, 4, 2),
                                  (256, 512, 4, 4), (256, 1024, 2, 4), (256, 1024, 1, 4), (512, 512, 7, 1),
                                  (512, 512, 4, 2), (1024, 256, 4, 2), (2048, 256, 4, 1)):
            us = B.kernel_ms(lambda i, g=grid, t=thr, k=kb, s=st: L.sepia_hip_read_probe_dma(
                buf, (i % ncopy) * span, nbytes, g, t, k, s), n, ["sepia_read_probe_dma"])["sepia_read_probe_dma"] * 1e3
            out.append(dict(size=label, probe="dma", grid=grid, threads=thr, kb=kb, stages=st, us=round(us, 2),
                            tbs=round(nbytes / us / 1e6, 2)))
            log("ceiling_dma", json.dumps(out[-1]))
    B.dev.free(buf)
    return out


def build_moe_layers(B, n_layers, types=C3_TYPES):
    """n_layers Inkling-shaped MoE layers resident in HBM: 256 routed experts (gate/up
    [3072x6144], down [6144x3072]) and 2 shared ones of the given formats (C3: Q2_K, Q3_K routed;
    Q4_K shared), f32 router [258, 6144] ~ N(0, 0.02), bias U(-0.1, 0.1). Returns (layers
    [(desc, buffers)], host routers [(rw, rb)], sizes)."""
    hip, L = B.hip, B.L
    H, I, NR, NS = 6144, 3072, 256, 2
    tg, td, tsg, tsd = types
    gb, db = mat_bytes(tg, I, H), mat_bytes(td, H, I)
    sgb, sdb = mat_bytes(tsg, I, H), mat_bytes(tsd, H, I)
    rng = np.random.default_rng(31)
    layers, host_router = [], []
    for li in range(n_layers):
        lb = dict(gate=B.private(NR * gb), up=B.private(NR * gb), down=B.private(NR * db),
                  s_gate=B.private(NS * sgb), s_up=B.private(NS * sgb), s_down=B.private(NS * sdb))
        B.synth(tg, lb["gate"], NR * I * H // GEOM[tg][0], 100 * li + 1)
        B.synth(tg, lb["up"], NR * I * H // GEOM[tg][0], 100 * li + 2)
        B.synth(td, lb["down"], NR * H * I // GEOM[td][0], 100 * li + 3)
        B.synth(tsg, lb["s_gate"], NS * I * H // GEOM[tsg][0], 100 * li + 4)
        B.synth(tsg, lb["s_up"], NS * I * H // GEOM[tsg][0], 100 * li + 5)
        B.synth(tsd, lb["s_down"], NS * H * I // GEOM[tsd][0], 100 * li + 6)
        rw = (rng.standard_normal((NR + NS, H)) * 0.02).astype(np.float32)
        rb = rng.uniform(-0.1, 0.1, NR).astype(np.float32)
        for key, arr in (("rw", rw), ("rb", rb)):
            sb = B.dev.shared_from(arr)
            lb[key] = B.private(arr.nbytes)
            B.dev.run(L.sepia_gpu_copy, sb, 0, lb[key], 0, arr.size)
            B.dev.free(sb)
        host_router.append((rw, rb))
        d = hip.MoeLayerDesc(hidden=H, inter=I, n_routed=NR, n_shared=NS, topk=6, route_scale=8.0,
                             global_scale=1.0, router_w=lb["rw"], router_bias=lb["rb"])
        d.gate, d.up, d.down = hip.ExpertTensor(lb["gate"], 0, gb, tg), hip.ExpertTensor(lb["up"], 0, gb, tg), \
            hip.ExpertTensor(lb["down"], 0, db, td)
        d.s_gate, d.s_up, d.s_down = hip.ExpertTensor(lb["s_gate"], 0, sgb, tsg), \
            hip.ExpertTensor(lb["s_up"], 0, sgb, tsg), hip.ExpertTensor(lb["s_down"], 0, sdb, tsd)
        layers.append((d, lb))
    return layers, host_router, (H, I, NR, NS, gb, db, sgb, sdb, types)


def layer_spec(B, lb, host_router, sizes, experts):
    """Oracle spec of a layer with the bytes of the given routed experts and the shared ones."""
    H, I, NR, NS, gb, db, sgb, sdb, (tg, td, tsg, tsd) = sizes
    rw, rb = host_router
    spec = dict(hidden=H, inter=I, n_routed=NR, n_shared=NS, topk=6, route_scale=8.0, global_scale=1.0,
                router_w=rw, router_bias=rb, t_gate=tg, t_up=tg, t_down=td, ts_gate=tsg, ts_up=tsg,
                ts_down=tsd, gate=[None] * NR, up=[None] * NR, down=[None] * NR,
                s_gate=[B.fetch(lb["s_gate"], s * sgb, sgb) for s in range(NS)],
                s_up=[B.fetch(lb["s_up"], s * sgb, sgb) for s in range(NS)],
                s_down=[B.fetch(lb["s_down"], s * sdb, sdb) for s in range(NS)])
    for e in sorted(set(int(v) for v in experts)):
        spec["gate"][e] = B.fetch(lb["gate"], e * gb, gb)
        spec["up"][e] = B.fetch(lb["up"], e * gb, gb)
        spec["down"][e] = B.fetch(lb["down"], e * db, db)
    return spec


def check_selection(oracle, logits, rb, n_routed, n_shared, topk, idx_gpu, what):
    """The GPU's selection must equal the oracle's (reference src/sepia.c:1329-1375) or differ only
    across a near-tie of the selection scores (rank topk vs topk + 1 closer than 1e-5: GPU expf and
    the router's f32 summation order can move such a tie). Returns the selection to check y with."""
    idx_ref, _ = oracle.route_select(logits, rb, n_routed, n_shared, topk, 8.0, 1.0)
    if list(idx_gpu) == list(idx_ref):
        return idx_ref
    score = 1.0 / (1.0 + np.exp(-logits[:n_routed].astype(np.float64))) + rb
    s_sorted = np.sort(score)[::-1]
    gap = s_sorted[topk - 1] - s_sorted[topk]
    if gap >= 1e-5:
        raise RuntimeError("%s: GPU selection %s differs from the oracle's %s (score gap %.3g)"
                           % (what, list(idx_gpu), list(idx_ref), gap))
    return np.asarray(idx_gpu, dtype=np.int32)


def run_c3(B, warmup, steps, cpu_seconds, n_layers=8, types=C3_TYPES, what="C3"):
    """full MoE decode layer, 256 routed (Q2_K/Q3_K) + 2 shared (Q4_K)
    experts resident, f32 router [258, 6144], top-6, no host round trip. types: the layer's
    formats (routed gate/up, routed down, shared gate/up, shared down), e.g. REAL_TYPES."""
    L = B.L
    layers, host_router, sizes = build_moe_layers(B, n_layers, types)
    H, I, NR, NS, gb, db, sgb, sdb, _ = sizes
    nx = 64
    xh, xs = B.vectors(H, nx, 41)
    y = B.private(H * 4)

    def step(i):
        d = layers[i % n_layers][0]
        return L.sepia_gpu_moe_decode(ctypes.byref(d), xs[i % nx], y, None)

    ms = B.timed_steps(step, warmup, steps)
    n_slots = 6 + NS
    per_token = (NR + NS) * H * 4 + 6 * (2 * gb + db) + NS * (2 * sgb + sdb)
    router = (NR + NS) * H * 4 + H * 4 + (NR + NS) * 4
    k_bytes = {"sepia_moe_route": router,
               "sepia_mq_gateup": 6 * 2 * gb + NS * 2 * sgb + H * 4 + n_slots * I * 4,
               "sepia_mq_down": 6 * db + NS * sdb + n_slots * I * 4 + H * 4}
    kms = B.kernel_ms(step, min(steps, 64), list(k_bytes))
    kms = {k: v for k, v in kms.items() if k in k_bytes}

    # parity at full size: selection and output of one token against the oracle
    import oracle
    nthr = min(16, os.cpu_count() or 1)
    d, lb = layers[0]
    route = B.dev.alloc(64)
    yb = B.dev.alloc(H * 4)
    B.dev.run(L.sepia_gpu_moe_decode, ctypes.byref(d), xs[0], yb, route)
    y_gpu = B.dev.download(yb, H)
    idx = B.dev.download(route, 6, dtype=np.int32)
    rw, rb = host_router[0]
    logits = oracle.linear_f32(rw, xh[0])
    chosen = check_selection(oracle, logits, rb, NR, NS, 6, idx, what)
    spec = layer_spec(B, lb, host_router[0], sizes, idx)
    want, _, _, _ = oracle.moe_layer(spec, xh[0], force_idx=chosen, threads=nthr)
    err = float(np.max(np.abs(y_gpu - want)))
    scale = float(np.max(np.abs(want)))
    if err > 1e-4 * scale:
        raise RuntimeError("%s parity: max|diff| %g > 1e-4 * %g" % (what, err, scale))
    s1, n1 = cpu_sample(lambda: oracle.moe_layer(spec, xh[0], force_idx=chosen, threads=1), cpu_seconds, 100)
    sN, nN = cpu_sample(lambda: oracle.moe_layer(spec, xh[0], force_idx=chosen, threads=nthr), cpu_seconds / 4, 100)
    B.dev.free(route)
    B.dev.free(yb)
    for d, lb in layers:
        for b in lb.values():
            B.dev.free(b)
    for b in xs + [y]:
        B.dev.free(b)
    measured = MEASURED_TRAFFIC_C3 if types == C3_TYPES else MEASURED_TRAFFIC_REAL if types == REAL_TYPES else {}
    kern = {k: dict(avg_launch_us=v * 1e3, bytes_per_launch=k_bytes[k], achieved_gbs=k_bytes[k] / (v * 1e-3) / 1e9,
                    traffic=measured.get(k))
            for k, v in kms.items()}
    return dict(ms=ms, us_per_token=ms * 1e3, kernel_sum_us=sum(kms.values()) * 1e3,
                bytes_per_token=per_token, gbs=per_token / (ms * 1e-3) / 1e9,
                roofline_us=per_token / (HBM_PEAK_GBS * 1e9) * 1e6,
                target_us=1.5 * per_token / (HBM_PEAK_GBS * 1e9) * 1e6,
                layers_rotated=n_layers, x_vectors=nx, kernels=kern,
                parity=dict(max_abs_diff=err, y_inf=scale, bound="1e-4*||y||_inf",
                            selection=[int(v) for v in idx], oracle_selection=[int(v) for v in chosen]),
                cpu=dict(s1=s1, n1=n1, sN=sN, nN=nN, threads=nthr))


def run_c5(B, warmup, steps, cpu_seconds, T=512, types=C3_TYPES):
    """the MoE layer for a batch of T tokens (prefill) with all 256 routed +
    2 shared experts resident, x ~ N(0,1) rounded to bf16-representable f32. types: the layer's
    formats (C3_TYPES: Q2_K / Q3_K routed, Q4_K shared, the int8 kernels; REAL_TYPES: the real
    checkpoint's IQ2_XS / IQ3_XXS routed, Q5_K / Q6_K shared, the f16 kernels)."""
    L = B.L
    layers, host_router, sizes = build_moe_layers(B, 1, types)
    H, I, NR, NS, gb, db, sgb, sdb, _ = sizes
    d, lb = layers[0]
    rng = np.random.default_rng(55)
    X = rng.standard_normal((T, H)).astype(np.float32)
    X = (X.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)
    sb = B.dev.shared_from(X)
    xb = B.private(X.nbytes)
    B.dev.run(L.sepia_gpu_copy, sb, 0, xb, 0, X.size)
    B.dev.free(sb)
    y = B.private(X.nbytes)

    def step(i):
        return L.sepia_gpu_moe_prefill(ctypes.byref(d), T, xb, y, None)

    ms = B.timed_steps(step, warmup, steps)
    knames = ["sepia_pf_route", "sepia_pf_route_m", "sepia_pf_select", "sepia_pf_group", "sepia_pf_split",
              "sepia_pf_gateup", "sepia_pf_down", "sepia_pf_combine", "sepia_pf_quant", "sepia_pf_gateup_q",
              "sepia_pf_down_q", "sepia_ph_quant", "sepia_ph_gateup", "sepia_ph_down"]
    kms = B.kernel_ms(step, min(steps, 5), knames)
    n_sel = 6 + NS
    route = B.dev.alloc(T * (6 + n_sel) * 4)
    yb = B.dev.alloc(X.nbytes)
    B.dev.run(L.sepia_gpu_moe_prefill, ctypes.byref(d), T, xb, yb, route)
    idx = B.dev.download(route, T * 6, dtype=np.int32).reshape(T, 6)
    touched = len(set(int(v) for v in idx.ravel()))
    wbytes = touched * (2 * gb + db) + NS * (2 * sgb + sdb) + (NR + NS) * H * 4
    act_bytes = 2 * T * H * 4
    flops = 2.0 * T * (6 * 3 * I * H + NS * 3 * I * H + (NR + NS) * H)
    # parity: every token's selection, and a sample of tokens' outputs, against the oracle
    import oracle
    rw, rb = host_router[0]
    chosen = [check_selection(oracle, oracle.linear_f32(rw, X[t]), rb, NR, NS, 6, idx[t], "C5 token %d" % t)
              for t in range(T)]
    sample = [0, 1, T // 2, T - 1]
    spec = layer_spec(B, lb, host_router[0], sizes, idx[sample].ravel())
    y_gpu = B.dev.download(yb, T * H).reshape(T, H)
    nthr = min(16, os.cpu_count() or 1)
    err, scale = 0.0, 0.0
    for t in sample:
        want, _, _, _ = oracle.moe_layer(spec, X[t], force_idx=chosen[t], threads=nthr)
        err = max(err, float(np.max(np.abs(y_gpu[t] - want))))
        scale = max(scale, float(np.max(np.abs(want))))
    if err > 1e-4 * scale:
        raise RuntimeError("C5 parity: max|diff| %g > 1e-4 * %g" % (err, scale))
    s1, n1 = cpu_sample(lambda: oracle.moe_layer(spec, X[0], force_idx=chosen[0], threads=1), cpu_seconds, 20)
    for b in list(lb.values()) + [xb, y, yb, route]:
        B.dev.free(b)
    sec = ms * 1e-3
    return dict(ms_per_layer=ms, tokens=T, tokens_per_s=T / sec, experts_touched=touched,
                weight_bytes=wbytes, hbm_gbs=(wbytes + act_bytes) / sec / 1e9,
                hbm_frac=(wbytes + act_bytes) / sec / 1e9 / HBM_PEAK_GBS,
                hbm_roofline_ms=(wbytes + act_bytes) / (HBM_PEAK_GBS * 1e9) * 1e3,
                gflop=flops / 1e9, tflops=flops / sec / 1e12, mfma_util_bf16=flops / sec / 2.5e15,
                # the int8 path issues three digit planes per product, at the 5.0 POP/s int8 peak
                mfma_util_int8_issued=3 * flops / sec / 5.0e15 if types == C3_TYPES else None,
                kernels_avg_ms={k: v for k, v in kms.items()},
                traffic_bytes=MEASURED_TRAFFIC_C5 if types == C3_TYPES else MEASURED_TRAFFIC_C5_REAL,
                parity=dict(tokens=sample, max_abs_diff=err, y_inf=scale, bound="1e-4*||y||_inf",
                            selections_checked=T),
                cpu_1core_ms_per_token=s1 * 1e3)


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--only", choices=["c3", "real", "c2", "c1", "c4", "c5", "c5real", "store", "copy", "ceiling",
                                       "ceiling_dma"],
                    default=None,
                    help="run one configuration (profiling runs; 'copy': the library's f32 copy kernel over "
                         "256 MiB, the reference for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE; 'ceiling': the "
                         "HBM read ceiling of a single launch at each kernel's size; 'ceiling_dma': the same read through "
                         "the decode kernels' LDS-DMA staging path); default: all")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--timing", choices=["graph", "step-graphs", "eager"], default="graph",
                    help="how the timed steps are issued (see Bench.timed_steps)")
    args = ap.parse_args()
    global TIMING
    TIMING = args.timing
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build measures one GPU only (the path has no multi-GPU "
              "component: each GPU would run it on its own experts' share). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    from sepia_amd import hip
    dev = hip.Device()
    B = Bench(dev)
    log("device", dev.name)
    extra = {}
    res = None
    t0 = time.time()
    ceil = None
    if args.only in (None, "ceiling"):
        ceil = run_ceiling(B)
        extra["hbm_read_ceiling"] = ceil
        log("ceiling", json.dumps(ceil))
    if args.only == "ceiling_dma":
        extra["hbm_read_ceiling_dma"] = run_ceiling_dma(B)
    if args.only in (None, "c3"):
        res = run_c3(B, args.warmup, args.steps, min(8.0, args.cpu_seconds))
        log("C3 %.2f us/token %.1f GB/s (%.1f%%) in %.0fs" % (res["us_per_token"], res["gbs"],
                                                              100 * res["gbs"] / HBM_PEAK_GBS, time.time() - t0))
    if args.only in (None, "real"):
        t1 = time.time()
        r = run_c3(B, args.warmup, args.steps, min(4.0, args.cpu_seconds), types=REAL_TYPES, what="C3 real types")
        r["workload"] = ("C3 shape with the real checkpoint's most common formats: IQ2_XS gate/up, IQ3_XXS down "
                         "(256 routed), Q5_K gate/up and Q6_K down (2 shared); 8 layers rotated")
        extra["C3_real_iq2xs_iq3xxs_q5k_q6k"] = r
        log("C3 real types %.2f us/token %.1f GB/s (%.1f%%) in %.0fs" % (r["us_per_token"], r["gbs"],
                                                                         100 * r["gbs"] / HBM_PEAK_GBS,
                                                                         time.time() - t1))
    if args.only in (None, "c2"):
        extra["C2_expert_ffn"] = run_c2(B, args.warmup, args.steps, min(4.0, args.cpu_seconds))
        log("C2", json.dumps(extra["C2_expert_ffn"]))
    if args.only in (None, "c1"):
        extra["C1_q4_k_4096x4096"] = run_matvec_rotation(B, "C1", Q4_K, 4096, 4096, args.warmup, args.steps,
                                                         min(3.0, args.cpu_seconds), 51)
        log("C1", json.dumps(extra["C1_q4_k_4096x4096"]))
    if args.only in (None, "c4"):
        for key, t in (("C4_iq3_xxs_6144x6144", IQ3_XXS), ("C4_iq2_xs_6144x6144_substitute", IQ2_XS)):
            extra[key] = run_matvec_rotation(B, key, t, 6144, 6144, args.warmup, args.steps,
                                             min(3.0, args.cpu_seconds), 61 + t)
            log(key, json.dumps(extra[key]))
    if args.only in (None, "c5"):
        extra["C5_moe_prefill_512"] = run_c5(B, min(args.warmup, 2), min(args.steps, 10), min(3.0, args.cpu_seconds))
        log("C5", json.dumps(extra["C5_moe_prefill_512"]))
    if args.only in (None, "c5", "c5real"):
        r = run_c5(B, min(args.warmup, 2), min(args.steps, 10), min(2.0, args.cpu_seconds), types=REAL_TYPES)
        r["workload"] = ("C5 with the real checkpoint's most common formats: IQ2_XS gate/up, IQ3_XXS down "
                         "(256 routed), Q5_K gate/up and Q6_K down (2 shared)")
        extra["C5_real_iq2xs_iq3xxs_q5k_q6k"] = r
        log("C5 real", json.dumps(r))
    if args.only in (None, "store"):
        extra["store_upload_c3_layer"] = run_store(B)
        log("store", json.dumps(extra["store_upload_c3_layer"]))
    if args.only == "copy":
        extra["copy_f32_256MiB"] = run_copy(B, args.steps)
        log("copy", json.dumps(extra["copy_f32_256MiB"]))
    if res is None:
        print(json.dumps(extra, indent=1))
        return

    dom = max(res["kernels"], key=lambda k: res["kernels"][k]["avg_launch_us"])
    kd = res["kernels"][dom]
    nproc = os.cpu_count() or 1
    line = {
        "metric": METRIC,
        "value": round(res["gbs"], 2),
        "unit": "GB/s",
        "us_per_token": round(res["us_per_token"], 3),
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["ms"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded random GGUF blocks, f16 scales U[2^-10,2^-6]; router N(0,0.02), "
                "bias U(-0.1,0.1); x ~ N(0,1))",
        "config": {"workload": "C3: full MoE decode layer at batch 1, hidden 6144: f32 router [258x6144], "
                               "top-6 of 256 routed experts (gate/up Q2_K [3072x6144], down Q3_K [6144x3072]) "
                               "+ 2 shared Q4_K experts; 8 layers (42 GB) resident in HBM and 64 x vectors, "
                               "rotated per step",
                   "bytes_per_token": res["bytes_per_token"], "us_per_token": round(res["us_per_token"], 3),
                   "kernel_sum_us": round(res["kernel_sum_us"], 3), "timing": TIMING,
                   "target_us_per_token": round(res["target_us"], 2),
                   "hbm_bound_us_per_token": round(res["roofline_us"], 2),
                   "hbm_frac": round(res["gbs"] / HBM_PEAK_GBS, 4)},
        "roofline": {"bound": "hbm", "achieved": round(kd["achieved_gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(kd["achieved_gbs"] / HBM_PEAK_GBS, 4), "traffic": MEASURED_TRAFFIC_C3.get(dom),
                     "kernel": dom, "bytes_per_launch": kd["bytes_per_launch"],
                     "avg_launch_us": round(kd["avg_launch_us"], 3),
                     "single_launch_ceiling_gbs": ceil["C3_gateup"]["gbs"] if ceil else None,
                     "frac_of_ceiling": round(kd["achieved_gbs"] / ceil["C3_gateup"]["gbs"], 4) if ceil else None,
                     "other_kernels": {k: {kk: (round(vv, 3) if isinstance(vv, float) else vv)
                                           for kk, vv in v.items() if kk != "traffic" or vv is not None}
                                       for k, v in res["kernels"].items() if k != dom}},
        "cpu_baseline": {"value": round(res["cpu"]["s1"] * 1e6, 1), "unit": "us/token", "cores": 1,
                         "kind": "port", "nproc": nproc,
                         "sample": "oracle MoE layer (the reference's mlp_moe_forward: f32 router, selection, "
                                   "qlinear per-row dequant + double accumulate) on the same token and experts, "
                                   "%d calls, %.1f ms/call on 1 core; %d threads: %.1f ms/call"
                                   % (res["cpu"]["n1"], res["cpu"]["s1"] * 1e3, res["cpu"]["threads"],
                                      res["cpu"]["sN"] * 1e3),
                         "cpu_model": cpu_model()},
        "parity": res["parity"],
        "extra": extra,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
