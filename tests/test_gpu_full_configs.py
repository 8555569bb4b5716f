"""BASELINE configurations C3 and C5 at their full size, through the C ABI.

C3: 256 routed experts (gate/up Q2_K [3072x6144], down Q3_K [6144x3072]) and
2 shared Q4_K experts resident in HBM, f32 router [258, 6144] ~ N(0, 0.02),
selection bias U(-0.1, 0.1), top-6 (reference src/sepia.c:1329-1470). The
selection runs route_pick with four experts per lane (E = 4), the branch a
layer of at most 64 experts never takes. A second router over the same
experts holds constructed exact ties: identical rows and biases inside one
lane's experts, across lanes, and at the rank-6 / rank-7 boundary, where the
reference's strict '>' arg-max must keep the lower index.

C5: the same layer for a 512-token batch (sepia_gpu_moe_prefill): every
token's selection against the oracle (near-ties per the reference's
protocol) and y against the oracle's single-token layer, for all 512 tokens
with the plain router (bf16-representable and full f32 x).

The real checkpoint's formats at the same size: IQ2_XS gate/up and IQ3_XXS
down routed, Q5_K gate/up and Q6_K down shared (docs/gguf-inventory-ud-q2_k_xl.md
in the reference): C3-shape decode, and C5 on the f16 prefill kernels.

Weights are generated on the GPU (sepia_hip_synth_blocks); only the experts
a checked token selects are copied back for the oracle.
"""
import ctypes
import os

import numpy as np
import pytest

from sepia_amd import hip, synth
from test_gpu_parity import Launches, assert_close, check_route

pytestmark = pytest.mark.gpu

THREADS = min(16, os.cpu_count() or 1)
H, I, NR, NS, TOPK = 6144, 3072, 256, 2, 6
Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ2_XS, IQ3_XXS = 10, 11, 12, 13, 14, 17, 18
C3_TYPES = (Q2_K, Q3_K, Q4_K, Q4_K)          # gate/up, down, shared gate/up, shared down
REAL_TYPES = (IQ2_XS, IQ3_XXS, Q5_K, Q6_K)
# constructed ties (expert ids; lane l of the selecting wave holds experts 4l .. 4l + 3)
TIE_IN_LANE = (8, 10)        # lane 2, register slots 0 and 2
TIE_ACROSS = (21, 100)       # lanes 5 and 25
SINGLE = 150
TIE_CUTOFF = (201, 230)      # lanes 50 and 57: only 201 may take the sixth slot


@pytest.fixture(scope="module")
def dev():
    return hip.Device()


def private_copy(dev, arr):
    """A private device buffer holding arr (through a shared staging buffer)."""
    a = np.ascontiguousarray(arr)
    sb = dev.shared_from(a)
    pb = dev.alloc(a.nbytes, private=True)
    dev.run(dev.L.sepia_gpu_copy, sb, 0, pb, 0, a.nbytes // 4)
    dev.free(sb)
    return pb


def fetch(dev, buf, off, nbytes):
    """Bytes [off, off + nbytes) of a private buffer (multiples of 4)."""
    sb = dev.alloc(nbytes)
    dev.run(dev.L.sepia_gpu_copy, buf, off, sb, 0, nbytes // 4)
    out = dev.download(sb, nbytes, dtype=np.uint8)
    dev.free(sb)
    return out


class FullLayer:
    """A full-size MoE layer resident on the GPU in the given formats, with a
    plain router and a router with constructed ties over the same experts."""

    def __init__(self, dev, types=C3_TYPES):
        self.dev = dev
        L = dev.L
        self.types = tg, td, tsg, tsd = types
        self.gb, self.db = synth.row_bytes(tg, H) * I, synth.row_bytes(td, I) * H
        self.sgb, self.sdb = synth.row_bytes(tsg, H) * I, synth.row_bytes(tsd, I) * H
        GB, DB, SGB, SDB = self.gb, self.db, self.sgb, self.sdb
        self.bufs = dict(gate=dev.alloc(NR * GB, private=True), up=dev.alloc(NR * GB, private=True),
                         down=dev.alloc(NR * DB, private=True), s_gate=dev.alloc(NS * SGB, private=True),
                         s_up=dev.alloc(NS * SGB, private=True), s_down=dev.alloc(NS * SDB, private=True))
        for k, t, n, seed in (("gate", tg, NR * I * H, 71), ("up", tg, NR * I * H, 72), ("down", td, NR * H * I, 73),
                              ("s_gate", tsg, NS * I * H, 74), ("s_up", tsg, NS * I * H, 75),
                              ("s_down", tsd, NS * H * I, 76)):
            dev.run(L.sepia_hip_synth_blocks, t, self.bufs[k], 0, n // synth.GEOM[t][0], seed, synth.SCALE_LO,
                    synth.SCALE_HI)
        rng = np.random.default_rng(2024)
        rw = (rng.standard_normal((NR + NS, H)) * 0.02).astype(np.float32)
        rb = rng.uniform(-0.1, 0.1, NR).astype(np.float32)
        self.routers = {"plain": (rw, rb)}
        rw_t, rb_t = rw.copy(), rb.copy()
        for (a, b), bias in ((TIE_IN_LANE, 10.0), (TIE_ACROSS, 9.0), (TIE_CUTOFF, 6.0)):
            rw_t[b] = rw_t[a]
            rb_t[a] = rb_t[b] = bias
        rb_t[SINGLE] = 8.0
        self.routers["ties"] = (rw_t, rb_t)
        self.descs = {}
        for name, (w, b) in self.routers.items():
            self.bufs["rw_" + name] = private_copy(dev, w)
            self.bufs["rb_" + name] = private_copy(dev, b)
            d = hip.MoeLayerDesc(hidden=H, inter=I, n_routed=NR, n_shared=NS, topk=TOPK, route_scale=8.0,
                                 global_scale=1.0, router_w=self.bufs["rw_" + name],
                                 router_bias=self.bufs["rb_" + name])
            d.gate = hip.ExpertTensor(self.bufs["gate"], 0, GB, tg)
            d.up = hip.ExpertTensor(self.bufs["up"], 0, GB, tg)
            d.down = hip.ExpertTensor(self.bufs["down"], 0, DB, td)
            d.s_gate = hip.ExpertTensor(self.bufs["s_gate"], 0, SGB, tsg)
            d.s_up = hip.ExpertTensor(self.bufs["s_up"], 0, SGB, tsg)
            d.s_down = hip.ExpertTensor(self.bufs["s_down"], 0, SDB, tsd)
            self.descs[name] = d
        self.shared = dict(s_gate=[fetch(dev, self.bufs["s_gate"], s * SGB, SGB) for s in range(NS)],
                           s_up=[fetch(dev, self.bufs["s_up"], s * SGB, SGB) for s in range(NS)],
                           s_down=[fetch(dev, self.bufs["s_down"], s * SDB, SDB) for s in range(NS)])
        self.cache = {}

    def spec(self, router, experts):
        """Oracle spec holding the bytes of the given routed experts."""
        rw, rb = self.routers[router]
        tg, td, tsg, tsd = self.types
        GB, DB = self.gb, self.db
        sp = dict(hidden=H, inter=I, n_routed=NR, n_shared=NS, topk=TOPK, route_scale=8.0, global_scale=1.0,
                  router_w=rw, router_bias=rb, t_gate=tg, t_up=tg, t_down=td, ts_gate=tsg, ts_up=tsg,
                  ts_down=tsd, gate=[None] * NR, up=[None] * NR, down=[None] * NR, **self.shared)
        for e in sorted(set(int(v) for v in experts)):
            if e not in self.cache:
                self.cache[e] = (fetch(self.dev, self.bufs["gate"], e * GB, GB),
                                 fetch(self.dev, self.bufs["up"], e * GB, GB),
                                 fetch(self.dev, self.bufs["down"], e * DB, DB))
            sp["gate"][e], sp["up"][e], sp["down"][e] = self.cache[e]
        return sp

    def close(self):
        for b in self.bufs.values():
            self.dev.free(b)


@pytest.fixture(scope="module")
def layer(dev):
    fl = FullLayer(dev)
    yield fl
    fl.close()


@pytest.fixture(scope="module")
def real_layer(dev):
    fl = FullLayer(dev, REAL_TYPES)
    yield fl
    fl.close()


def decode(dev, desc, x):
    xb = dev.shared_from(x)
    yb, rb = dev.alloc(H * 4), dev.alloc(64 * 4)
    dev.run(dev.L.sepia_gpu_moe_decode, ctypes.byref(desc), xb, yb, rb)
    y = dev.download(yb, H)
    idx = dev.download(rb, TOPK, dtype=np.int32)
    w = dev.download(rb, TOPK + NS, offset=TOPK * 4)
    for b in (xb, yb, rb):
        dev.free(b)
    return y, idx, w


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_c3_decode_full(dev, orc, layer, seed):
    """C3 at full size, plain router: selection against the oracle, y within
    1e-4 * ||y||_inf of the oracle's layer."""
    rng = np.random.default_rng(seed + 10)
    x = synth.normal_vector(rng, H)
    y, idx, w = decode(dev, layer.descs["plain"], x)
    rw, rb = layer.routers["plain"]
    logits = orc.linear_f32(rw, x)
    sp = layer.spec("plain", idx)
    chosen = check_route(orc, sp, logits, idx, w)
    y_ref, _, _, _ = orc.moe_layer(sp, x, force_idx=chosen, threads=THREADS)
    assert_close(y, y_ref, what="C3 seed %d" % seed, gate=False)


def test_c3_decode_ties(dev, orc, layer):
    """Exact ties inside one lane, across lanes and at the cut-off: the GPU's
    selection equals the oracle's exactly, in the oracle's order."""
    rng = np.random.default_rng(77)
    x = synth.normal_vector(rng, H)
    y, idx, w = decode(dev, layer.descs["ties"], x)
    rw, rb = layer.routers["ties"]
    logits = orc.linear_f32(rw, x)
    idx_ref, w_ref = orc.route_select(logits, rb, NR, NS, TOPK, 8.0, 1.0)
    want = [TIE_IN_LANE[0], TIE_IN_LANE[1], TIE_ACROSS[0], TIE_ACROSS[1], SINGLE, TIE_CUTOFF[0]]
    assert list(idx_ref) == want, "constructed ties did not rank as planned: %s" % list(idx_ref)
    assert list(idx) == want, "GPU selection %s, oracle %s" % (list(idx), want)
    assert np.allclose(w, w_ref, rtol=1e-5, atol=0)
    sp = layer.spec("ties", idx)
    y_ref, _, _, _ = orc.moe_layer(sp, x, threads=THREADS)
    assert_close(y, y_ref, what="C3 ties", gate=False)


@pytest.mark.parametrize("router,x_kind", [("plain", "bf16"), ("plain", "f32"), ("ties", "bf16")])
def test_c5_prefill_full(dev, orc, layer, router, x_kind):
    """C5 at full size: 512 tokens over all 256 routed experts on the default
    (int8) path. Every token's selection against the oracle; y of every token
    for the plain router -- so every unit of up to 32 (token, expert) pairs,
    the last partial unit of each expert included, is checked -- with x
    bf16-representable and full f32; y on 16 tokens
    for the router with constructed ties."""
    T = 512
    rng = np.random.default_rng({"plain": 55, "ties": 56}[router] + (7 if x_kind == "f32" else 0))
    X = rng.standard_normal((T, H)).astype(np.float32)
    if x_kind == "bf16":
        X = (X.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)
    n_sel = TOPK + NS
    xb = dev.shared_from(X)
    yb, rb = dev.alloc(X.nbytes), dev.alloc(T * (TOPK + n_sel) * 4)
    dev.run(dev.L.sepia_gpu_moe_prefill, ctypes.byref(layer.descs[router]), T, xb, yb, rb)
    Y = dev.download(yb, T * H).reshape(T, H)
    idx = dev.download(rb, T * TOPK, dtype=np.int32).reshape(T, TOPK)
    w = dev.download(rb, T * n_sel, offset=T * TOPK * 4).reshape(T, n_sel)
    for b in (xb, yb, rb):
        dev.free(b)
    rw, rb_h = layer.routers[router]
    sp0 = dict(n_routed=NR, n_shared=NS, topk=TOPK, route_scale=8.0, global_scale=1.0, router_bias=rb_h)
    chosen = [check_route(orc, sp0, orc.linear_f32(rw, X[t]), idx[t], w[t]) for t in range(T)]
    if router == "plain":
        # 3072 (token, expert) pairs over 256 experts: well over half of them take tokens
        assert len(set(idx.ravel().tolist())) >= 128
    check = list(range(T)) if router == "plain" else list(range(8)) + [int(t) for t in np.linspace(8, T - 1, 8)]
    sp = layer.spec(router, np.concatenate([idx[t] for t in check]))
    for n, t in enumerate(check):
        y_ref, _, _, _ = orc.moe_layer(sp, X[t], force_idx=chosen[t], threads=THREADS)
        assert_close(Y[t], y_ref, what="C5 %s %s token %d" % (router, x_kind, t), gate=False)
        if n % 128 == 127:
            print("C5 %s %s: %d tokens checked" % (router, x_kind, n + 1), flush=True)


@pytest.mark.parametrize("seed", [0, 1])
def test_c3_real_types_decode_full(dev, orc, real_layer, seed):
    """The C3 layer in the real checkpoint's formats at full size: selection
    against the oracle, y within 1e-4 * ||y||_inf of the oracle's layer."""
    rng = np.random.default_rng(seed + 20)
    x = synth.normal_vector(rng, H)
    y, idx, w = decode(dev, real_layer.descs["plain"], x)
    rw, rb = real_layer.routers["plain"]
    sp = real_layer.spec("plain", idx)
    chosen = check_route(orc, sp, orc.linear_f32(rw, x), idx, w)
    y_ref, _, _, _ = orc.moe_layer(sp, x, force_idx=chosen, threads=THREADS)
    assert_close(y, y_ref, what="C3 real types seed %d" % seed, gate=False)


@pytest.mark.timeout(600)
def test_c5_real_types_prefill_full(dev, orc, real_layer):
    """C5 in the real checkpoint's formats at full size on the f16 prefill
    kernels (the default path for these formats): 512 tokens over all 256
    routed experts, every token's selection and every token's y against the
    oracle, so every unit of up to 32 pairs is checked, the shared experts'
    16 units and each expert's last partial unit included."""
    T = 512
    rng = np.random.default_rng(57)
    X = rng.standard_normal((T, H)).astype(np.float32)
    X = (X.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)
    n_sel = TOPK + NS
    xb = dev.shared_from(X)
    yb, rb = dev.alloc(X.nbytes), dev.alloc(T * (TOPK + n_sel) * 4)
    with Launches(dev) as n:
        dev.run(dev.L.sepia_gpu_moe_prefill, ctypes.byref(real_layer.descs["plain"]), T, xb, yb, rb)
        assert n.count("sepia_ph_gateup") == 1 and n.count("sepia_ph_down") == 1
    Y = dev.download(yb, T * H).reshape(T, H)
    idx = dev.download(rb, T * TOPK, dtype=np.int32).reshape(T, TOPK)
    w = dev.download(rb, T * n_sel, offset=T * TOPK * 4).reshape(T, n_sel)
    for b in (xb, yb, rb):
        dev.free(b)
    rw, rb_h = real_layer.routers["plain"]
    sp0 = dict(n_routed=NR, n_shared=NS, topk=TOPK, route_scale=8.0, global_scale=1.0, router_bias=rb_h)
    chosen = [check_route(orc, sp0, orc.linear_f32(rw, X[t]), idx[t], w[t]) for t in range(T)]
    assert len(set(idx.ravel().tolist())) >= 128
    sp = real_layer.spec("plain", idx.ravel())
    for t in range(T):
        y_ref, _, _, _ = orc.moe_layer(sp, X[t], force_idx=chosen[t], threads=THREADS)
        assert_close(Y[t], y_ref, what="C5 real types token %d" % t, gate=False)
        if t % 128 == 127:
            print("C5 real types: %d tokens checked" % (t + 1), flush=True)


def test_decode_many_experts_em16(dev, orc):
    """More than 256 routed experts (route_pick with 16 register slots a lane,
    E = 5) on the matrix-core FFN launches."""
    from test_gpu_parity import make_layer, run_moe
    rng = np.random.default_rng(3000)
    desc, spec, bufs = make_layer(dev, rng, hidden=1024, inter=1024, n_routed=320, n_shared=1,
                                  tg=Q2_K, tu=Q2_K, td=Q3_K, ts=Q4_K)
    try:
        for rep in range(2):
            x = synth.normal_vector(rng, 1024)
            y, idx, w = run_moe(dev, desc, x)
            y_ref, logits, idx_ref, w_ref = orc.moe_layer(spec, x, threads=THREADS)
            chosen = check_route(orc, spec, logits, idx, w)
            if chosen != list(idx_ref):
                y_ref, _, _, _ = orc.moe_layer(spec, x, force_idx=chosen, threads=THREADS)
            assert_close(y, y_ref, what="320 experts rep %d" % rep, gate=False)
    finally:
        for b in bufs.values():
            dev.free(b)
