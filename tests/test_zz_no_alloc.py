"""sepia_hip_moe_decode_noalloc (every scratch byte in the library's fixed
device array) against sepia_gpu_moe_decode, through the C ABI: the same
selection, weights and y, bit for bit, on two calls in a row (the second on a
smaller layer), with the library's allocation count and growable scratch
unchanged across the calls; and a layer too large for the array rejected
before anything is queued, while the regular entry takes the same layer."""
import ctypes
import os

import numpy as np
import pytest

from sepia_amd import hip, synth
from test_gpu_parity import assert_close, check_route, make_layer

pytestmark = pytest.mark.gpu

THREADS = min(16, os.cpu_count() or 1)


@pytest.fixture(scope="module")
def dev():
    return hip.Device()


def decode(dev, fn, desc, x):
    xb = dev.shared_from(x)
    yb, rb = dev.alloc(x.nbytes), dev.alloc(64 * 4)
    dev.run(fn, ctypes.byref(desc), xb, yb, rb)
    y = dev.download(yb, x.size)
    route = dev.download(rb, desc.topk + desc.topk + desc.n_shared, dtype=np.uint32)
    for b in (xb, yb, rb):
        dev.free(b)
    return y, route


def noalloc_twice(dev, cases):
    """The allocation-free entry on each case in a row, with its inputs and
    outputs allocated beforehand; the library's allocations and scratch
    region must not change across the calls."""
    L = dev.L
    io = []
    for desc, _spec, _bufs, x in cases:
        io.append((dev.shared_from(x), dev.alloc(x.nbytes), dev.alloc(64 * 4)))
    n0, s0 = L.sepia_hip_alloc_count(), L.sepia_hip_scratch_bytes()
    for (desc, _spec, _bufs, _x), (xb, yb, rb) in zip(cases, io):
        dev.run(L.sepia_hip_moe_decode_noalloc, ctypes.byref(desc), xb, yb, rb)
    assert L.sepia_hip_alloc_count() == n0, "the allocation-free entry allocated"
    assert L.sepia_hip_scratch_bytes() == s0, "the allocation-free entry grew the library's scratch"
    got = []
    for (desc, _spec, _bufs, x), (xb, yb, rb) in zip(cases, io):
        got.append((dev.download(yb, x.size), dev.download(rb, desc.topk + desc.topk + desc.n_shared,
                                                            dtype=np.uint32)))
        for b in (xb, yb, rb):
            dev.free(b)
    return got


def test_noalloc_matches_decode(dev, orc):
    L = dev.L
    rng = np.random.default_rng(6060)
    cases = []
    for hidden, inter, nr, ts in ((6144, 3072, 16, 12), (2048, 1024, 8, 10)):
        desc, spec, bufs = make_layer(dev, rng, hidden=hidden, inter=inter, n_routed=nr, n_shared=2,
                                      tg=10, tu=10, td=11, ts=ts)
        cases.append((desc, spec, bufs, synth.normal_vector(rng, hidden)))
    # the allocation-free entry first (run alone in a fresh process, the
    # library's scratch region does not exist yet and must stay so), twice
    # in a row: the large layer, then the smaller one
    got = noalloc_twice(dev, cases)
    cases = [c + decode(dev, L.sepia_gpu_moe_decode, c[0], c[3]) for c in cases]
    # and again after the regular entry has run
    got2 = noalloc_twice(dev, [c[:4] for c in cases])
    for (y, route), (y2, route2) in zip(got, got2):
        assert np.array_equal(route, route2) and np.array_equal(y.view(np.uint32), y2.view(np.uint32))
    for (desc, spec, bufs, x, want_y, want_route), (y, route) in zip(cases, got):
        assert np.array_equal(route, want_route), (route, want_route)
        assert np.array_equal(y.view(np.uint32), want_y.view(np.uint32))
        tk = desc.topk
        idx = route[:tk].view(np.int32)
        w = route[tk:].view(np.float32)
        y_ref, logits, idx_ref, _ = orc.moe_layer(spec, x, threads=THREADS)
        chosen = check_route(orc, spec, logits, idx, w)
        if chosen != list(idx_ref):
            y_ref, _, _, _ = orc.moe_layer(spec, x, force_idx=chosen, threads=THREADS)
        assert_close(y, y_ref, what="noalloc hidden %d" % desc.hidden, gate=False)
    for c in cases:
        for b in c[2].values():
            dev.free(b)


def test_noalloc_rejects_oversized_layer(dev):
    """64 slots of hidden 8192 + inter 8448 need more than the 4 MiB array:
    refused (0) with nothing queued and nothing allocated; the batch itself
    stays usable, and the regular entry accepts the same layer (so the size
    is what was refused)."""
    L = dev.L
    H, I, NR, NS, TK = 8192, 8448, 62, 2, 62
    gb, db = synth.row_bytes(10, H) * I, synth.row_bytes(11, I) * H
    sgb, sdb = synth.row_bytes(12, H) * I, synth.row_bytes(12, I) * H
    bufs = dict(gate=dev.alloc(NR * gb, private=True), up=dev.alloc(NR * gb, private=True),
                down=dev.alloc(NR * db, private=True), s_gate=dev.alloc(NS * sgb, private=True),
                s_up=dev.alloc(NS * sgb, private=True), s_down=dev.alloc(NS * sdb, private=True),
                rw=dev.alloc((NR + NS) * H * 4, private=True), rb=dev.alloc(NR * 4, private=True),
                x=dev.alloc(H * 4, private=True), y=dev.alloc(H * 4, private=True))
    try:
        d = hip.MoeLayerDesc(hidden=H, inter=I, n_routed=NR, n_shared=NS, topk=TK, route_scale=8.0,
                             global_scale=1.0, router_w=bufs["rw"], router_bias=bufs["rb"])
        d.gate, d.up = hip.ExpertTensor(bufs["gate"], 0, gb, 10), hip.ExpertTensor(bufs["up"], 0, gb, 10)
        d.down = hip.ExpertTensor(bufs["down"], 0, db, 11)
        d.s_gate, d.s_up = hip.ExpertTensor(bufs["s_gate"], 0, sgb, 12), hip.ExpertTensor(bufs["s_up"], 0, sgb, 12)
        d.s_down = hip.ExpertTensor(bufs["s_down"], 0, sdb, 12)
        n0 = L.sepia_hip_alloc_count()
        dev.begin()
        try:
            assert L.sepia_hip_moe_decode_noalloc(ctypes.byref(d), bufs["x"], bufs["y"], None) == 0
        finally:
            assert L.sepia_gpu_end() == 1
        assert L.sepia_hip_alloc_count() == n0
        # all-zero weights, router and x: the regular entry runs the same layer
        dev.run(L.sepia_gpu_moe_decode, ctypes.byref(d), bufs["x"], bufs["y"], None)
    finally:
        for b in bufs.values():
            dev.free(b)
