"""Attention ABI functions (rel_project, rel_project_off, banded_attn) through
the C ABI against the oracle's restatement of the reference's
attn_forward_chunk (src/sepia.c:1203-1247), at the model's two layer
geometries (docs/inkling-config.json: sliding H 64 / Hkv 16 / Dh 128 /
window = rel_extent 512; global H 64 / Hkv 8 / Dh 128 / rel_extent 1024;
d_rel 16), with kv ranges inside, at and past the band, several spans per
token, and batches of more than one launch of tokens. The reference's own
gate for these kernels (--gpu-compare-attn) runs in test_reference_host.py.
"""
import ctypes
import os

import numpy as np
import pytest

from sepia_amd import hip
from test_gpu_parity import assert_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    return hip.Device()


def rel_project(dev, r_vec, rel_proj, T, H, d_rel, R, off=0):
    rb = dev.shared_from(r_vec)
    pb = dev.alloc(rel_proj.nbytes + off)
    dev.upload(pb, rel_proj, offset=off)
    ob = dev.alloc(T * H * R * 4)
    if off:
        dev.run(dev.L.sepia_gpu_rel_project_off, rb, pb, off, ob, T, H, d_rel, R)
    else:
        dev.run(dev.L.sepia_gpu_rel_project, rb, pb, ob, T, H, d_rel, R)
    out = dev.download(ob, T * H * R)
    for b in (rb, pb, ob):
        dev.free(b)
    return out


@pytest.mark.parametrize("T,H,d_rel,R,off", [(1, 64, 16, 512, 0), (8, 64, 16, 1024, 0), (3, 64, 16, 1024, 4096),
                                             (70, 64, 16, 512, 8), (2, 5, 130, 300, 0)])
def test_rel_project(dev, orc, T, H, d_rel, R, off):
    rng = np.random.default_rng(T * 1000 + R)
    r_vec = rng.standard_normal(T * H * d_rel).astype(np.float32)
    rel_proj = (rng.standard_normal(d_rel * R) * 0.05).astype(np.float32)
    got = rel_project(dev, r_vec, rel_proj, T, H, d_rel, R, off)
    want = orc.rel_project(r_vec, rel_proj, T, H, d_rel, R)
    assert_close(got, want, what="rel_project T=%d R=%d" % (T, R))


def banded(dev, q, k, v, rl, lo, hi, tau, T, H, Hkv, Dh, R, qpb, kv_dim):
    bufs = [dev.shared_from(a) for a in (q, k, v, rl)]
    ob = dev.alloc(T * H * Dh * 4)
    lo_a = (ctypes.c_int64 * T)(*[int(a) for a in lo])
    hi_a = (ctypes.c_int64 * T)(*[int(a) for a in hi])
    tau_a = (ctypes.c_float * T)(*[float(a) for a in tau])
    dev.run(dev.L.sepia_gpu_banded_attn, bufs[0], bufs[1], bufs[2], bufs[3], ob,
            ctypes.cast(lo_a, ctypes.c_void_p), ctypes.cast(hi_a, ctypes.c_void_p),
            ctypes.cast(tau_a, ctypes.c_void_p), T, H, Hkv, Dh, R, qpb, kv_dim, 1.0 / Dh)
    out = dev.download(ob, T * H * Dh)
    for b in bufs + [ob]:
        dev.free(b)
    return out


# (label, sliding, q_pos of the last token, T): kv ranges inside / at / past the band,
# many spans, a batch spanning two launches of tokens
CASES = [("sliding_short", True, 100, 1), ("sliding_window", True, 511, 1), ("sliding_long", True, 3000, 4),
         ("global_short", False, 100, 1), ("global_band_edge", False, 1027, 8), ("global_long", False, 20000, 1),
         ("global_first_token", False, 0, 1), ("sliding_batch", True, 700, 70), ("global_batch", False, 130, 66)]


@pytest.mark.parametrize("label,sliding,q_last,T", CASES, ids=[c[0] for c in CASES])
def test_banded_attn(dev, orc, label, sliding, q_last, T):
    H, Dh, d_rel = 64, 128, 16
    Hkv, R, window = (16, 512, 512) if sliding else (8, 1024, None)
    kv_dim = Hkv * Dh
    rng = np.random.default_rng(len(label) * 31 + q_last)
    qpb = q_last - T + 1
    cap = q_last + 1
    q = (rng.standard_normal(T * H * Dh) * 0.3).astype(np.float32)
    k = (rng.standard_normal(cap * kv_dim) * 0.5).astype(np.float32)
    v = (rng.standard_normal(cap * kv_dim) * 0.5).astype(np.float32)
    rl = (rng.standard_normal(T * H * R) * 0.5).astype(np.float32)
    lo = [max(0, qpb + t - window + 1) if sliding else 0 for t in range(T)]
    hi = [qpb + t for t in range(T)]
    tau = [1.0 if sliding else 1.0 + 0.1 * np.log(max(1.0, (qpb + t + 1) / 128.0)) for t in range(T)]
    got = banded(dev, q, k, v, rl, lo, hi, tau, T, H, Hkv, Dh, R, qpb, kv_dim)
    want = orc.banded_attn(q, k, v, rl, lo, hi, np.array(tau, np.float32), T, H, Hkv, Dh, R, qpb, kv_dim, 1.0 / Dh)
    assert_close(got, want, what="banded_attn %s" % label)


def test_banded_attn_rejections(dev):
    """A kv range past the query position, a head dim over 128 and a ragged
    GQA group are refused with 0 (and a log line) before any launch."""
    L = dev.L
    T, H, Hkv, Dh, R = 1, 8, 2, 128, 16
    bufs = [dev.alloc(1 << 20) for _ in range(5)]
    lo = (ctypes.c_int64 * 1)(0)
    hi_bad = (ctypes.c_int64 * 1)(6)
    hi_ok = (ctypes.c_int64 * 1)(5)
    tau = (ctypes.c_float * 1)(1.0)
    c = lambda a: ctypes.cast(a, ctypes.c_void_p)
    dev.begin()
    try:
        assert L.sepia_gpu_banded_attn(*bufs, c(lo), c(hi_bad), c(tau), T, H, Hkv, Dh, R, 5, Hkv * Dh, 1 / Dh) == 0
        assert L.sepia_gpu_banded_attn(*bufs, c(lo), c(hi_ok), c(tau), T, H, Hkv, 256, R, 5, Hkv * 256, 1 / 256) == 0
        assert L.sepia_gpu_banded_attn(*bufs, c(lo), c(hi_ok), c(tau), T, H, 3, Dh, R, 5, 3 * Dh, 1 / Dh) == 0
    finally:
        assert L.sepia_gpu_end() == 1
        for b in bufs:
            dev.free(b)
