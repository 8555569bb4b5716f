"""The on-disk stores straight into HBM: resident.bin and a layer's experts
uploaded through the C ABI (store.c), read back byte for byte, and a MoE
layer assembled from the two stores (sepia_hip_moe_layer_from_stores) run
against the oracle on the same bytes. The fixtures are the reference's
formats (sepia_amd/store_synth.py; the smoke fixture is the one the
reference's own loader accepts, tests/test_store.py)."""
import ctypes
import json
import os

import numpy as np
import pytest

from sepia_amd import hip, store_synth
from test_gpu_parity import THREADS, Launches, assert_close, check_route

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    return hip.Device()


def fetch(dev, buf, off, nbytes):
    """Bytes [off, off + nbytes) of a private buffer (off, nbytes multiples of 4)."""
    pad = (nbytes + 3) // 4 * 4
    sb = dev.alloc(pad)
    dev.run(dev.L.sepia_gpu_copy, buf, off, sb, 0, pad // 4)
    out = dev.download(sb, pad, dtype=np.uint8)[:nbytes]
    dev.free(sb)
    return out.tobytes()


def load_stores(dev, paths, layer):
    L = dev.L
    t = L.sepia_hip_manifest_load(paths["manifest"].encode(), paths["bin"].encode())
    idx = L.sepia_hip_index_load(paths["index"].encode())
    assert t and idx
    rbuf = L.sepia_hip_manifest_upload(t)
    assert rbuf
    ex = (hip.ExpertTensor * 3)()
    ebuf = L.sepia_hip_index_upload_layer(idx, None, layer, ex)
    assert ebuf
    return t, idx, rbuf, ebuf, ex


def close_stores(dev, t, idx, *bufs):
    for b in bufs:
        dev.free(b)
    dev.L.sepia_hip_manifest_free(t)
    dev.L.sepia_hip_index_free(idx)


@pytest.fixture
def real_store(tmp_path):
    """Real-checkpoint formats at a matrix-core shape: IQ2_XS gate/up, IQ3_XXS
    down, Q5_K/Q6_K shared; 16 routed experts over two GGUF parts."""
    paths, host = store_synth.write_layer_store(str(tmp_path / "real"), np.random.default_rng(21), layer=5,
                                                hidden=2048, inter=1024, n_routed=16, n_shared=2,
                                                types=(17, 18, 13, 14), n_parts=2, extra_layers=(6,))
    return paths, host


@pytest.mark.parametrize("call", [0, 1])
def test_uploads_byte_exact(dev, real_store, call):
    """resident.bin (18.7 MB, not a whole number of pages) and the layer's
    runs (9.7 MB from byte 1152 of a part) take the split reads of a chunk
    by several threads; the second call reuses the staging buffers the
    first one left behind."""
    paths, host = real_store
    t, idx, rbuf, ebuf, ex = load_stores(dev, paths, 5)
    try:
        with open(paths["bin"], "rb") as f:
            blob = f.read()
        assert len(blob) > 4 << 20 and len(blob) % 4096
        assert fetch(dev, rbuf, 0, len(blob)) == blob
        h = host[5]
        for k, kind in enumerate(("gate", "up", "down")):
            assert ex[k].stride == h[kind][0].nbytes and ex[k].ggml_type == h["t_" + kind]
            got = fetch(dev, ebuf, ex[k].off, 16 * ex[k].stride)
            assert got == b"".join(m.tobytes() for m in h[kind]), kind
    finally:
        close_stores(dev, t, idx, rbuf, ebuf)


def test_upload_follows_the_index_order(dev, real_store):
    """Experts listed out of file order (runs broken, one slice from the
    other layer's tensor) land where the index puts them: slot e of the
    stack holds the bytes the index names for expert e."""
    paths, host = real_store
    with open(paths["index"]) as f:
        doc = json.load(f)
    g = doc["moe_layers"]["5"]["gate"]["experts"]
    g[3], g[9] = g[9], g[3]
    doc["moe_layers"]["5"]["up"]["experts"][0] = dict(doc["moe_layers"]["6"]["up"]["experts"][11])
    with open(paths["index"], "w") as f:
        json.dump(doc, f)
    t, idx, rbuf, ebuf, ex = load_stores(dev, paths, 5)
    try:
        h5, h6 = host[5], host[6]
        want_g = [m.tobytes() for m in h5["gate"]]
        want_g[3], want_g[9] = want_g[9], want_g[3]
        assert fetch(dev, ebuf, ex[0].off, 16 * ex[0].stride) == b"".join(want_g)
        want_u = [m.tobytes() for m in h5["up"]]
        want_u[0] = h6["up"][11].tobytes()
        assert fetch(dev, ebuf, ex[1].off, 16 * ex[1].stride) == b"".join(want_u)
    finally:
        close_stores(dev, t, idx, rbuf, ebuf)


def test_upload_rejects_truncated_part(dev, real_store):
    """Part 2 ends with layer 6's down tensor: cut short, layer 6 is refused
    before anything is allocated, while layer 5 (no slice in that tail)
    still loads."""
    paths, _ = real_store
    L = dev.L
    idx = L.sepia_hip_index_load(paths["index"].encode())
    part = os.path.join(os.path.dirname(paths["index"]), store_synth.GGUF_DIR, L.sepia_hip_index_part(idx, 1).decode())
    os.truncate(part, os.path.getsize(part) - 1000)
    ex = (hip.ExpertTensor * 3)()
    try:
        assert not L.sepia_hip_index_upload_layer(idx, None, 6, ex)
        assert not L.sepia_hip_index_upload_layer(idx, None, 4, ex)   # not in the index
        b = L.sepia_hip_index_upload_layer(idx, None, 5, ex)
        assert b
        dev.free(b)
    finally:
        L.sepia_hip_index_free(idx)


def spec_of(host, topk, route_scale, gscale):
    s = dict(host)
    s.update(topk=topk, route_scale=route_scale, global_scale=gscale)
    return s


@pytest.mark.parametrize("layer", [5, 6])
def test_moe_layer_from_stores(dev, orc, real_store, layer):
    """The descriptor from the two stores drives sepia_gpu_moe_decode on the
    matrix-core launches; y against the oracle on the same bytes, twice."""
    paths, host = real_store
    t, idx, rbuf, ebuf, ex = load_stores(dev, paths, layer)
    desc = hip.MoeLayerDesc()
    try:
        assert dev.L.sepia_hip_moe_layer_from_stores(t, rbuf, layer, ex, 16, 6, 8.0, ctypes.byref(desc)) == 1
        assert (desc.hidden, desc.inter, desc.n_routed, desc.n_shared, desc.topk) == (2048, 1024, 16, 2, 6)
        assert desc.global_scale == 1.0 and desc.s_down.ggml_type == 14 and desc.down.ggml_type == 18
        spec = spec_of(host[layer], 6, 8.0, 1.0)
        rng = np.random.default_rng(layer)
        for rep in range(2):
            x = rng.standard_normal(2048).astype(np.float32)
            xb, yb, rb = dev.shared_from(x), dev.alloc(2048 * 4), dev.alloc(64 * 4)
            with Launches(dev) as n:
                dev.run(dev.L.sepia_gpu_moe_decode, ctypes.byref(desc), xb, yb, rb)
                assert n.count("sepia_mq_gateup") == 1 and n.count("sepia_mq_down") == 1
            y = dev.download(yb, 2048)
            sel = dev.download(rb, 6, dtype=np.int32)
            w = dev.download(rb, 8, offset=24)
            for b in (xb, yb, rb):
                dev.free(b)
            y_ref, logits, idx_ref, _ = orc.moe_layer(spec, x, threads=THREADS)
            chosen = check_route(orc, spec, logits, sel, w)
            if chosen != list(idx_ref):
                y_ref, _, _, _ = orc.moe_layer(spec, x, force_idx=chosen, threads=THREADS)
            assert_close(y, y_ref, what="store layer %d rep %d" % (layer, rep), gate=False)
    finally:
        close_stores(dev, t, idx, rbuf, ebuf)


def test_layer_from_stores_rejects_bad_shapes(dev, real_store):
    paths, _ = real_store
    t, idx, rbuf, ebuf, ex = load_stores(dev, paths, 5)
    desc = hip.MoeLayerDesc()
    L = dev.L
    try:
        assert L.sepia_hip_moe_layer_from_stores(t, rbuf, 9, ex, 16, 6, 8.0, ctypes.byref(desc)) == 0   # no layer 9
        assert L.sepia_hip_moe_layer_from_stores(t, rbuf, 5, ex, 17, 6, 8.0, ctypes.byref(desc)) == 0   # n_routed
        bad = (hip.ExpertTensor * 3)(*ex)
        bad[2].stride -= 98
        assert L.sepia_hip_moe_layer_from_stores(t, rbuf, 5, bad, 16, 6, 8.0, ctypes.byref(desc)) == 0
    finally:
        close_stores(dev, t, idx, rbuf, ebuf)


def test_smoke_fixture_qlinear(dev, tmp_path):
    """The smoke fixture's resident Q8_0 tensor through sepia_gpu_matvec_q
    at its offset in the uploaded resident.bin: the expected y is exact."""
    info = store_synth.write_smoke_fixture(str(tmp_path / "smoke"))
    L = dev.L
    t = L.sepia_hip_manifest_load(info["manifest"].encode(), info["bin"].encode())
    rbuf = L.sepia_hip_manifest_upload(t)
    try:
        e = L.sepia_hip_manifest_find(t, b"blk.0.attn_r.weight").contents
        assert (e.ggml_type, e.shape[0], e.shape[1]) == (8, 32, 3)
        xb, yb = dev.shared_from(np.array(info["x"], np.float32)), dev.alloc(3 * 4)
        dev.run(L.sepia_gpu_matvec_q, 8, rbuf, e.offset, xb, yb, 3, 32)
        assert list(dev.download(yb, 3)) == info["y"]
        dev.free(xb)
        dev.free(yb)
    finally:
        dev.free(rbuf)
        L.sepia_hip_manifest_free(t)
