"""Pins the CPU oracle before anything is compared against it.

Every check here compares the oracle with something independent of it: the
reference's own golden fixtures, the reference's src/quants.c compiled into
oracle/_ref, a vectorised numpy decoder, closed forms, or brute force.
"""
import glob
import math
import os
import struct

import numpy as np
import pytest

import np_quants
from conftest import GOLDEN
from sepia_amd import synth

FIX = os.path.join(GOLDEN, "quants")


def read_sqfx(path):
    with open(path, "rb") as f:
        magic, ver, t, nb, be, bb = struct.unpack("<6I", f.read(24))
        assert magic == 0x58465153 and ver == 1
        raw = np.frombuffer(f.read(nb * bb), dtype=np.uint8)
        expect = np.frombuffer(f.read(nb * be * 4), dtype="<f4")
    return t, nb, be, bb, raw, expect


def read_sqlx(path):
    with open(path, "rb") as f:
        magic, ver, t, out_dim, in_dim = struct.unpack("<5I", f.read(20))
        assert magic == 0x584C5153 and ver == 1
        rb = {8: 34}[t] * (in_dim // 32)
        w = np.frombuffer(f.read(rb * out_dim), dtype=np.uint8)
        x = np.frombuffer(f.read(in_dim * 4), dtype="<f4")
        y = np.frombuffer(f.read(out_dim * 4), dtype="<f4")
    return t, out_dim, in_dim, w, x, y


SQFX = sorted(p for p in glob.glob(os.path.join(FIX, "*.bin")) if not os.path.basename(p).startswith("qlinear"))


def test_fixtures_present():
    names = sorted(os.path.basename(p) for p in SQFX)
    assert names == ["f16.bin", "iq2_xs.bin", "iq3_xxs.bin", "iq4_xs.bin",
                     "q4_k.bin", "q5_k.bin", "q6_k.bin", "q8_0.bin"]


@pytest.mark.parametrize("path", SQFX, ids=lambda p: os.path.basename(p))
def test_sqfx_bitwise(orc, path):
    """Reference golden fixtures (tools/fixtures/quants, written by gguf-py)."""
    t, nb, be, bb, raw, expect = read_sqfx(path)
    assert orc.GEOM[t] == (be, bb)
    got = orc.dequantize(t, raw, nb * be)
    assert np.array_equal(got.view(np.uint32), expect.view(np.uint32))


def test_sqlx_bitwise(orc):
    t, out_dim, in_dim, w, x, y = read_sqlx(os.path.join(FIX, "qlinear_q8_0.bin"))
    got = orc.qlinear(t, w, out_dim, in_dim, x)
    assert np.array_equal(got.view(np.uint32), y.view(np.uint32))


def test_f16_all_patterns(orc):
    """Every binary16 pattern: numpy's exact conversion for non-NaN values; NaNs keep
    sign and payload with no quieting (src/quants.c:71-72)."""
    bits = np.arange(65536, dtype=np.uint16)
    raw = bits.view(np.uint8)
    got = orc.dequantize(orc.F16, raw, 65536).view(np.uint32)
    ref = bits.view(np.float16).astype(np.float32).view(np.uint32)
    nan = ((bits >> 10) & 31 == 31) & (bits & 0x3FF != 0)
    assert np.array_equal(got[~nan], ref[~nan])
    nb = bits[nan].astype(np.uint32)
    assert np.array_equal(got[nan], ((nb >> 15) << 31) | 0x7F800000 | ((nb & 0x3FF) << 13))


needs_ref = pytest.mark.skipif(not os.path.exists(os.path.join(os.path.dirname(GOLDEN), "..", "oracle", "_ref",
                                                                "libref_quants.so")),
                               reason="reference quants.c not compiled here (oracle/_ref absent)")


@needs_ref
@pytest.mark.parametrize("t", [1, 8, 12, 13, 14, 17, 18, 23], ids=lambda t: "type%d" % t)
@pytest.mark.parametrize("mode", ["patched", "raw"])
def test_differential_vs_reference(orc, t, mode):
    """Fresh random blocks through the reference's own dequantize_row, bitwise.
    'raw' leaves the f16 scale fields random too (subnormal, inf and NaN scales)."""
    rng = np.random.default_rng(1000 + t + (7 if mode == "raw" else 0))
    be, bb = orc.GEOM[t]
    nb = 4096 if be > 1 else 1 << 16
    if mode == "patched":
        raw = synth.random_blocks(t, nb, rng)
    else:
        raw = rng.integers(0, 256, size=nb * bb, dtype=np.uint8)
    got = orc.dequantize(t, raw, nb * be)
    ref = orc.ref_dequantize(t, raw, nb * be)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("mode", ["patched", "raw"])
@pytest.mark.parametrize("t,fn", [(10, np_quants.q2_k), (11, np_quants.q3_k)], ids=["q2_k", "q3_k"])
def test_unpinned_kquants_vs_numpy(orc, t, fn, mode):
    """Q2_K/Q3_K are not in the reference: a second, vectorised decoder must agree bitwise."""
    rng = np.random.default_rng(77 + t)
    be, bb = orc.GEOM[t]
    nb = 4096
    raw = synth.random_blocks(t, nb, rng) if mode == "patched" else rng.integers(0, 256, nb * bb, dtype=np.uint8)
    got = orc.dequantize(t, raw, nb * be)
    with np.errstate(invalid="ignore", over="ignore"):
        exp = fn(raw)
    assert np.array_equal(got.view(np.uint32), exp.astype(np.float32).view(np.uint32))


def _f16b(v):
    return np.array([v], dtype=np.float16).view(np.uint8)


def test_q2_k_probe_blocks(orc):
    """Closed-form Q2_K blocks: one quant set at a time lands at weight 128h + 32s + l."""
    d, dmin = 2.0 ** -8, 2.0 ** -9
    for (h, s, l, v, sc, m) in [(0, 0, 0, 3, 5, 2), (0, 1, 17, 2, 15, 0), (1, 3, 31, 1, 1, 15), (1, 2, 8, 3, 9, 7)]:
        blk = np.zeros(84, dtype=np.uint8)
        blk[80:82] = _f16b(d)
        blk[82:84] = _f16b(dmin)
        g = 8 * h + 2 * s + (l >= 16)
        blk[g] = sc | (m << 4)
        blk[16 + 32 * h + l] = v << (2 * s)
        out = orc.dequantize(orc.Q2_K, blk, 256)
        w = 128 * h + 32 * s + l
        expect = np.zeros(256, dtype=np.float32)
        grp = slice(128 * h + 32 * s + 16 * (l >= 16), 128 * h + 32 * s + 16 * (l >= 16) + 16)
        expect[grp] = -(dmin * m)
        expect[w] = d * sc * v - dmin * m
        assert np.array_equal(out, expect), (h, s, l)


def test_q3_k_probe_blocks(orc):
    """Closed-form Q3_K blocks: high-mask bit 4h + s of byte l lifts weight 128h + 32s + l
    from q - 4 to q; the 6-bit scale j = 8h + 2s + l//16 is split over the nibble and the
    2-bit field of byte 8 + j % 4 at shift 2*(j // 4)."""
    d = 2.0 ** -7
    for (h, s, l, sc) in [(0, 0, 3, 33), (0, 3, 20, 63), (1, 0, 0, 0), (1, 2, 31, 45), (1, 3, 16, 17)]:
        j = 8 * h + 2 * s + (l >= 16)
        blk = np.zeros(110, dtype=np.uint8)
        blk[108:110] = _f16b(d)
        s12 = np.zeros(12, dtype=np.uint8)
        nib, top = sc & 15, sc >> 4
        if j < 8:
            s12[j] |= nib
        else:
            s12[j - 8] |= nib << 4
        s12[8 + j % 4] |= top << (2 * (j // 4))
        blk[96:108] = s12
        blk[l] = 1 << (4 * h + s)            # hmask: this weight keeps q, all others get -4
        blk[32 + 32 * h + l] = 2 << (2 * s)   # q2 = 2 for this weight
        out = orc.dequantize(orc.Q3_K, blk, 256)
        w = 128 * h + 32 * s + l
        dl = np.float32(d) * np.float32(sc - 32)
        grp0 = 128 * h + 32 * s + 16 * (l >= 16)
        # every other group has scale -32 (stored 0): q = -4 there
        assert out[w] == dl * 2
        others = np.delete(np.arange(grp0, grp0 + 16), w - grp0)
        assert np.all(out[others] == dl * -4)
        rest = np.setdiff1d(np.arange(256), np.arange(grp0, grp0 + 16))
        assert np.all(out[rest] == np.float32(d) * np.float32(-32) * -4)


def test_iq2_xxs_structure_with_stand_in_codebook(orc):
    """IQ2_XXS's real codebook is absent offline; with any stand-in table the oracle's
    decode must match the vectorised decoder (structure only; parity unpinned)."""
    rng = np.random.default_rng(5)
    levels = np.array([0x08, 0x19, 0x2B], dtype=np.uint64)
    grid = np.zeros(256, dtype=np.uint64)
    for k in range(8):
        grid |= levels[rng.integers(0, 3, 256)] << np.uint64(8 * k)
    orc.set_iq2xxs_grid(grid)
    try:
        raw = synth.random_blocks(16, 1024, rng)
        got = orc.dequantize(16, raw, 1024 * 256)
        exp = np_quants.iq2_xxs(raw, grid)
        assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))
    finally:
        orc.set_iq2xxs_grid(None)
    assert not orc.lib().orc_supported(16)


def test_unsupported_and_misaligned(orc):
    assert not orc.lib().orc_supported(2)
    assert orc.lib().orc_row_bytes(12, 300) == 0
    raw = np.zeros(144, dtype=np.uint8)
    out = np.zeros(256, dtype=np.float32)
    assert orc.lib().orc_dequantize_row(12, orc._ptr(raw), orc._ptr(out), 255) == 0


@pytest.mark.parametrize("t", [8, 10, 11, 12, 13, 14, 17, 18, 23])
def test_qlinear_sequential_double(orc, t):
    """y[o] = float32(sequential float64 sum of deq(W[o,i]) * x[i]) (src/sepia.c:731-753):
    numpy's cumsum is a sequential float64 accumulation; rows decoded independently."""
    rng = np.random.default_rng(t)
    be, bb = orc.GEOM[t]
    out_dim, in_dim = 7, 4 * 256
    w = synth.random_matrix(t, out_dim, in_dim, rng)
    x = synth.normal_vector(rng, in_dim)
    y = orc.qlinear(t, w, out_dim, in_dim, x)
    rb = in_dim // be * bb
    for o in range(out_dim):
        row = w[o * rb:(o + 1) * rb]
        deq = orc.ref_dequantize(t, row, in_dim) if (t in orc.REF_TYPES and orc.ref_lib()) else \
            (np_quants.q2_k(row) if t == 10 else np_quants.q3_k(row) if t == 11 else orc.dequantize(t, row, in_dim))
        exp = np.float32(np.cumsum(deq.astype(np.float64) * x.astype(np.float64))[-1])
        assert y[o].view(np.uint32) == exp.view(np.uint32), o
    y4 = orc.qlinear(t, w, out_dim, in_dim, x, threads=4)
    assert np.array_equal(y.view(np.uint32), y4.view(np.uint32))


def test_activations_closed_form(orc):
    L = orc.lib()
    for v in np.concatenate([np.linspace(-30, 30, 601), [0.0, -0.0, 1e-30, -1e-30, 80.0, -80.0]]):
        v32 = float(np.float32(v))
        s = 1.0 / (1.0 + math.exp(-v32))
        assert abs(L.orc_sigmoid(v32) - s) <= 3e-7 * max(s, 1e-30)
        assert abs(L.orc_silu(v32) - v32 * s) <= 3e-7 * max(abs(v32 * s), 1e-30)
        ls = -math.log1p(math.exp(-v32)) if v32 >= 0 else v32 - math.log1p(math.exp(v32))
        assert abs(L.orc_logsigmoid(v32) - ls) <= 3e-7 * max(abs(ls), 1e-30)


def _sig(z):
    return 1.0 / (1.0 + np.exp(-z.astype(np.float64)))


@pytest.mark.parametrize("seed", range(8))
def test_route_select_brute_force(orc, seed):
    """Selection = stable top-k of sigmoid(logit) + bias; weights = sigma(z_j) / sum sigma(z)
    * route_scale * global_scale over selected + shared-sink logits (exp(logsigmoid) = sigmoid,
    a closed form independent of the oracle's log-sum-exp route)."""
    rng = np.random.default_rng(seed)
    n_r, n_s, k = 256, 2, 6
    logits = rng.standard_normal(n_r + n_s).astype(np.float32) * 2
    bias = rng.uniform(-0.1, 0.1, n_r).astype(np.float32)
    rs, gs = 8.0, float(np.float32(rng.uniform(0.5, 1.5)))
    idx, w = orc.route_select(logits, bias, n_r, n_s, k, rs, gs)
    score = _sig(logits[:n_r]) + bias.astype(np.float64)
    order = np.argsort(-score, kind="stable")[:k]
    assert list(idx) == list(order)
    z = np.concatenate([logits[idx], logits[n_r:]])
    sg = _sig(z)
    exp_w = sg / sg.sum() * rs * gs
    assert np.allclose(w, exp_w, rtol=2e-6, atol=0)
    assert abs(w.astype(np.float64).sum() - rs * gs) <= 1e-5 * rs * gs


def test_route_bias_is_selection_only(orc):
    rng = np.random.default_rng(3)
    n_r, n_s, k = 64, 2, 6
    logits = rng.standard_normal(n_r + n_s).astype(np.float32)
    b0 = np.zeros(n_r, dtype=np.float32)
    idx0, w0 = orc.route_select(logits, b0, n_r, n_s, k, 8.0, 1.0)
    # a bias that keeps the same experts on top leaves the weights bit-identical
    b1 = b0.copy()
    b1[idx0] += 0.05
    idx1, w1 = orc.route_select(logits, b1, n_r, n_s, k, 8.0, 1.0)
    assert list(idx1) == list(idx0) and np.array_equal(w1, w0)
    # a bias that promotes another expert changes the selection, and the weights are
    # those of the raw logits of the new selection
    out = [i for i in range(n_r) if i not in idx0][0]
    b2 = b0.copy()
    b2[out] = 10.0
    idx2, w2 = orc.route_select(logits, b2, n_r, n_s, k, 8.0, 1.0)
    assert idx2[0] == out
    assert np.array_equal(w2, orc.route_weights(logits, n_r, n_s, idx2, 8.0, 1.0))


def test_route_ties_lowest_index(orc):
    logits = np.zeros(34, dtype=np.float32)
    idx, w = orc.route_select(logits, np.zeros(32, dtype=np.float32), 32, 2, 6, 8.0, 1.0)
    assert list(idx) == [0, 1, 2, 3, 4, 5]
    assert np.allclose(w, 1.0, rtol=1e-6)


def test_expert_ffn_is_composition(orc):
    rng = np.random.default_rng(11)
    H, I = 512, 256
    g = synth.random_matrix(10, I, H, rng)
    u = synth.random_matrix(10, I, H, rng)
    dn = synth.random_matrix(11, H, I, rng)
    x = synth.normal_vector(rng, H)
    y = orc.expert_ffn(10, g, 10, u, 11, dn, H, I, x)
    h = orc.silu_mul(orc.qlinear(10, g, I, H, x), orc.qlinear(10, u, I, H, x))
    assert np.array_equal(y, orc.qlinear(11, dn, H, I, h))


def _inkling_golden():
    return np.load(os.path.join(GOLDEN, "inkling_moe.npz"))


def test_route_select_vs_transformers_inkling(orc):
    """Selection set and mixing weights against the third-party InklingTopkRouter
    (float64), vectors written by tests/golden/make_inkling_moe.py."""
    d = _inkling_golden()
    nr, ns, k = d["router_b"].size, d["router_w"].shape[0] - d["router_b"].size, int(d["topk"])
    for t in range(d["x"].shape[0]):
        logits = orc.linear_f32(d["router_w"], d["x"][t])
        np.testing.assert_allclose(logits[:nr], d["logits"][t], rtol=0, atol=1e-6)
        idx, w = orc.route_select(logits, d["router_b"], nr, ns, k, float(d["route_scale"]), float(d["global_scale"]))
        order = np.argsort(idx)
        assert np.array_equal(np.asarray(idx)[order], d["idx"][t])
        np.testing.assert_allclose(np.asarray(w[:k])[order], d["w_routed"][t], rtol=2e-6)
        np.testing.assert_allclose(w[k:], d["gammas"][t], rtol=2e-6)


def test_moe_layer_vs_transformers_inkling(orc):
    """Whole-layer composition (routed weight after down, shared gamma before
    down, sum) against the third-party InklingMoE (float64), f32 weights."""
    d = _inkling_golden()
    nr, ns = d["router_b"].size, d["router_w"].shape[0] - d["router_b"].size
    H, I = d["x"].shape[1], d["gate"].shape[1]
    as_bytes = lambda a: [np.ascontiguousarray(m, dtype=np.float32).view(np.uint8).ravel() for m in a]
    spec = dict(hidden=H, inter=I, n_routed=nr, n_shared=ns, topk=int(d["topk"]),
                route_scale=float(d["route_scale"]), global_scale=float(d["global_scale"]),
                router_w=d["router_w"], router_bias=d["router_b"], t_gate=0, t_up=0, t_down=0,
                ts_gate=0, ts_up=0, ts_down=0, gate=as_bytes(d["gate"]), up=as_bytes(d["up"]),
                down=as_bytes(d["down"]), s_gate=as_bytes(d["s_gate"]), s_up=as_bytes(d["s_up"]),
                s_down=as_bytes(d["s_down"]))
    for t in range(d["x"].shape[0]):
        y, _, idx, _ = orc.moe_layer(spec, d["x"][t])
        assert np.array_equal(np.sort(idx), d["idx"][t])
        want = d["y"][t]
        assert np.max(np.abs(y - want)) <= 2e-6 * np.max(np.abs(want))


# ------------------------------------------------------------------ attention
def test_rel_project_is_a_matrix_product(orc):
    """rel_logits = r_vec @ rel_proj per (t, h) row: against numpy's float64 product."""
    rng = np.random.default_rng(11)
    T, H, d_rel, R = 3, 5, 16, 40
    rv = rng.standard_normal((T, H, d_rel)).astype(np.float32)
    rp = rng.standard_normal((d_rel, R)).astype(np.float32)
    got = orc.rel_project(rv, rp, T, H, d_rel, R).reshape(T, H, R)
    want = rv.reshape(T * H, d_rel).astype(np.float64) @ rp.astype(np.float64)
    assert np.allclose(got, want.reshape(T, H, R), rtol=1e-6, atol=1e-6)


def _attn_case(rng, T, H, Hkv, Dh, R, cap):
    q = rng.standard_normal((T, H, Dh)).astype(np.float32)
    k = rng.standard_normal((cap, Hkv, Dh)).astype(np.float32)
    v = rng.standard_normal((cap, Hkv, Dh)).astype(np.float32)
    rl = rng.standard_normal((T, H, R)).astype(np.float32)
    return q, k, v, rl


def test_banded_attn_single_key_returns_its_value(orc):
    """One kv position: the softmax weight is exactly 1, so the output is that v row."""
    rng = np.random.default_rng(12)
    T, H, Hkv, Dh, R = 2, 4, 2, 8, 6
    q, k, v, rl = _attn_case(rng, T, H, Hkv, Dh, R, 10)
    lo, hi = [3, 9], [3, 9]
    out = orc.banded_attn(q, k, v, rl, lo, hi, np.ones(T, np.float32), T, H, Hkv, Dh, R, 9, Hkv * Dh, 1 / Dh)
    out = out.reshape(T, H, Dh)
    for t, kv in enumerate(lo):
        for h in range(H):
            assert np.array_equal(out[t, h], v[kv, h // (H // Hkv)])


def test_banded_attn_equal_scores_average_v(orc):
    """Equal keys and a band bias of zero give equal weights: the output is the
    mean of the window's v rows (GQA: heads of a group read the same kv head)."""
    rng = np.random.default_rng(13)
    T, H, Hkv, Dh, R, cap = 1, 4, 2, 8, 4, 12
    q, k, v, rl = _attn_case(rng, T, H, Hkv, Dh, R, cap)
    k[:] = k[0]
    rl[:] = 0.0
    out = orc.banded_attn(q, k, v, rl, [2], [11], np.ones(1, np.float32), T, H, Hkv, Dh, R, 11, Hkv * Dh, 1 / Dh)
    out = out.reshape(H, Dh)
    for h in range(H):
        assert np.allclose(out[h], v[2:12, h // 2].astype(np.float64).mean(axis=0), rtol=1e-6, atol=1e-6)


def test_banded_attn_brute_force(orc):
    """Small cases against a float64 softmax written with numpy, covering the
    band cut-off (dist >= rel_extent gets no bias), tau on the bias only,
    sliding windows and GQA."""
    rng = np.random.default_rng(14)
    T, H, Hkv, Dh, R = 3, 6, 3, 8, 5
    qpb, cap = 7, 10
    q, k, v, rl = _attn_case(rng, T, H, Hkv, Dh, R, cap)
    lo, hi, tau = [0, 4, 2], [7, 8, 9], np.array([1.0, 1.3, 0.7], np.float32)
    got = orc.banded_attn(q, k, v, rl, lo, hi, tau, T, H, Hkv, Dh, R, qpb, Hkv * Dh, 1 / Dh).reshape(T, H, Dh)
    for t in range(T):
        q_pos = qpb + t
        for h in range(H):
            hk = h // (H // Hkv)
            kvs = np.arange(lo[t], hi[t] + 1)
            dist = q_pos - kvs
            bias = np.where(dist < R, rl[t, h, np.minimum(dist, R - 1)].astype(np.float64) * tau[t], 0.0)
            s = (k[kvs, hk].astype(np.float64) @ q[t, h].astype(np.float64)) / Dh + bias
            p = np.exp(s - s.max())
            want = (p / p.sum()) @ v[kvs, hk].astype(np.float64)
            assert np.allclose(got[t, h], want, rtol=1e-5, atol=1e-6), (t, h)


def test_banded_attn_rejects_kv_past_query(orc):
    rng = np.random.default_rng(15)
    q, k, v, rl = _attn_case(rng, 1, 2, 1, 4, 3, 6)
    with pytest.raises(ValueError):
        orc.banded_attn(q, k, v, rl, [0], [5], np.ones(1, np.float32), 1, 2, 1, 4, 3, 4, 4, 0.25)
