"""Non-finite activations, through the C ABI.

The reference's qlinear sums (double)w * (double)x, so a NaN or an infinity
in x makes every output that depends on it non-finite (src/sepia.c:731-735,
:742-753); its selection with all-NaN router logits takes the lowest unused
index each round (strict '>' never prefers a NaN, src/sepia.c:1338-1346).
The library quantizes x per 16-column segment (decode) or per row
(prefill); a segment or row holding a NaN or an infinity gets an infinite
scale, so these outputs come out non-finite too, on every kernel path.
"""
import ctypes

import numpy as np
import pytest

from sepia_amd import hip, synth
from test_gpu_parity import gpu_matvec_q, make_layer, run_prefill

pytestmark = pytest.mark.gpu

TYPES = [10, 11, 12, 13, 14, 8, 17, 18, 23]
PATHS = {"mq": dict(mq=1, tile=1), "generic": dict(mq=0, tile=0), "tile": dict(mq=0, tile=1)}


@pytest.fixture(scope="module")
def dev():
    return hip.Device()


@pytest.fixture(params=list(PATHS))
def path(dev, request):
    for k, v in PATHS[request.param].items():
        assert dev.L.sepia_hip_set_option(k.encode(), v) == 1
    yield request.param
    for k in ("mq", "tile"):
        dev.L.sepia_hip_set_option(k.encode(), 1)


@pytest.mark.parametrize("bad", [np.nan, np.inf, -np.inf], ids=["nan", "inf", "-inf"])
@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("shape", [(64, 2048), (3072, 6144)], ids=str)
def test_matvec_nonfinite_x(dev, orc, path, t, shape, bad):
    out_dim, in_dim = shape
    if path == "tile" and t not in (10, 11, 12):
        pytest.skip("the tile kernels take Q2_K, Q3_K and Q4_K only")
    rng = np.random.default_rng(31 * t + out_dim)
    w = synth.random_matrix(t, out_dim, in_dim, rng)
    x = synth.normal_vector(rng, in_dim)
    x[in_dim // 2 + 5] = bad
    y = gpu_matvec_q(dev, t, w, out_dim, in_dim, x)
    want = orc.qlinear(t, w, out_dim, in_dim, x)
    assert not np.any(np.isfinite(want))          # the reference: every row non-finite
    assert not np.any(np.isfinite(y)), "%d of %d rows finite" % (int(np.isfinite(y).sum()), out_dim)


def test_matvec_nan_meets_zero_weights(dev, orc):
    """A NaN in x reaches every row (each row reads every column); with the
    NaN's weights all zero the reference still gives NaN (0 * NaN), so the
    library must not skip zero weights either."""
    t, out_dim, in_dim = 8, 32, 512
    rng = np.random.default_rng(5)
    w = synth.random_matrix(t, out_dim, in_dim, rng).reshape(out_dim, -1, 34)
    w[:, 3, 2:] = 0                                # block 3 (columns 96..127): all-zero codes
    w = w.reshape(-1)
    x = synth.normal_vector(rng, in_dim)
    x[100] = np.nan
    y = gpu_matvec_q(dev, t, w, out_dim, in_dim, x)
    want = orc.qlinear(t, w, out_dim, in_dim, x)
    assert np.all(np.isnan(want)) and np.all(np.isnan(y))


@pytest.mark.parametrize("types", [(10, 10, 11, 12), (17, 17, 18, 13)], ids=["q2k_q3k_q4k", "iq2xs_iq3xxs_q5k"])
def test_moe_decode_nan_x(dev, orc, types):
    """x with a NaN: the router logits are NaN, the selection is experts
    0..5 (the reference's arg-max over all-NaN scores), y is all NaN."""
    tg, tu, td, ts = types
    rng = np.random.default_rng(11)
    desc, spec, bufs = make_layer(dev, rng, hidden=2048, inter=1024, n_routed=16, n_shared=2,
                                  tg=tg, tu=tu, td=td, ts=ts)
    x = synth.normal_vector(rng, 2048)
    x[777] = np.nan
    xb, yb, rb = dev.shared_from(x), dev.alloc(2048 * 4), dev.alloc(256)
    dev.run(dev.L.sepia_gpu_moe_decode, ctypes.byref(desc), xb, yb, rb)
    y = dev.download(yb, 2048)
    idx = list(dev.download(rb, 6, dtype=np.int32))
    y_ref, _, idx_ref, _ = orc.moe_layer(spec, x)
    assert list(idx_ref) == [0, 1, 2, 3, 4, 5] and idx == list(idx_ref), idx
    assert np.all(np.isnan(y_ref)) and not np.any(np.isfinite(y))
    for b in list(bufs.values()) + [xb, yb, rb]:
        dev.free(b)


@pytest.mark.parametrize("kind", ["int8", "f16", "bf16"])
def test_moe_prefill_nonfinite_token(dev, orc, kind):
    """One token of the batch with an infinity: its output row is
    non-finite; every other token's row is bitwise what it is when that
    token is finite (each output element is its own dot product). int8: a
    Q2_K / Q3_K / Q4_K layer on the int8 kernels; f16: a layer of the real
    checkpoint's formats on the f16 kernels; bf16: the Q2_K layer on the bf16
    kernels."""
    rng = np.random.default_rng(12)
    types = dict(tg=17, tu=17, td=18, ts=13, tsd=14) if kind == "f16" else dict(tg=10, tu=10, td=11, ts=12)
    desc, spec, bufs = make_layer(dev, rng, hidden=2048, inter=1024, n_routed=16, n_shared=2, **types)
    X = rng.standard_normal((24, 2048)).astype(np.float32)
    assert dev.L.sepia_hip_set_option(b"pf_q", 0 if kind == "bf16" else 1) == 1
    try:
        y0, _, _ = run_prefill(dev, desc, X)
        Xb = X.copy()
        Xb[9, 1500] = np.inf
        y1, idx1, _ = run_prefill(dev, desc, Xb)
    finally:
        dev.L.sepia_hip_set_option(b"pf_q", 1)
    assert np.all(np.isfinite(y0))
    assert not np.any(np.isfinite(y1[9]))
    others = [t for t in range(24) if t != 9]
    assert np.array_equal(y1[others].view(np.uint32), y0[others].view(np.uint32))
    for b in bufs.values():
        dev.free(b)
