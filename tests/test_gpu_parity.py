"""GPU parity: libsepia_hip.so (through its C ABI) against the CPU oracle.

Bars:
  * dequantized weights bit-exact against the reference's dequantize_row;
  * matvec and MoE outputs within max|diff| <= 1e-4 * ||y||_inf of the oracle
    (which accumulates in float64), and the reference's own GPU gate
    (relative error with a 1e-3 * scale floor <= 2e-4, src/sepia.c:4557-4589).
"""
import ctypes
import glob
import os
import struct
import zlib

import numpy as np
import pytest

import np_quants
from conftest import GOLDEN
from sepia_amd import hip, synth

pytestmark = pytest.mark.gpu

THREADS = min(16, os.cpu_count() or 1)
TOL = 1e-4


@pytest.fixture(scope="module")
def dev():
    return hip.Device()


def assert_close(got, want, tol=TOL, what="", gate=True):
    """max|got - want| <= tol * ||want||_inf (BASELINE's bar) and, for single
    ops (gate=True), the reference's per-op GPU gate (src/sepia.c:4557-4589:
    |got - want| / max(|want|, 1e-3 * max|want|) <= 2e-4). Composite outputs
    (the expert FFN, the MoE layer, whose slots add into y with atomics in
    completion order) are held to BASELINE's bar only: the reference applies
    its gate per op kind, never to a whole layer."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert np.all(np.isfinite(got)), what
    scale = float(np.max(np.abs(want))) if want.size else 0.0
    err = float(np.max(np.abs(got - want))) if want.size else 0.0
    assert err <= tol * scale, "%s: max|diff| %.3e > %.1e * %.3e" % (what, err, tol, scale)
    if not gate:
        return
    floor = max(1e-6, 1e-3 * scale)
    rel = np.abs(got - want) / np.maximum(np.abs(want), floor)
    assert float(rel.max()) <= 2e-4, "%s: reference gate rel %.3e" % (what, float(rel.max()))


def gpu_dequant(dev, t, raw, n, raw_off=0):
    rb = dev.alloc(raw.nbytes + raw_off + 1)
    dev.upload(rb, raw, offset=raw_off)
    ob = dev.alloc(n * 4)
    dev.run(dev.L.sepia_gpu_dequant_rows, t, rb, raw_off, ob, n)
    out = dev.download(ob, n)
    dev.free(rb)
    dev.free(ob)
    return out


def gpu_matvec_q(dev, t, w, out_dim, in_dim, x, w_off=0):
    wb = dev.alloc(w.nbytes + w_off)
    dev.upload(wb, w, offset=w_off)
    xb = dev.shared_from(x)
    yb = dev.alloc(out_dim * 4)
    dev.run(dev.L.sepia_gpu_matvec_q, t, wb, w_off, xb, yb, out_dim, in_dim)
    y = dev.download(yb, out_dim)
    for b in (wb, xb, yb):
        dev.free(b)
    return y


def test_device(dev):
    assert dev.L.sepia_gpu_available() == 1
    assert dev.name
    print("device:", dev.name)


# --------------------------------------------------------------- dequant
SQFX = sorted(p for p in glob.glob(os.path.join(GOLDEN, "quants", "*.bin"))
              if not os.path.basename(p).startswith("qlinear"))


@pytest.mark.parametrize("path", SQFX, ids=lambda p: os.path.basename(p))
def test_dequant_golden_bitwise(dev, path):
    """The reference's --gpu-quants gate (src/sepia.c:5944-6004) on its own fixtures."""
    with open(path, "rb") as f:
        magic, ver, t, nb, be, bb = struct.unpack("<6I", f.read(24))
        raw = np.frombuffer(f.read(nb * bb), dtype=np.uint8)
        expect = np.frombuffer(f.read(nb * be * 4), dtype="<f4")
    got = gpu_dequant(dev, t, raw, nb * be)
    assert np.array_equal(got.view(np.uint32), expect.view(np.uint32))


ALL_Q = [8, 10, 11, 12, 13, 14, 17, 18, 23]


@pytest.fixture(scope="module")
def stand_in_iq2xxs(dev, orc):
    """IQ2_XXS's codebook is unavailable offline: a seeded stand-in table (magnitudes
    from the format's 3 levels) exercises the decode structure on both sides."""
    rng = np.random.default_rng(2024)
    levels = np.array([0x08, 0x19, 0x2B], dtype=np.uint64)
    grid = np.zeros(256, dtype=np.uint64)
    for k in range(8):
        grid |= levels[rng.integers(0, 3, 256)] << np.uint64(8 * k)
    g = np.ascontiguousarray(grid)
    assert dev.L.sepia_hip_set_iq2xxs_grid(g.ctypes.data) == 1
    orc.set_iq2xxs_grid(grid)
    yield grid
    orc.set_iq2xxs_grid(None)


@pytest.mark.parametrize("t", ALL_Q + [16])
@pytest.mark.parametrize("raw_off", [0, 2, 3])
def test_dequant_random_bitwise(dev, orc, stand_in_iq2xxs, t, raw_off):
    rng = np.random.default_rng(100 * t + raw_off)
    be, bb = orc.GEOM[t]
    nb = 1024 if be == 256 else 4096
    raw = synth.random_blocks(t, nb, rng)
    got = gpu_dequant(dev, t, raw, nb * be, raw_off)
    want = orc.dequantize(t, raw, nb * be)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    if t == 16:
        assert np.array_equal(want.view(np.uint32), np_quants.iq2_xxs(raw, stand_in_iq2xxs).view(np.uint32))


@pytest.mark.parametrize("t", ALL_Q)
def test_dequant_raw_bytes(dev, orc, t):
    """Fully random blocks: subnormal/inf/NaN scale fields. Finite results are
    bit-exact; NaN positions agree."""
    rng = np.random.default_rng(7 * t)
    be, bb = orc.GEOM[t]
    nb = 512
    raw = rng.integers(0, 256, nb * bb, dtype=np.uint8)
    got = gpu_dequant(dev, t, raw, nb * be)
    want = orc.dequantize(t, raw, nb * be)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_dequant_f16_all_patterns(dev, orc):
    bits = np.arange(65536, dtype=np.uint16).view(np.uint8)
    got = gpu_dequant(dev, 1, bits, 65536)
    want = orc.dequantize(1, bits, 65536)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# ---------------------------------------------------------------- matvec
def check_matvec(dev, orc, t, out_dim, in_dim, seed, w_off=0):
    rng = np.random.default_rng(seed)
    w = synth.random_matrix(t, out_dim, in_dim, rng)
    x = synth.normal_vector(rng, in_dim)
    y = gpu_matvec_q(dev, t, w, out_dim, in_dim, x, w_off)
    want = orc.qlinear(t, w, out_dim, in_dim, x, threads=THREADS)
    assert_close(y, want, what="type %d %dx%d off %d" % (t, out_dim, in_dim, w_off))


@pytest.mark.parametrize("t", ALL_Q + [16])
@pytest.mark.parametrize("shape", [(1, 256), (5, 512), (64, 2048), (257, 3072)], ids=str)
def test_matvec_q_small(dev, orc, stand_in_iq2xxs, t, shape):
    out_dim, in_dim = shape
    check_matvec(dev, orc, t, out_dim, in_dim, seed=t * 1000 + out_dim)


@pytest.mark.parametrize("t", [11, 12, 17])
@pytest.mark.parametrize("w_off", [2, 6, 130])
def test_matvec_q_weight_offset(dev, orc, t, w_off):
    check_matvec(dev, orc, t, 33, 1024, seed=99 + w_off, w_off=w_off)


def test_matvec_q_reference_fixture_gate(dev, orc):
    """The reference's gate reshapes each SQFX fixture into a 4-row matrix with
    x from rand_r; here x is seeded uniform [-1, 1) (src/sepia.c:6006-6043)."""
    for path in SQFX:
        with open(path, "rb") as f:
            magic, ver, t, nb, be, bb = struct.unpack("<6I", f.read(24))
            raw = np.frombuffer(f.read(nb * bb), dtype=np.uint8)
        if t == 1:
            continue
        out_dim = 4
        in_dim = nb // out_dim * be
        x = np.random.default_rng(20260720 ^ t).uniform(-1, 1, in_dim).astype(np.float32)
        y = gpu_matvec_q(dev, t, raw, out_dim, in_dim, x)
        assert_close(y, orc.qlinear(t, raw, out_dim, in_dim, x), what=os.path.basename(path))


CONFIG_SHAPES = [
    ("C1 q4_k 4096x4096", 12, 4096, 4096),
    ("C2 gate q2_k 3072x6144", 10, 3072, 6144),
    ("C2 down q3_k 6144x3072", 11, 6144, 3072),
    ("C3 shared q4_k 3072x6144", 12, 3072, 6144),
    ("C4 iq3_xxs 6144x6144", 18, 6144, 6144),
    ("C4 sub iq2_xs 6144x6144", 17, 6144, 6144),
    ("real gate iq2_xs 3072x6144", 17, 3072, 6144),
    ("real down iq4_xs 6144x3072", 23, 6144, 3072),
    ("real shared q5_k 3072x6144", 13, 3072, 6144),
    ("real shared q6_k 6144x3072", 14, 6144, 3072),
]


@pytest.mark.parametrize("name,t,out_dim,in_dim", CONFIG_SHAPES, ids=[c[0] for c in CONFIG_SHAPES])
def test_matvec_q_config_shapes(dev, orc, name, t, out_dim, in_dim):
    check_matvec(dev, orc, t, out_dim, in_dim, seed=zlib.crc32(name.encode()) & 0xFFFF)


@pytest.fixture
def kernel_path(dev, request):
    """Force one kernel family: the matrix-core kernels (the default), the
    generic per-row kernel, or the tile kernels with 1, 2 or 3 row steps per
    workgroup."""
    L = dev.L
    mode = request.param
    if mode != "mq":
        assert L.sepia_hip_set_option(b"mq", 0) == 1
    if mode == "generic":
        assert L.sepia_hip_set_option(b"tile", 0) == 1
    elif mode != "mq":
        assert L.sepia_hip_set_option(b"tile_t", {"t1": 1, "t2": 2, "t3": 3}[mode]) == 1
    yield mode
    L.sepia_hip_set_option(b"mq", 1)
    L.sepia_hip_set_option(b"tile", 1)
    L.sepia_hip_set_option(b"tile_t", 0)


TILE_SHAPES = [(10, 3072, 6144), (11, 6144, 3072), (12, 4096, 4096), (12, 33, 1024), (10, 17, 2048),
               (11, 1, 3072), (12, 200, 6144), (10, 50, 8192), (12, 40, 12288), (11, 70, 12288)]


@pytest.mark.parametrize("kernel_path", ["mq", "generic", "t1", "t2", "t3"], indirect=True)
@pytest.mark.parametrize("t,out_dim,in_dim", TILE_SHAPES, ids=lambda v: str(v))
def test_matvec_q_kernel_paths(dev, orc, kernel_path, t, out_dim, in_dim):
    check_matvec(dev, orc, t, out_dim, in_dim, seed=out_dim * 7 + t)


class Launches:
    """Counts, per kernel name, the launches of the dev.run calls made inside
    the block (the library's launch profiler, sepia_hip_profile_*)."""

    def __init__(self, dev):
        self.dev = dev

    def __enter__(self):
        dev, L = self.dev, self.dev.L
        self.orig = dev.run
        L.sepia_hip_profile_reset()

        def run(fn, *args):
            dev.begin()
            try:
                assert L.sepia_hip_profile_start() == 1
                ok = fn(*args)
                assert L.sepia_hip_profile_stop() == 1
            finally:
                end_ok = L.sepia_gpu_end()
            dev.check(ok, fn.__name__)
            dev.check(end_ok, "end")

        dev.run = run
        return self

    def __exit__(self, *exc):
        self.dev.run = self.orig

    def count(self, kernel):
        import ctypes
        n, ms = ctypes.c_int64(), ctypes.c_double()
        assert self.dev.L.sepia_hip_profile_query(kernel.encode(), ctypes.byref(n), ctypes.byref(ms)) == 1
        return n.value


@pytest.fixture
def mq_geometry(dev, request):
    """Force the matrix-core workgroup geometry: P parts per item, C items side
    by side, S ring stages per wave."""
    L = dev.L
    for k, v in zip(("mq_p", "mq_c", "mq_s"), request.param):
        assert L.sepia_hip_set_option(k.encode(), v) == 1
    yield request.param
    for k in ("mq_p", "mq_c", "mq_s"):
        L.sepia_hip_set_option(k.encode(), 0)


MQ_NAMES = {10: "sepia_mq_mv_q2_k", 11: "sepia_mq_mv_q3_k", 12: "sepia_mq_mv_q4_k", 17: "sepia_mq_mv_iq2_xs",
            18: "sepia_mq_mv_iq3_xxs", 13: "sepia_mq_mv_q5_k", 14: "sepia_mq_mv_q6_k", 23: "sepia_mq_mv_iq4_xs",
            8: "sepia_mq_mv_q8_0"}
# (type, rows, cols, (P, C, S)): several items per workgroup (12288 and 8200
# rows), long rows (12288 columns: 12 quads), partial row groups, every ring
# depth, parts that do not divide the quads.
MQ_GEOMETRIES = [
    (10, 12288, 2048, (1, 1, 1)), (10, 12288, 2048, (1, 1, 3)), (10, 12288, 2048, (2, 1, 2)),
    (10, 12288, 2048, (1, 3, 2)), (10, 12288, 2048, (2, 2, 3)),
    (11, 70, 12288, (1, 1, 3)), (11, 70, 12288, (5, 1, 2)), (11, 70, 12288, (3, 1, 1)),
    (12, 8200, 4096, (1, 1, 2)), (12, 8200, 4096, (4, 3, 1)), (12, 8200, 4096, (3, 2, 2)),
    (17, 12288, 2048, (1, 2, 2)), (17, 70, 12288, (3, 1, 3)), (17, 6144, 6144, (2, 2, 1)),
    (18, 12288, 2048, (2, 1, 2)), (18, 70, 12288, (4, 1, 2)), (18, 6144, 6144, (1, 2, 3)),
    (13, 12288, 2048, (1, 1, 2)), (13, 70, 12288, (3, 1, 2)), (13, 3072, 6144, (2, 1, 1)),
    (14, 12288, 2048, (2, 1, 1)), (14, 70, 12288, (5, 1, 1)), (14, 6144, 3072, (1, 2, 2)),
    (23, 12288, 2048, (1, 2, 2)), (23, 70, 12288, (3, 1, 3)), (23, 6144, 3072, (2, 1, 2)),
    (8, 12288, 2048, (1, 1, 1)), (8, 70, 12288, (4, 1, 1)), (8, 3072, 6144, (2, 1, 1)),
]


@pytest.mark.parametrize("t,out_dim,in_dim,mq_geometry", MQ_GEOMETRIES, indirect=["mq_geometry"],
                         ids=lambda v: str(v))
def test_matvec_mq_geometries(dev, orc, t, out_dim, in_dim, mq_geometry):
    with Launches(dev) as n:
        check_matvec(dev, orc, t, out_dim, in_dim, seed=out_dim + in_dim + t)
        assert n.count(MQ_NAMES[t]) == 1, "the matrix-core kernel did not run"


@pytest.mark.parametrize("t,w_off", [(10, 4), (10, 132), (12, 4), (12, 1028), (11, 2), (11, 4)])
def test_matvec_q_tile_offsets(dev, orc, t, w_off):
    check_matvec(dev, orc, t, 100, 2048, seed=3 + w_off, w_off=w_off)


@pytest.mark.parametrize("t", [13, 14, 23, 8])
@pytest.mark.parametrize("w_off", [4, 132, 2])
def test_matvec_mq_offsets_new_formats(dev, orc, t, w_off):
    """Q5_K, Q6_K, IQ4_XS and Q8_0 weights 4-byte aligned at an offset into
    their buffer take the matrix-core kernel (the launch count shows it); at
    a 2-byte offset another kernel, with the same result bar. 33 rows leave a
    partial row group; the last row's last block ends at the buffer's end."""
    with Launches(dev) as n:
        check_matvec(dev, orc, t, 33, 2048, seed=41 + w_off + t, w_off=w_off)
        assert n.count(MQ_NAMES[t]) == (0 if w_off % 4 else 1)


def test_matvec_q_repeat_stable(dev, orc):
    """Back-to-back calls reuse the arrival counters: results stay identical."""
    rng = np.random.default_rng(8)
    t, out_dim, in_dim = 10, 3072, 6144
    w = synth.random_matrix(t, out_dim, in_dim, rng)
    x = synth.normal_vector(rng, in_dim)
    wb, xb, yb = dev.shared_from(w), dev.shared_from(x), dev.alloc(out_dim * 4)
    outs = []
    for _ in range(3):
        dev.begin()
        for _ in range(5):
            assert dev.L.sepia_gpu_matvec_q(t, wb, 0, xb, yb, out_dim, in_dim) == 1
        dev.end()
        outs.append(dev.download(yb, out_dim))
    assert all(np.array_equal(o.view(np.uint32), outs[0].view(np.uint32)) for o in outs)
    assert_close(outs[0], orc.qlinear(t, w, out_dim, in_dim, x, threads=THREADS))
    for b in (wb, xb, yb):
        dev.free(b)


def test_read_probe(dev):
    """The measurement probe reads whole 16-byte words of a buffer and leaves
    it unchanged; misaligned or out-of-range requests are refused."""
    L = dev.L
    data = np.arange(1 << 18, dtype=np.uint32)
    b = dev.shared_from(data)
    dev.begin()
    try:
        assert L.sepia_hip_read_probe(b, 0, data.nbytes, 1024) == 1
        assert L.sepia_hip_read_probe(b, 4096, 65536, 7) == 1
        assert L.sepia_hip_read_probe(b, 8, 4096, 4) == 0             # offset not a multiple of 16
        assert L.sepia_hip_read_probe(b, 0, 4100, 4) == 0             # size not a multiple of 16
        assert L.sepia_hip_read_probe(b, 16, data.nbytes, 4) == 0     # past the end
        assert L.sepia_hip_read_probe(b, 0, 4096, 0) == 0             # no workgroups
        # through LDS-DMA rings: every allowed shape, chunks that do not
        # fill their last step, more workgroups than steps
        for kb, st, thr in ((7, 1, 1024), (7, 2, 512), (4, 1, 1024), (4, 2, 1024), (4, 4, 512), (2, 4, 1024),
                            (1, 4, 1024)):
            assert L.sepia_hip_read_probe_dma(b, 0, data.nbytes, 256, thr, kb, st) == 1
            assert L.sepia_hip_read_probe_dma(b, 4096, 65536 + 48, 7, thr, kb, st) == 1
            assert L.sepia_hip_read_probe_dma(b, 0, 4096, 64, thr, kb, st) == 1
        assert L.sepia_hip_read_probe_dma(b, 0, 4096, 4, 1024, 7, 2) == 0   # rings beyond the LDS
        assert L.sepia_hip_read_probe_dma(b, 0, 4096, 4, 256, 3, 1) == 0    # no such shape
        assert L.sepia_hip_read_probe_dma(b, 0, 4096, 4, 100, 4, 1) == 0    # not whole waves
        assert L.sepia_hip_read_probe_dma(b, 16, data.nbytes, 4, 256, 4, 1) == 0   # past the end
    finally:
        assert L.sepia_gpu_end() == 1
    assert np.array_equal(dev.download(b, data.size, dtype=np.uint32), data)
    dev.free(b)


def test_matvec_q_rejections(dev):
    L = dev.L
    w = dev.alloc(144 * 4)
    x = dev.alloc(256 * 4)
    y = dev.alloc(16)
    assert L.sepia_gpu_matvec_q(12, w, 0, x, y, 4, 256) == 0          # no batch
    dev.begin()
    try:
        assert L.sepia_gpu_matvec_q(2, w, 0, x, y, 4, 256) == 0       # Q4_0: unsupported
        assert L.sepia_gpu_matvec_q(12, w, 0, x, y, 4, 255) == 0      # ragged in_dim
        assert L.sepia_gpu_matvec_q(12, w, 2, x, y, 4, 256) == 0      # past the end of w
        assert L.sepia_gpu_matvec_q(12, w, 0, x, y, 5, 256) == 0      # y too small / w too small
        assert L.sepia_gpu_matvec_q(12, w, 0, x, y, 0, 256) == 0
        assert L.sepia_gpu_dequant_rows(12, w, 0, x, 300) == 0
        assert L.sepia_gpu_matvec_q(12, w, 0, x, y, 4, 256) == 1
    finally:
        assert L.sepia_gpu_end() == 1
    assert L.sepia_gpu_begin() == 1
    assert L.sepia_gpu_begin() == 0                                    # already open
    assert L.sepia_gpu_flush() == 1
    assert L.sepia_gpu_end() == 1
    assert L.sepia_gpu_end() == 0
    for b in (w, x, y):
        dev.free(b)


# ---------------------------------------------------------------- f32 ops
def test_f32_ops(dev, orc):
    L = dev.L
    rng = np.random.default_rng(5)
    n, rows, out_dim = 1000, 3, 77
    a = rng.standard_normal(rows * n).astype(np.float32)
    b = rng.standard_normal(rows * n).astype(np.float32)
    wv = rng.standard_normal(n).astype(np.float32)
    W = rng.standard_normal((out_dim, n)).astype(np.float32)
    ba, bbuf, bw, bW = dev.shared_from(a), dev.shared_from(b), dev.shared_from(wv), dev.shared_from(W, extra=64)
    out = dev.alloc(rows * n * 4)

    dev.run(L.sepia_gpu_silu_mul, ba, bbuf, out, rows * n)
    z = dev.download(out, rows * n)
    assert np.allclose(z, orc.silu_mul(a, b), rtol=2e-6, atol=1e-7)

    dev.run(L.sepia_gpu_add, ba, bbuf, out, rows * n)
    assert np.array_equal(dev.download(out, rows * n), a + b)

    dev.run(L.sepia_gpu_scale, float(np.float32(0.37)), ba, out, rows * n)
    assert np.array_equal(dev.download(out, rows * n), a * np.float32(0.37))

    dev.run(L.sepia_gpu_copy, ba, 8, out, 4, n)
    assert np.array_equal(dev.download(out, n, offset=4), a[2:2 + n])

    dev.run(L.sepia_gpu_matvec, bW, ba, out, out_dim, n)
    assert_close(dev.download(out, out_dim), orc.linear_f32(W, a[:n]), what="matvec f32")
    # matvec_off at a 4-byte (not 16-byte) offset: the scalar-load path
    flat = rng.standard_normal(out_dim * n + 1).astype(np.float32)
    bflat = dev.shared_from(flat)
    dev.run(L.sepia_gpu_matvec_off, bflat, 4, ba, out, out_dim, n)
    assert_close(dev.download(out, out_dim), orc.linear_f32(flat[1:].reshape(out_dim, n), a[:n]),
                 what="matvec_off")
    dev.free(bflat)

    dev.run(L.sepia_gpu_rmsnorm, bw, ba, out, rows, n, 1e-6)
    x2 = a.reshape(rows, n).astype(np.float64)
    ref = wv * (x2 / np.sqrt((x2 ** 2).mean(axis=1, keepdims=True) + 1e-6))
    assert np.allclose(dev.download(out, rows * n).reshape(rows, n), ref, rtol=1e-5, atol=1e-6)

    dev.run(L.sepia_gpu_softmax, ba, out, rows, n)
    e = np.exp(x2 - x2.max(axis=1, keepdims=True))
    assert np.allclose(dev.download(out, rows * n).reshape(rows, n), e / e.sum(axis=1, keepdims=True),
                       rtol=1e-5, atol=1e-9)
    for buf in (ba, bbuf, bw, bW, out):
        dev.free(buf)


def test_sconv_and_hist_roll(dev):
    L = dev.L
    rng = np.random.default_rng(9)
    C, K = 40, 4
    for T in (1, 2, 3, 7):
        w = rng.standard_normal((C, K)).astype(np.float32)
        hist = rng.standard_normal((K - 1, C)).astype(np.float32)
        inp = rng.standard_normal((T, C)).astype(np.float32)
        bw, bh, bi, bo = dev.shared_from(w), dev.shared_from(hist), dev.shared_from(inp), dev.alloc(T * C * 4)
        dev.run(L.sepia_gpu_sconv, bw, bh, bi, bo, C, K, T)
        win = np.concatenate([hist, inp]).astype(np.float64)
        ref = inp + np.stack([(w * win[t:t + K].T).sum(axis=1) for t in range(T)])
        assert np.allclose(dev.download(bo, T * C).reshape(T, C), ref, rtol=1e-5, atol=1e-5)
        dev.run(L.sepia_gpu_sconv_hist_roll, bh, bi, C, K, T)
        assert np.array_equal(dev.download(bh, (K - 1) * C).reshape(K - 1, C),
                              np.concatenate([hist, inp])[-(K - 1):])
        for b in (bw, bh, bi, bo):
            dev.free(b)


def test_selftest_touch_and_wrap(dev):
    import mmap
    L = dev.L
    m = mmap.mmap(-1, 8192)
    arr = np.frombuffer(m, dtype=np.float32)
    arr[:] = np.arange(2048, dtype=np.float32)
    import ctypes
    addr = ctypes.addressof(ctypes.c_char.from_buffer(m))
    wb = L.sepia_gpu_wrap_mmap(addr, 8192)
    assert wb
    assert L.sepia_gpu_host_ptr(wb) == addr
    assert L.sepia_gpu_wrap_mmap(addr + 4, 100) is None          # not page-aligned
    out = dev.alloc(8192)
    dev.run(L.sepia_gpu_copy, wb, 0, out, 0, 2048)
    assert np.array_equal(dev.download(out, 2048), np.arange(2048, dtype=np.float32))
    assert L.sepia_gpu_selftest_touch(out, 2048) == 1
    assert np.array_equal(dev.download(out, 2048), np.arange(2048, dtype=np.float32))
    dev.free(out)
    dev.free(wb)
    del arr
    m.close()


def test_shared_slab_uploaded_once(dev, orc):
    """Shared-buffer synchronisation: a slab the host fills once through
    host_ptr is uploaded once however many batches read it; an op uploads only
    the range it reads (here whole 64 KiB chunks: an expert is 9 of them); a
    later host_ptr re-arms the slab and the next op sees the host's new
    bytes."""
    L = dev.L
    t, rows, cols, n_exp, C = 12, 256, 4096, 16, 1 << 16
    mb = rows * synth.row_bytes(t, cols)
    rng = np.random.default_rng(808)
    mats = [synth.random_matrix(t, rows, cols, rng) for _ in range(n_exp)]
    slab = dev.alloc(n_exp * mb)
    dev.upload(slab, np.concatenate(mats))
    x = synth.normal_vector(rng, cols)
    xb = dev.shared_from(x)
    yb = dev.alloc(rows * 4)

    def chunks(off, n, total):
        c0, c1 = off // C, (off + n - 1) // C
        return sum(min((c + 1) * C, total) - c * C for c in range(c0, c1 + 1))

    def uploaded():
        return int(L.sepia_hip_uploaded_bytes())

    u0 = uploaded()
    dev.run(L.sepia_gpu_matvec_q, t, slab, 3 * mb, xb, yb, rows, cols)
    assert uploaded() - u0 == chunks(3 * mb, mb, n_exp * mb) + cols * 4
    u1 = uploaded()
    for _ in range(5):
        dev.run(L.sepia_gpu_matvec_q, t, slab, 3 * mb, xb, yb, rows, cols)
    assert uploaded() == u1, "a clean slab range was uploaded again"
    assert_close(dev.download(yb, rows), orc.qlinear(t, mats[3], rows, cols, x, threads=THREADS), what="slab e3")
    u2 = uploaded()
    dev.run(L.sepia_gpu_matvec_q, t, slab, 7 * mb, xb, yb, rows, cols)
    # expert 7's chunks (disjoint from expert 3's) and y, which the download above re-armed
    assert uploaded() - u2 == chunks(7 * mb, mb, n_exp * mb) + rows * 4
    assert_close(dev.download(yb, rows), orc.qlinear(t, mats[7], rows, cols, x, threads=THREADS), what="slab e7")
    new3 = synth.random_matrix(t, rows, cols, rng)
    dev.upload(slab, new3, offset=3 * mb)
    u3 = uploaded()
    dev.run(L.sepia_gpu_matvec_q, t, slab, 3 * mb, xb, yb, rows, cols)
    assert uploaded() - u3 == chunks(3 * mb, mb, n_exp * mb) + rows * 4
    assert_close(dev.download(yb, rows), orc.qlinear(t, new3, rows, cols, x, threads=THREADS), what="slab e3 new")
    for b in (slab, xb, yb):
        dev.free(b)



def test_freed_buffers_come_back_cleared(dev):
    """sepia_gpu_free keeps buffers of up to 64 MB; an allocation of the same
    kind and length takes one back without a new device or pinned
    allocation, and finds it cleared like a new buffer: the host copy, and
    the device copy an op reads before the host touches the buffer."""
    L = dev.L
    n = 3 * (1 << 16) + 256
    sevens = np.full(n // 4, 7.0, np.float32)
    a, out = dev.shared_from(sevens), dev.alloc(n)
    dev.run(L.sepia_gpu_copy, a, 0, out, 0, n // 4)
    assert np.all(dev.download(out, n // 4) == 7.0)
    p = dev.alloc(n, private=True)
    dev.run(L.sepia_gpu_copy, a, 0, p, 0, n // 4)
    for buf in (a, out, p):
        dev.free(buf)
    c0 = L.sepia_hip_alloc_count()
    b, c = dev.alloc(n), dev.alloc(n)
    q = dev.alloc(n, private=True)
    assert L.sepia_hip_alloc_count() == c0, "a freed buffer of the same length was not reused"
    dev.run(L.sepia_gpu_copy, b, 0, c, 0, n // 4)        # b's device copy, untouched by the host
    assert np.all(dev.download(c, n // 4) == 0.0)
    dev.run(L.sepia_gpu_copy, q, 0, c, 0, n // 4)        # the private one's
    assert np.all(dev.download(c, n // 4) == 0.0)
    assert np.all(dev.download(b, n // 4) == 0.0)        # b's host copy
    for buf in (b, c, q):
        dev.free(buf)


def test_shared_slab_partial_chunk_writes(dev, orc):
    """The reference's expert cache hands a slab's host pointer out once per
    miss, and its loader threads fill that expert's slot while hit experts of
    the same slab are already dispatched (src/sepia.c:3249-3290, :3908-3935).
    Slots smaller than a chunk share chunks, so an op that reads one slot
    must not mark the neighbouring bytes clean: a write the host makes there
    afterwards, through the pointer it already holds, reaches the op that
    reads it."""
    L = dev.L
    t, rows, cols, n_exp = 8, 5, 256, 12
    mb = rows * synth.row_bytes(t, cols)        # 1360 bytes: many slots per 64 KiB chunk
    rng = np.random.default_rng(809)
    mats = [synth.random_matrix(t, rows, cols, rng) for _ in range(n_exp)]
    slab = dev.alloc(n_exp * mb)
    hp = L.sepia_gpu_host_ptr(slab)
    dev.check(hp, "host_ptr")
    for e in (0, 1, 2):
        ctypes.memmove(hp + e * mb, mats[e].ctypes.data, mb)
    x = synth.normal_vector(rng, cols)
    xb = dev.shared_from(x)
    yb = dev.alloc(rows * 4)
    for e in (1, 0, 2):
        dev.run(L.sepia_gpu_matvec_q, t, slab, e * mb, xb, yb, rows, cols)
        assert_close(dev.download(yb, rows), orc.qlinear(t, mats[e], rows, cols, x), what="slot %d" % e)
    # later "loader" writes through the same pointer, no new host_ptr call
    for e in range(3, n_exp):
        ctypes.memmove(hp + e * mb, mats[e].ctypes.data, mb)
        dev.run(L.sepia_gpu_matvec_q, t, slab, e * mb, xb, yb, rows, cols)
        assert_close(dev.download(yb, rows), orc.qlinear(t, mats[e], rows, cols, x), what="slot %d" % e)
    # a slot rewritten after it was read, in the same way
    new1 = synth.random_matrix(t, rows, cols, rng)
    ctypes.memmove(hp + 1 * mb, new1.ctypes.data, mb)
    dev.run(L.sepia_gpu_matvec_q, t, slab, 1 * mb, xb, yb, rows, cols)
    assert_close(dev.download(yb, rows), orc.qlinear(t, new1, rows, cols, x), what="slot 1 rewritten")
    for b in (slab, xb, yb):
        dev.free(b)

# ------------------------------------------------------------------- MoE
@pytest.fixture
def mq_vector(dev, request):
    """Force how the matrix-core kernels read their vector: 1 = from global
    memory after the weight prologue, 2 = by LDS DMA ahead of it, 3 = by
    converter waves (DMA into the XQ place, converted there while the other
    waves decode their first step), 4 = the same conversion by the first
    stepping waves before they issue their own weights (the FFN gate/up
    launch only; the others keep the planner's choice)."""
    assert dev.L.sepia_hip_set_option(b"mq_x", request.param) == 1
    yield request.param
    dev.L.sepia_hip_set_option(b"mq_x", 0)


@pytest.mark.parametrize("mq_vector", [1, 2, 3, 4], indirect=True, ids=["global", "dma", "conv", "sconv"])
@pytest.mark.parametrize("t,out_dim,in_dim", [(12, 4096, 4096), (10, 3072, 6144), (11, 6144, 3072),
                                              (10, 12288, 2048), (12, 40, 12288), (17, 6144, 6144),
                                              (18, 6144, 6144), (18, 257, 3072), (17, 33, 1024)],
                         ids=lambda v: str(v))
def test_matvec_mq_vector_paths(dev, orc, mq_vector, t, out_dim, in_dim):
    with Launches(dev) as n:
        check_matvec(dev, orc, t, out_dim, in_dim, seed=out_dim + in_dim + t)
        assert n.count(MQ_NAMES[t]) == 1


def make_layer(dev, rng, hidden, inter, n_routed, n_shared, tg, tu, td, ts, rw_off=0, topk=6, tsd=None):
    """Shared buffers with seeded host data; returns (desc, spec, keep). The
    router matrix starts rw_off bytes into its buffer. Without shared experts
    their buffers hold a placeholder (never read). ts: the shared experts'
    format (tsd, if given, that of their down projection)."""
    tsd = ts if tsd is None else tsd
    gate = [synth.random_matrix(tg, inter, hidden, rng) for _ in range(n_routed)]
    up = [synth.random_matrix(tu, inter, hidden, rng) for _ in range(n_routed)]
    down = [synth.random_matrix(td, hidden, inter, rng) for _ in range(n_routed)]
    sg = [synth.random_matrix(ts, inter, hidden, rng) for _ in range(n_shared)]
    su = [synth.random_matrix(ts, inter, hidden, rng) for _ in range(n_shared)]
    sd = [synth.random_matrix(tsd, hidden, inter, rng) for _ in range(n_shared)]
    rw = (rng.standard_normal((n_routed + n_shared, hidden)) * 0.02).astype(np.float32)
    rb = rng.uniform(-0.1, 0.1, n_routed).astype(np.float32)
    bufs = {k: dev.shared_from(np.concatenate(v) if v else np.zeros(256, np.uint8)) for k, v in
            dict(gate=gate, up=up, down=down, s_gate=sg, s_up=su, s_down=sd).items()}
    bufs["rw"] = dev.alloc(rw.nbytes + rw_off)
    dev.upload(bufs["rw"], rw, offset=rw_off)
    bufs["rb"] = dev.shared_from(rb)
    d = hip.MoeLayerDesc()
    d.hidden, d.inter, d.n_routed, d.n_shared, d.topk = hidden, inter, n_routed, n_shared, topk
    d.route_scale, d.global_scale = 8.0, 1.0
    d.router_w, d.router_bias = bufs["rw"], bufs["rb"]
    d.router_w_off = rw_off
    for name, t, lst in (("gate", tg, gate), ("up", tu, up), ("down", td, down),
                         ("s_gate", ts, sg), ("s_up", ts, su), ("s_down", tsd, sd)):
        setattr(d, name, hip.ExpertTensor(bufs[name], 0, lst[0].nbytes if lst else 0, t))
    spec = dict(hidden=hidden, inter=inter, n_routed=n_routed, n_shared=n_shared, topk=topk, route_scale=8.0,
                global_scale=1.0, router_w=rw, router_bias=rb, t_gate=tg, t_up=tu, t_down=td,
                ts_gate=ts, ts_up=ts, ts_down=tsd, gate=gate, up=up, down=down, s_gate=sg, s_up=su, s_down=sd)
    return d, spec, bufs


def run_moe(dev, desc, x):
    import ctypes
    xb = dev.shared_from(x)
    yb = dev.alloc(x.nbytes)
    rb = dev.alloc(64 * 4)
    dev.run(dev.L.sepia_gpu_moe_decode, ctypes.byref(desc), xb, yb, rb)
    y = dev.download(yb, x.size)
    idx = dev.download(rb, desc.topk, dtype=np.int32)
    w = dev.download(rb, desc.topk + desc.n_shared, offset=desc.topk * 4)
    for b in (xb, yb, rb):
        dev.free(b)
    return y, idx, w


def check_route(orc, spec, logits, idx_gpu, w_gpu):
    """Selection must match the oracle's, or differ only across a near-tie of the
    selection scores (the reference's near-tie protocol); weights then follow
    the GPU's selection."""
    idx_ref, w_ref = orc.route_select(logits, spec["router_bias"], spec["n_routed"], spec["n_shared"],
                                      spec["topk"], spec["route_scale"], spec["global_scale"])
    if list(idx_gpu) != list(idx_ref):
        score = 1.0 / (1.0 + np.exp(-logits[:spec["n_routed"]].astype(np.float64))) + spec["router_bias"]
        s_sorted = np.sort(score)[::-1]
        gap = s_sorted[spec["topk"] - 1] - s_sorted[spec["topk"]]
        assert gap < 1e-5 and set(idx_gpu) ^ set(idx_ref), (idx_gpu, idx_ref, gap)
        w_ref = orc.route_weights(logits, spec["n_routed"], spec["n_shared"], idx_gpu, spec["route_scale"],
                                  spec["global_scale"])
    # The weights are exp(logsigmoid(logit) - lse): a logit's absolute error is
    # about their relative error. The GPU routers sum 6144 f32 products in
    # another order than the oracle's double sum (|error| up to a few 1e-5 at
    # C3's logit sizes), so 1e-4 relative; y is held to its own bar.
    assert np.allclose(w_gpu, w_ref, rtol=1e-4, atol=0), (w_gpu, w_ref)
    return list(idx_gpu)


@pytest.mark.parametrize("types", [(10, 10, 11, 12), (17, 17, 18, 13), (17, 17, 23, 14)],
                         ids=["q2k_q3k_q4k", "iq2xs_iq3xxs_q5k", "iq2xs_iq4xs_q6k"])
@pytest.mark.parametrize("seed", [0, 1])
def test_moe_decode_small(dev, orc, types, seed):
    rng = np.random.default_rng(seed)
    tg, tu, td, ts = types
    desc, spec, bufs = make_layer(dev, rng, hidden=1024, inter=512, n_routed=32, n_shared=2,
                                  tg=tg, tu=tu, td=td, ts=ts)
    x = synth.normal_vector(rng, 1024)
    y, idx, w = run_moe(dev, desc, x)
    y_ref, logits, idx_ref, w_ref = orc.moe_layer(spec, x, threads=THREADS)
    chosen = check_route(orc, spec, logits, idx, w)
    if chosen != list(idx_ref):
        y_ref, _, _, _ = orc.moe_layer(spec, x, force_idx=chosen, threads=THREADS)
    assert_close(y, y_ref, what="moe small", gate=False)
    for b in bufs.values():
        dev.free(b)


@pytest.mark.parametrize("kernel_path", ["mq", "generic", "t1", "t3"], indirect=True)
@pytest.mark.parametrize("types", [(10, 10, 11, 12), (12, 12, 12, 10), (11, 11, 10, 11)],
                         ids=["q2k_q3k_q4k", "q4k_q4k_q2k", "q3k_q2k_q3k"])
def test_moe_decode_tile_shapes(dev, orc, kernel_path, types):
    """Tile-eligible layer (hidden 2048, inter 1024): router + x planes +
    mixed-format gate/up and down launches."""
    rng = np.random.default_rng(zlib.crc32(repr(types).encode()) & 0xFFFF)
    tg, tu, td, ts = types
    desc, spec, bufs = make_layer(dev, rng, hidden=2048, inter=1024, n_routed=16, n_shared=2,
                                  tg=tg, tu=tu, td=td, ts=ts)
    x = synth.normal_vector(rng, 2048)
    y, idx, w = run_moe(dev, desc, x)
    y_ref, logits, idx_ref, w_ref = orc.moe_layer(spec, x, threads=THREADS)
    chosen = check_route(orc, spec, logits, idx, w)
    if chosen != list(idx_ref):
        y_ref, _, _, _ = orc.moe_layer(spec, x, force_idx=chosen, threads=THREADS)
    assert_close(y, y_ref, what="moe tile %s" % kernel_path, gate=False)
    for b in bufs.values():
        dev.free(b)


@pytest.mark.parametrize("rw_off", [0, 4])
def test_moe_decode_c3_shape(dev, orc, rw_off):
    """BASELINE configs[2] shapes (hidden 6144, inter 3072, Q2_K/Q3_K routed,
    Q4_K shared, top-6) with 16 routed experts resident; rw_off 4 takes the
    router's unaligned path (x then reaches gate/up as f32)."""
    rng = np.random.default_rng(300 + rw_off)
    desc, spec, bufs = make_layer(dev, rng, hidden=6144, inter=3072, n_routed=16, n_shared=2,
                                  tg=10, tu=10, td=11, ts=12, rw_off=rw_off)
    x = synth.normal_vector(rng, 6144)
    y, idx, w = run_moe(dev, desc, x)
    y_ref, logits, idx_ref, w_ref = orc.moe_layer(spec, x, threads=THREADS)
    chosen = check_route(orc, spec, logits, idx, w)
    if chosen != list(idx_ref):
        y_ref, _, _, _ = orc.moe_layer(spec, x, force_idx=chosen, threads=THREADS)
    assert_close(y, y_ref, what="moe c3 shape", gate=False)
    for b in bufs.values():
        dev.free(b)


@pytest.mark.parametrize("mq_geometry", [(1, 1, 1), (1, 3, 2), (3, 1, 2), (2, 1, 3)], indirect=True,
                         ids=lambda v: str(v))
def test_moe_decode_mq_geometries(dev, orc, mq_geometry):
    """C3 layer shapes (16 routed experts resident) under forced matrix-core
    geometries; both FFN kernels must be the matrix-core ones."""
    rng = np.random.default_rng(77)
    desc, spec, bufs = make_layer(dev, rng, hidden=6144, inter=3072, n_routed=16, n_shared=2,
                                  tg=10, tu=10, td=11, ts=12)
    x = synth.normal_vector(rng, 6144)
    with Launches(dev) as n:
        y, idx, w = run_moe(dev, desc, x)
        assert n.count("sepia_mq_gateup") == 1 and n.count("sepia_mq_down") == 1
    y_ref, logits, idx_ref, w_ref = orc.moe_layer(spec, x, threads=THREADS)
    chosen = check_route(orc, spec, logits, idx, w)
    if chosen != list(idx_ref):
        y_ref, _, _, _ = orc.moe_layer(spec, x, force_idx=chosen, threads=THREADS)
    assert_close(y, y_ref, what="moe mq %s" % (mq_geometry,), gate=False)
    for b in bufs.values():
        dev.free(b)


@pytest.mark.parametrize("types,n_routed,n_shared,topk",
                         [((10, 10, 11, 12), 16, 2, 6), ((12, 12, 12, 10), 16, 2, 6), ((11, 11, 10, 11), 16, 2, 6),
                          ((10, 10, 11, 12), 16, 0, 6), ((10, 10, 11, 12), 8, 1, 1)],
                         ids=["q2k_q3k_q4k", "q4k_q4k_q2k", "q3k_q2k_q3k", "no_shared", "top1"])
def test_moe_decode_slots(dev, orc, types, n_routed, n_shared, topk):
    """C3 layer shapes with mixed formats (routed and shared workgroups on
    geometries of their own formats), without shared experts and with a
    single routed slot: the router and the two matrix-core FFN launches (the
    launch counts show it) give the oracle's result twice in a row (the down
    launch's arrival counters must be back at zero after the first)."""
    rng = np.random.default_rng(9100 + types[0] + n_shared + topk)
    tg, tu, td, ts = types
    desc, spec, bufs = make_layer(dev, rng, hidden=6144, inter=3072, n_routed=n_routed, n_shared=n_shared,
                                  tg=tg, tu=tu, td=td, ts=ts, topk=topk)
    for rep in range(2):
        x = synth.normal_vector(rng, 6144)
        with Launches(dev) as n:
            y, idx, w = run_moe(dev, desc, x)
            assert n.count("sepia_moe_route") == 1
            assert n.count("sepia_mq_gateup") == 1 and n.count("sepia_mq_down") == 1
        y_ref, logits, idx_ref, w_ref = orc.moe_layer(spec, x, threads=THREADS)
        chosen = check_route(orc, spec, logits, idx, w)
        if chosen != list(idx_ref):
            y_ref, _, _, _ = orc.moe_layer(spec, x, force_idx=chosen, threads=THREADS)
        assert_close(y, y_ref, what="moe slots rep %d" % rep, gate=False)
    for b in bufs.values():
        dev.free(b)


# The real checkpoint's layers (reference docs/gguf-inventory-ud-q2_k_xl.md:
# 72-111, 214-235): IQ2_XS gate/up with IQ3_XXS down (57 layers) or IQ4_XS
# down (7 layers), IQ3_XXS gate/up on the last layer; shared experts Q5_K,
# Q6_K or Q8_0. (gate, up, down, shared gate/up, shared down).
REAL_LAYERS = [((17, 17, 18, 13, 14), "iq2xs_iq3xxs__q5k_q6k"), ((17, 17, 23, 13, 14), "iq2xs_iq4xs__q5k_q6k"),
               ((18, 18, 18, 8, 8), "iq3xxs__q8_0"), ((17, 17, 18, 14, 13), "iq2xs_iq3xxs__q6k_q5k"),
               ((17, 17, 23, 8, 14), "iq2xs_iq4xs__q8_0_q6k")]


@pytest.mark.parametrize("types", [t for t, _ in REAL_LAYERS], ids=[n for _, n in REAL_LAYERS])
def test_moe_decode_real_types(dev, orc, types):
    """The real checkpoint's formats at its layer shape (hidden 6144, inter
    3072, top-6 + 2 shared; 16 routed experts resident): the router and the
    two matrix-core FFN launches, their codebooks in LDS, routed and shared
    workgroups each on its own format (the launch counts show the path), twice
    in a row (the arrival counters must be back at zero)."""
    rng = np.random.default_rng(zlib.crc32(repr(types).encode()) & 0xFFFF)
    tg, tu, td, ts, tsd = types
    desc, spec, bufs = make_layer(dev, rng, hidden=6144, inter=3072, n_routed=16, n_shared=2,
                                  tg=tg, tu=tu, td=td, ts=ts, tsd=tsd)
    for rep in range(2):
        x = synth.normal_vector(rng, 6144)
        with Launches(dev) as n:
            y, idx, w = run_moe(dev, desc, x)
            assert n.count("sepia_moe_route") == 1
            assert n.count("sepia_mq_gateup") == 1 and n.count("sepia_mq_down") == 1
        y_ref, logits, idx_ref, w_ref = orc.moe_layer(spec, x, threads=THREADS)
        chosen = check_route(orc, spec, logits, idx, w)
        if chosen != list(idx_ref):
            y_ref, _, _, _ = orc.moe_layer(spec, x, force_idx=chosen, threads=THREADS)
        assert_close(y, y_ref, what="moe real types rep %d" % rep, gate=False)
    for b in bufs.values():
        dev.free(b)


@pytest.mark.parametrize("mq_vector", [1, 2, 3, 4], indirect=True, ids=["global", "dma", "conv", "sconv"])
def test_moe_decode_mq_vector_paths(dev, orc, mq_vector):
    """C3 layer shapes with 16 routed experts resident; gate/up and down read x
    and h either way."""
    rng = np.random.default_rng(500 + mq_vector)
    desc, spec, bufs = make_layer(dev, rng, hidden=6144, inter=3072, n_routed=16, n_shared=2,
                                  tg=10, tu=10, td=11, ts=12)
    for rep in range(2):
        x = synth.normal_vector(rng, 6144)
        with Launches(dev) as n:
            y, idx, w = run_moe(dev, desc, x)
            assert n.count("sepia_mq_gateup") == 1 and n.count("sepia_mq_down") == 1
        y_ref, logits, idx_ref, w_ref = orc.moe_layer(spec, x, threads=THREADS)
        chosen = check_route(orc, spec, logits, idx, w)
        if chosen != list(idx_ref):
            y_ref, _, _, _ = orc.moe_layer(spec, x, force_idx=chosen, threads=THREADS)
        assert_close(y, y_ref, what="moe mq_x %d rep %d" % (mq_vector, rep), gate=False)
    for b in bufs.values():
        dev.free(b)


def run_prefill(dev, desc, X):
    import ctypes
    T, H = X.shape
    n_sel = desc.topk + desc.n_shared
    xb = dev.shared_from(X)
    yb = dev.alloc(X.nbytes)
    rb = dev.alloc(T * (desc.topk + n_sel) * 4)
    dev.run(dev.L.sepia_gpu_moe_prefill, ctypes.byref(desc), T, xb, yb, rb)
    y = dev.download(yb, T * H).reshape(T, H)
    idx = dev.download(rb, T * desc.topk, dtype=np.int32).reshape(T, desc.topk)
    w = dev.download(rb, T * n_sel, offset=T * desc.topk * 4).reshape(T, n_sel)
    for b in (xb, yb, rb):
        dev.free(b)
    return y, idx, w


@pytest.mark.parametrize("kernel_path", ["mq", "generic"], indirect=True)
def test_moe_route_exact_ties(dev, orc, kernel_path):
    """Exactly equal selection scores: 200 routed experts (four to a lane of
    the selecting wave) whose router rows and biases repeat in pairs over
    three groups, so equal scores sit side by side in one lane and across
    lanes. Each selection (the gate/up launch's on the matrix-core path, the
    router's last workgroup on the generic one, and the prefill's per-token
    one) must be the oracle's exactly: the largest score first, the lowest
    expert index among equals."""
    rng = np.random.default_rng(777)
    n_routed, n_shared, topk, H = 200, 2, 6, 1024
    desc, spec, bufs = make_layer(dev, rng, hidden=H, inter=1024, n_routed=n_routed, n_shared=n_shared,
                                  tg=10, tu=10, td=11, ts=12)
    grp = (np.arange(n_routed) // 2) % 3
    base = (rng.standard_normal((3, H)) * 0.02).astype(np.float32)
    rw = np.concatenate([base[grp], (rng.standard_normal((n_shared, H)) * 0.02).astype(np.float32)])
    rb = np.array([0.05, -0.02, 0.01], dtype=np.float32)[grp]
    dev.upload(bufs["rw"], rw)
    dev.upload(bufs["rb"], rb)
    spec["router_w"], spec["router_bias"] = rw, rb
    for rep in range(2):
        x = synth.normal_vector(rng, H)
        y, idx, w = run_moe(dev, desc, x)
        _, logits, idx_ref, _ = orc.moe_layer(spec, x, threads=THREADS)
        assert list(idx) == list(idx_ref), (rep, list(idx), list(idx_ref))
        assert len(set(grp[idx_ref])) == 1   # all six from one group of tied scores
        w_ref = orc.route_weights(logits, n_routed, n_shared, idx_ref, 8.0, 1.0)
        assert np.allclose(w, w_ref, rtol=1e-4, atol=0), (w, w_ref)
    if kernel_path == "mq":
        X = np.stack([synth.normal_vector(rng, H) for _ in range(3)])
        _, pidx, _ = run_prefill(dev, desc, X)
        for t in range(3):
            _, _, idx_ref, _ = orc.moe_layer(spec, X[t], threads=THREADS)
            assert list(pidx[t]) == list(idx_ref), (t, list(pidx[t]), list(idx_ref))
    for b in bufs.values():
        dev.free(b)


def bf16_normal(rng, shape):
    """N(0,1) f32 values rounded toward zero to bf16 (exactly representable in bf16)."""
    v = rng.standard_normal(shape).astype(np.float32)
    return (v.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)


# (hidden, inter, n_routed, n_shared), (gate/up, down, shared gate/up[, shared down]) formats, tokens
PREFILL_CASES = [
    ((2048, 1024, 16, 2), (10, 11, 12), 40),
    ((6144, 3072, 16, 2), (10, 11, 12), 48),      # BASELINE configs[4] shapes, 16 experts resident
    ((2048, 1024, 12, 1), (17, 18, 14), 33),      # IQ2_XS / IQ3_XXS routed, Q6_K shared
    ((1024, 2048, 8, 2), (13, 23, 11), 20),       # Q5_K / IQ4_XS routed, Q3_K shared (bf16 kernels)
    ((2048, 1024, 12, 1), (11, 10, 10), 37),      # Q3_K / Q2_K routed, Q2_K shared
    # the real checkpoint's format mixes (the f16 kernels on the default path)
    ((6144, 3072, 16, 2), (17, 18, 13, 14), 48),  # IQ2_XS / IQ3_XXS routed, Q5_K / Q6_K shared
    ((2048, 1024, 12, 2), (17, 23, 13, 14), 40),  # IQ4_XS down
    ((1024, 2048, 8, 2), (13, 14, 13, 14), 20),   # Q5_K / Q6_K routed
    ((256, 512, 8, 1), (17, 18, 13, 14), 11),     # the smallest grids: one 256-row workgroup per slice row
    ((2048, 1024, 8, 0), (17, 18, 13, 14), 15),   # no shared experts (f16 kernels)
    ((2048, 1024, 8, 0), (10, 11, 12), 15),       # no shared experts (int8 kernels)
    ((2048, 1024, 8, 2), (17, 18, 13, 14), 1),    # one token: every unit a single pair (f16)
    ((2048, 1024, 8, 2), (10, 11, 12), 1),        # one token (int8)
]
# Layers with Q8_0 projections: the f16 kernels only (no bf16 kernel takes Q8_0).
PREFILL_CASES_Q8 = [
    ((2048, 1024, 12, 2), (18, 18, 8, 8), 37),    # IQ3_XXS gate/up (layer 65), Q8_0 shared
    ((2048, 1024, 8, 1), (8, 23, 8, 14), 9),      # Q8_0 routed, one M tile per unit
]


PF_PATHS = {"q": dict(pf_q=1, pf_h=1, pf_route_m=1), "tile": dict(pf_q=0, pf_h=0, pf_route_m=0)}


@pytest.mark.parametrize("path", ["q", "tile"])
@pytest.mark.parametrize("x_kind", ["bf16", "f32"])
@pytest.mark.parametrize("shape,types,T", PREFILL_CASES, ids=lambda v: str(v))
def test_moe_prefill(dev, orc, shape, types, T, x_kind, path):
    """Every token of the batch against the oracle's single-token layer (its
    own routing, near-ties per the reference protocol); two runs bitwise equal.
    x either bf16-representable or full f32. path: a layer of Q2_K / Q3_K /
    Q4_K projections on the int8 matrix cores, and a layer of the real
    checkpoint's formats (IQ2_XS, IQ3_XXS, IQ4_XS, Q5_K, Q6_K) on the f16
    ones (q, the default; options pf_q, pf_h), or either on the bf16 kernels
    with bit-exact dequantized weights (tile; pf_q 0 and pf_h 0, which also
    runs the router on sepia_pf_route, pf_route_m 0). Layers with other
    format mixes take the bf16 kernels on both paths."""
    hidden, inter, n_routed, n_shared = shape
    tgu, td, ts = types[:3]
    tsd = types[3] if len(types) > 3 else None
    rng = np.random.default_rng(hidden + 7 * T + tgu)
    desc, spec, bufs = make_layer(dev, rng, hidden=hidden, inter=inter, n_routed=n_routed, n_shared=n_shared,
                                  tg=tgu, tu=tgu, td=td, ts=ts, tsd=tsd)
    X = bf16_normal(rng, (T, hidden)) if x_kind == "bf16" else rng.standard_normal((T, hidden)).astype(np.float32)
    for k, v in PF_PATHS[path].items():
        assert dev.L.sepia_hip_set_option(k.encode(), v) == 1
    try:
        y, idx, w = run_prefill(dev, desc, X)
        y2, _, _ = run_prefill(dev, desc, X)
    finally:
        for k, v in PF_PATHS["q"].items():
            dev.L.sepia_hip_set_option(k.encode(), v)
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))
    for t in range(T):
        y_ref, logits, idx_ref, w_ref = orc.moe_layer(spec, X[t], threads=THREADS)
        chosen = check_route(orc, spec, logits, idx[t], w[t])
        if chosen != list(idx_ref):
            y_ref, _, _, _ = orc.moe_layer(spec, X[t], force_idx=chosen, threads=THREADS)
        assert_close(y[t], y_ref, what="prefill %s token %d" % (types, t), gate=False)
    for b in bufs.values():
        dev.free(b)


@pytest.mark.parametrize("x_kind", ["bf16", "f32"])
@pytest.mark.parametrize("shape,types,T", PREFILL_CASES_Q8, ids=lambda v: str(v))
def test_moe_prefill_q8_0(dev, orc, shape, types, T, x_kind):
    """Layers with Q8_0 projections on the f16 kernels (the default path)
    against the oracle, two runs bitwise equal; with pf_h 0 the library
    refuses them (no other prefill kernel takes Q8_0)."""
    test_moe_prefill(dev, orc, shape, types, T, x_kind, "q")
    rng = np.random.default_rng(5)
    desc, _spec, bufs = make_layer(dev, rng, hidden=shape[0], inter=shape[1], n_routed=shape[2], n_shared=shape[3],
                                   tg=types[0], tu=types[0], td=types[1], ts=types[2], tsd=types[3])
    X = rng.standard_normal((4, shape[0])).astype(np.float32)
    xb, yb = dev.shared_from(X), dev.alloc(X.nbytes)
    assert dev.L.sepia_hip_set_option(b"pf_h", 0) == 1
    try:
        dev.begin()
        try:
            assert dev.L.sepia_gpu_moe_prefill(ctypes.byref(desc), 4, xb, yb, None) == 0
        finally:
            assert dev.L.sepia_gpu_end() == 1
    finally:
        dev.L.sepia_hip_set_option(b"pf_h", 1)
    for b in list(bufs.values()) + [xb, yb]:
        dev.free(b)


@pytest.mark.parametrize("off", [0, 2])
def test_moe_prefill_row_alignment(dev, orc, off):
    """The int8 prefill path stages weight blocks from 4-byte boundaries, so
    the host takes it only when every projection's base, expert stride and
    row bytes are multiples of 4. A Q2_K/Q3_K/Q4_K layer whose routed gate
    starts 2 bytes into its buffer runs on the bf16 kernels instead (launch
    counts asserted); both match the oracle."""
    rng = np.random.default_rng(97 + off)
    desc, spec, bufs = make_layer(dev, rng, hidden=2048, inter=1024, n_routed=8, n_shared=1,
                                  tg=10, tu=10, td=11, ts=12)
    g = np.concatenate(spec["gate"])
    bufs["gate_off"] = dev.alloc(g.nbytes + off)
    dev.upload(bufs["gate_off"], g, offset=off)
    desc.gate = hip.ExpertTensor(bufs["gate_off"], off, spec["gate"][0].nbytes, 10)
    X = bf16_normal(rng, (12, 2048))
    with Launches(dev) as ln:
        y, idx, w = run_prefill(dev, desc, X)
    q = ln.count("sepia_pf_gateup_q")
    assert (q > 0) == (off == 0) and (ln.count("sepia_pf_gateup") > 0) == (off != 0), (off, q)
    for t in range(X.shape[0]):
        y_ref, logits, idx_ref, w_ref = orc.moe_layer(spec, X[t], threads=THREADS)
        chosen = check_route(orc, spec, logits, idx[t], w[t])
        if chosen != list(idx_ref):
            y_ref, _, _, _ = orc.moe_layer(spec, X[t], force_idx=chosen, threads=THREADS)
        assert_close(y[t], y_ref, what="prefill rows at offset %d, token %d" % (off, t), gate=False)
    for b in bufs.values():
        dev.free(b)


def test_moe_prefill_matches_decode(dev, orc):
    """A prefill batch and token-by-token decode of the same layer agree to the
    layer bar. Their routers sum the logits in different orders, so a token
    may be routed differently only across a near-tie of the selection scores
    (check_route against the oracle's logits); at least 10 of the 12 tokens
    must be compared."""
    rng = np.random.default_rng(4242)
    desc, spec, bufs = make_layer(dev, rng, hidden=2048, inter=1024, n_routed=16, n_shared=2,
                                  tg=10, tu=10, td=11, ts=12)
    X = bf16_normal(rng, (12, 2048))
    y, idx, wp = run_prefill(dev, desc, X)
    compared = 0
    for t in range(12):
        yd, idd, wd = run_moe(dev, desc, X[t].copy())
        logits = orc.linear_f32(spec["router_w"], X[t])
        check_route(orc, spec, logits, idx[t], wp[t])
        check_route(orc, spec, logits, idd, wd)
        if list(idd) == list(idx[t]):
            assert_close(y[t], yd, what="prefill vs decode token %d" % t, gate=False)
            compared += 1
    assert compared >= 10, "only %d of 12 tokens routed alike" % compared
    for b in bufs.values():
        dev.free(b)


def run_expert_ffn(dev, tensors, n_experts, expert, hidden, inter, x):
    import ctypes
    xb = dev.shared_from(x)
    yb = dev.alloc(hidden * 4)
    g, u, d = (ctypes.byref(t) for t in tensors)
    dev.run(dev.L.sepia_gpu_expert_ffn, g, u, d, n_experts, expert, hidden, inter, xb, yb)
    y = dev.download(yb, hidden)
    dev.free(xb)
    dev.free(yb)
    return y


@pytest.mark.parametrize("kernel_path", ["mq", "generic", "t1", "t2", "t3"], indirect=True)
@pytest.mark.parametrize("types,hidden,inter", [((10, 10, 11), 6144, 3072), ((12, 12, 12), 4096, 2048),
                                                ((11, 11, 10), 2048, 1024)],
                         ids=["c2_q2k_q3k", "q4k_4096", "q3k_q2k_2048"])
def test_expert_ffn(dev, orc, kernel_path, types, hidden, inter):
    """One routed expert (BASELINE configs[1] at its real shape first) picked
    out of a stack of three."""
    rng = np.random.default_rng(hidden + inter + types[0])
    tg, tu, td = types
    n_e, e = 3, 1
    gate = [synth.random_matrix(tg, inter, hidden, rng) for _ in range(n_e)]
    up = [synth.random_matrix(tu, inter, hidden, rng) for _ in range(n_e)]
    down = [synth.random_matrix(td, hidden, inter, rng) for _ in range(n_e)]
    bufs = [dev.shared_from(np.concatenate(v)) for v in (gate, up, down)]
    tensors = [hip.ExpertTensor(b, 0, v[0].nbytes, t) for b, v, t in zip(bufs, (gate, up, down), types)]
    x = synth.normal_vector(rng, hidden)
    y = run_expert_ffn(dev, tensors, n_e, e, hidden, inter, x)
    want = orc.expert_ffn(tg, gate[e], tu, up[e], td, down[e], hidden, inter, x, threads=THREADS)
    assert_close(y, want, what="expert ffn %s" % kernel_path, gate=False)
    for b in bufs:
        dev.free(b)


@pytest.mark.parametrize("types,hidden,inter", [((10, 10, 11), 6144, 3072), ((12, 12, 10), 4096, 2048),
                                                ((11, 11, 12), 2048, 8192), ((10, 10, 10), 1024, 1024),
                                                ((12, 12, 11), 3072, 4096), ((17, 17, 23), 6144, 3072),
                                                ((13, 13, 14), 4096, 2048), ((8, 8, 18), 2048, 3072),
                                                ((14, 14, 8), 1024, 1024)],
                         ids=["c2", "units_half", "two_units_per_wg", "tiny", "q4k_q3k", "iq2xs_iq4xs",
                              "q5k_q6k", "q8_0_iq3xxs", "q6k_q8_0_tiny"])
def test_expert_ffn_shapes(dev, orc, types, hidden, inter):
    """The expert FFN on the matrix-core launches over shapes with fewer row
    groups than workgroups, several row groups per workgroup and long rows;
    each shape runs twice."""
    rng = np.random.default_rng(7 * hidden + inter)
    tg, tu, td = types
    n_e, e = 2, 1
    gate = [synth.random_matrix(tg, inter, hidden, rng) for _ in range(n_e)]
    up = [synth.random_matrix(tu, inter, hidden, rng) for _ in range(n_e)]
    down = [synth.random_matrix(td, hidden, inter, rng) for _ in range(n_e)]
    bufs = [dev.shared_from(np.concatenate(v)) for v in (gate, up, down)]
    tensors = [hip.ExpertTensor(b, 0, v[0].nbytes, t) for b, v, t in zip(bufs, (gate, up, down), types)]
    try:
        for k in range(2):
            x = synth.normal_vector(rng, hidden)
            with Launches(dev) as n:
                y = run_expert_ffn(dev, tensors, n_e, e, hidden, inter, x)
                assert n.count("sepia_mq_gateup") == 1 and n.count("sepia_mq_down") == 1
            want = orc.expert_ffn(tg, gate[e], tu, up[e], td, down[e], hidden, inter, x, threads=THREADS)
            assert_close(y, want, what="expert ffn %dx%d run %d" % (hidden, inter, k), gate=False)
    finally:
        for b in bufs:
            dev.free(b)
