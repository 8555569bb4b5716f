"""Kernel-side failure reports reach the host.

The only spin waits in the kernels are the matrix-core launches' waits on
LDS counters (converter waves publishing the XQ vector), bounded in time.
When one expires the wave goes on, so the launch's outputs are invalid; it
records error code 5 in the library's device error word, and sepia_gpu_end
reports it: a log line and a return of 0 (the reference's convention for a
failed batch, src/sepia_gpu.h:1-3, :81-88), then the word is clear again.
The expiry is forced from the host by a bound of one tick; nothing in the
launch indexes memory by the values it then reads too early.
"""
import ctypes

import numpy as np
import pytest

from sepia_amd import hip, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    return hip.Device()


def matvec_batch(dev, t, w, x, out_dim, in_dim):
    """One matvec_q in its own batch; (op ok, end ok, y)."""
    L = dev.L
    wb, xb, yb = dev.shared_from(w), dev.shared_from(x), dev.alloc(out_dim * 4)
    dev.begin()
    ok = L.sepia_gpu_matvec_q(t, wb, 0, xb, yb, out_dim, in_dim)
    end_ok = L.sepia_gpu_end()
    y = dev.download(yb, out_dim)
    for b in (wb, xb, yb):
        dev.free(b)
    return ok, end_ok, y


def test_wait_expiry_fails_the_batch(dev, orc):
    L = dev.L
    t, out_dim, in_dim = 18, 6144, 6144
    rng = np.random.default_rng(404)
    w = synth.random_matrix(t, out_dim, in_dim, rng)
    x = synth.normal_vector(rng, in_dim)
    assert L.sepia_hip_take_device_error() == 0
    assert L.sepia_hip_set_option(b"mq_x", 3) == 1          # converter waves: the others wait on them
    try:
        assert L.sepia_hip_set_option(b"wait_ticks", 1) == 1
        try:
            ok, end_ok, _ = matvec_batch(dev, t, w, x, out_dim, in_dim)
        finally:
            assert L.sepia_hip_set_option(b"wait_ticks", 0) == 1
        assert ok == 1 and end_ok == 0, (ok, end_ok)
        assert L.sepia_hip_take_device_error() == 0          # end reported and cleared it
        ok, end_ok, y = matvec_batch(dev, t, w, x, out_dim, in_dim)
    finally:
        L.sepia_hip_set_option(b"mq_x", 0)
    assert ok == 1 and end_ok == 1
    want = orc.qlinear(t, w, out_dim, in_dim, x)
    assert float(np.max(np.abs(y - want))) <= 1e-4 * float(np.max(np.abs(want)))
