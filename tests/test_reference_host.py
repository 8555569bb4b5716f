"""The reference's own engine driving this library.

oracle/_ref/sepia_hip is the reference's unmodified src/sepia.c (with its
quants.c and tokenizer.c) linked against sepia_amd/lib/libsepia_hip.so in
place of its Metal shim (oracle/Makefile, target ref). Its GPU gates are
weight-free and run here:

  --metal --gpu-selftest     wrap_mmap / alloc / free / host_ptr / touch
                             dispatch (reference src/sepia.c:4449-4540);
  --metal --gpu-quants F...  bitwise GPU dequant against the SQFX fixtures'
                             expected floats, then matvec_q against the
                             reference's CPU qlinear at its relative-error
                             gate (src/sepia.c:5903-6061);
  --metal --gpu-compare-attn the attention path (f32 matvec, sconv, rmsnorm,
                             rel_project, banded_attn) at the model's sliding
                             and global geometries against its CPU
                             attn_forward_chunk, kv ranges up to 130000
                             (src/sepia.c:4900-5200, :5217-5326).

The CPU tests check that the binary resolves every GPU symbol it calls in
this library and that it fails cleanly when no GPU initialises.
"""
import glob
import os
import re
import subprocess

import pytest

from conftest import GOLDEN, ROOT
from sepia_amd import hip

BIN = os.path.join(ROOT, "oracle", "_ref", "sepia_hip")
HAVE_GPU = os.path.exists("/dev/kfd") and os.access("/dev/kfd", os.R_OK)

needs_bin = pytest.mark.skipif(not os.path.exists(BIN),
                               reason="oracle/_ref/sepia_hip not built (the reference checkout was absent at build)")


def run(*args, timeout=120):
    return subprocess.run([BIN, *args], capture_output=True, text=True, timeout=timeout)


@needs_bin
def test_reference_engine_links_this_library():
    ldd = subprocess.run(["ldd", BIN], capture_output=True, text=True, check=True).stdout
    assert re.search(r"libsepia_hip\.so => \S*sepia_amd/lib/libsepia_hip\.so", ldd), ldd
    undef = set(re.findall(r"\bU (sepia_gpu_\w+)", subprocess.run(["nm", "-u", BIN], capture_output=True,
                                                                  text=True, check=True).stdout))
    exported = set(re.findall(r"\bT (sepia_\w+)", subprocess.run(
        ["nm", "-D", "--defined-only", hip.LIB_PATH], capture_output=True, text=True, check=True).stdout))
    assert len(undef) >= 25 and undef <= exported, undef - exported


@needs_bin
@pytest.mark.skipif(HAVE_GPU, reason="checks the no-GPU failure path")
def test_reference_engine_without_gpu_fails_cleanly():
    r = run("--metal", "--gpu-selftest")
    assert r.returncode != 0
    assert "sepia: hip:" in r.stderr and "initialization failed" in r.stderr, r.stderr


@needs_bin
@pytest.mark.gpu
def test_reference_gpu_selftest():
    r = run("--metal", "--gpu-selftest")
    assert r.returncode == 0, r.stderr
    assert "gpu selftest ok" in r.stdout, (r.stdout, r.stderr)


@needs_bin
@pytest.mark.gpu
def test_reference_gpu_quants_gate():
    fixtures = sorted(glob.glob(os.path.join(GOLDEN, "quants", "*.bin")))
    r = run("--metal", "--gpu-quants", *fixtures)
    assert r.returncode == 0, (r.stdout, r.stderr)
    assert "gpu-quants ok" in r.stdout, r.stdout
    lines = [ln for ln in r.stdout.splitlines() if ln.startswith("gpu-quants: ") and "type" in ln]
    dq = [ln for ln in lines if "dequant" in ln]
    mv = [ln for ln in lines if "matvec" in ln]
    # the seven quantized types the reference has GPU kernels for, dequant and matvec each
    assert len(dq) == 7 and all(ln.rstrip().endswith("ok") for ln in dq), dq
    assert len(mv) == 7 and all(ln.rstrip().endswith("ok") for ln in mv), mv


@needs_bin
@pytest.mark.gpu
def test_reference_gpu_compare_attn_gate():
    r = run("--metal", "--gpu-compare-attn", timeout=600)
    assert r.returncode == 0, (r.stdout, r.stderr)
    assert "gpu compare attn ok" in r.stdout, r.stdout
    cases = [ln for ln in r.stdout.splitlines() if ln.startswith("gpu-compare-attn: ") and "max_rel_err" in ln
             and "worst case" not in ln]
    assert len(cases) == 7 and all(ln.rstrip().endswith("ok") for ln in cases), cases
