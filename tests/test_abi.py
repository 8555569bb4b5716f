"""CPU-side checks of the C-ABI library: it loads, exports every function the
headers declare with the reference's 30-symbol surface intact, and follows
the reference's error convention (0/NULL plus a log line, never an exit)
when used without an initialised device. No GPU compute is issued here."""
import os
import re
import subprocess
import sys

import pytest

from conftest import ROOT
from sepia_amd import hip

# The reference's src/sepia_gpu.h function names (30), which a drop-in must keep.
REFERENCE_ABI = {
    "sepia_gpu_available", "sepia_gpu_init", "sepia_gpu_shutdown", "sepia_gpu_device_name",
    "sepia_gpu_wrap_mmap", "sepia_gpu_alloc", "sepia_gpu_free", "sepia_gpu_host_ptr", "sepia_gpu_gpu_addr",
    "sepia_gpu_selftest_touch", "sepia_gpu_begin", "sepia_gpu_flush", "sepia_gpu_end", "sepia_gpu_rmsnorm",
    "sepia_gpu_matvec", "sepia_gpu_silu_mul", "sepia_gpu_add", "sepia_gpu_softmax", "sepia_gpu_sconv",
    "sepia_gpu_matvec_q", "sepia_gpu_dequant_rows", "sepia_gpu_rel_project", "sepia_gpu_banded_attn",
    "sepia_gpu_matvec_off", "sepia_gpu_rmsnorm_off", "sepia_gpu_sconv_off", "sepia_gpu_rel_project_off",
    "sepia_gpu_copy", "sepia_gpu_scale", "sepia_gpu_sconv_hist_roll",
}

HAVE_GPU = os.path.exists("/dev/kfd") and os.access("/dev/kfd", os.R_OK)


@pytest.fixture(scope="module")
def lib():
    return hip.load()


def test_reference_abi_declared():
    declared = hip.declared_symbols()
    assert len(REFERENCE_ABI) == 30
    assert REFERENCE_ABI <= declared


def test_every_declared_symbol_exported(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", hip.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\bT (sepia_\w+)", out))
    missing = hip.declared_symbols() - exported
    assert not missing, missing
    for name in hip.declared_symbols():
        assert hasattr(lib, name)
    assert set(hip.PROTOTYPES) == hip.declared_symbols()


def test_code_object_has_every_kernel():
    """The host looks kernels up by name; each one it names must be in the code object."""
    src = open(os.path.join(ROOT, "sepia_amd", "csrc", "sepia_hip.c")).read()
    names = re.findall(r'"(sepia_[a-z0-9_]+)"', src.split("k_names[K_COUNT]")[1].split("};")[0])
    blob = open(hip.HSACO_PATH, "rb").read()
    for n in names:
        assert (n + ".kd").encode() in blob, n


def _run_isolated(code):
    """Run code in a fresh interpreter (the library keeps process-wide state)."""
    return subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, cwd=ROOT, timeout=120)


@pytest.mark.skipif(HAVE_GPU, reason="checks the no-device path")
def test_no_device_error_convention():
    code = r'''
import ctypes
from sepia_amd import hip
L = hip.load()
assert L.sepia_gpu_available() == 0
assert L.sepia_gpu_init(b"") == 0
assert L.sepia_gpu_init(hip.LIB_DIR.encode()) == 0
assert L.sepia_gpu_device_name() is None
assert L.sepia_gpu_alloc(16, 0) is None
assert L.sepia_gpu_wrap_mmap(None, 16) is None
assert L.sepia_gpu_begin() == 0
assert L.sepia_gpu_end() == 0
assert L.sepia_gpu_flush() == 0
assert L.sepia_gpu_matvec_q(12, None, 0, None, None, 4, 256) == 0
assert L.sepia_gpu_dequant_rows(12, None, 0, None, 256) == 0
assert L.sepia_gpu_host_ptr(None) is None
assert L.sepia_gpu_gpu_addr(None) == 0
L.sepia_gpu_free(None)
L.sepia_gpu_shutdown()
assert L.sepia_hip_stream() is None
print("ok")
'''
    r = _run_isolated(code)
    assert r.returncode == 0, r.stderr
    assert r.stdout.strip() == "ok"
    assert "sepia: hip:" in r.stderr


def test_struct_layout_matches_header(tmp_path):
    """ctypes mirrors of the extension structs agree with the C compiler's layout."""
    c = tmp_path / "lay.c"
    c.write_text(r'''
#include <stdio.h>
#include <stddef.h>
#include "sepia_hip_ext.h"
int main(void) {
    printf("%zu %zu %zu %zu %zu %zu\n", sizeof(SepiaExpertTensor), sizeof(SepiaMoeLayerDesc),
           offsetof(SepiaMoeLayerDesc, router_w), offsetof(SepiaMoeLayerDesc, gate),
           offsetof(SepiaMoeLayerDesc, s_down), offsetof(SepiaExpertTensor, ggml_type));
    return 0;
}''')
    exe = tmp_path / "lay"
    subprocess.run(["gcc", "-std=c11", "-I" + hip.INCLUDE_DIR, "-o", str(exe), str(c)], check=True)
    got = list(map(int, subprocess.run([str(exe)], capture_output=True, text=True).stdout.split()))
    import ctypes
    exp = [ctypes.sizeof(hip.ExpertTensor), ctypes.sizeof(hip.MoeLayerDesc), hip.MoeLayerDesc.router_w.offset,
           hip.MoeLayerDesc.gate.offset, hip.MoeLayerDesc.s_down.offset, hip.ExpertTensor.ggml_type.offset]
    assert got == exp
