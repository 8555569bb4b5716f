"""sepia_amd -- MI355X-native quantized-weight hot path of SEPIA.

The product is libsepia_hip.so (sepia_amd/lib): a C host backend
(csrc/sepia_hip.c) implementing SEPIA's GPU ABI (include/sepia_gpu.h) over
hand-written gfx950 kernels (csrc/kernels, built into sepia_kernels.hsaco).
This package adds only the ctypes bindings used by tests and the benchmark
(hip.py) and the seeded synthetic-input generator (synth.py).
"""
import os
import subprocess

PKG = os.path.dirname(os.path.abspath(__file__))


def build():
    """Compile the code object and the host library in-tree (always rebuilds)."""
    subprocess.run(["make", "-s", "-B", "-C", PKG], check=True)
