"""The kernarg warm-up reads only inside each kernel's argument segment.

sepia_kernarg_warm<BYTES>() (kernels/common.h) touches every 64-byte line of
the first BYTES of the kernel's argument segment at entry. That is only
defined if BYTES does not exceed the segment, whose size the compiler
records per kernel in the code object's metadata (.kernarg_segment_size).
This test reads that metadata from the built gfx950 code object (unbundled
with clang-offload-bundler, notes read with llvm-readelf) and checks every
warm-up site of the kernel sources against the kernels it is compiled into.
CPU only: it reads the build output, nothing runs on a GPU.
"""
import os
import re
import subprocess

import pytest

from conftest import ROOT

LLVM = "/opt/rocm/llvm/bin"
HSACO = os.path.join(ROOT, "sepia_amd", "lib", "sepia_kernels.hsaco")
KDIR = os.path.join(ROOT, "sepia_amd", "csrc", "kernels")


def kernel_segments(tmp_path):
    """{kernel name: kernarg segment bytes} from the built code object."""
    co = str(tmp_path / "gfx950.co")
    subprocess.run([os.path.join(LLVM, "clang-offload-bundler"), "--unbundle", "--type=o",
                    "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", "--input=" + HSACO, "--output=" + co],
                   check=True, capture_output=True)
    notes = subprocess.run([os.path.join(LLVM, "llvm-readelf"), "--notes", co], check=True,
                           capture_output=True, text=True).stdout
    meta = notes[notes.index("amdhsa.kernels:"):]
    out = {}
    # one YAML map per kernel, each opening with "  - .agpr_count:"
    for block in re.split(r"\n  - (?=\.agpr_count:)", meta)[1:]:
        name = re.search(r"^    \.name:\s+(\S+)", block, flags=re.M)
        size = re.search(r"^    \.kernarg_segment_size:\s+(\d+)", block, flags=re.M)
        if name and size:
            out[name.group(1)] = int(size.group(1))
    return out


def warm_sites():
    """(kernel name or macro name prefix, is_prefix, BYTES) per warm-up call."""
    sites = []
    for fn in sorted(os.listdir(KDIR)):
        if not fn.endswith((".h", ".hip")):
            continue
        text = open(os.path.join(KDIR, fn)).read()
        for m in re.finditer(r"sepia_kernarg_warm<(\d+)>\s*\(\)", text):
            heads = list(re.finditer(r"void\s+(sepia_\w+?)(##\w+)?\s*\(", text[:m.start()]))
            assert heads, "%s: warm-up outside a kernel" % fn
            sites.append((heads[-1].group(1), bool(heads[-1].group(2)), int(m.group(1))))
    return sites


@pytest.mark.skipif(not os.path.exists(HSACO), reason="code object not built")
def test_kernarg_warm_within_segment(tmp_path):
    seg = kernel_segments(tmp_path)
    assert len(seg) > 50, sorted(seg)
    sites = warm_sites()
    assert len(sites) >= 4, sites
    for name, is_prefix, nbytes in sites:
        kernels = [k for k in seg if (k.startswith(name) if is_prefix else k == name)]
        assert kernels, "no kernel %s%s in the code object" % (name, "*" if is_prefix else "")
        for k in kernels:
            assert nbytes <= seg[k], "%s warms %d bytes of a %d-byte argument segment" % (k, nbytes, seg[k])
