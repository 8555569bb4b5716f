"""No bounded spin wait reloads anything through the vector memory path.

The kernels' bounded waits (an LDS counter polled with s_sleep between
polls, bounded by s_memrealtime against the library's wait bound) must
not put a vector memory load (or a vmcnt wait) in the poll loop: under a
launch's weight stream such a load takes a loaded memory round trip, and
each poll then sees the counter that much late. The wait bound lives in
constant memory for this reason, read by one scalar load before the loop.

CPU only: the test disassembles the built gfx950 code object and checks
every poll loop, from its s_sleep to the loop's branch.
"""
import os
import re
import subprocess

import pytest

from conftest import ROOT

LLVM = "/opt/rocm/llvm/bin"
HSACO = os.path.join(ROOT, "sepia_amd", "lib", "sepia_kernels.hsaco")
VLOAD = re.compile(r"^(global_load|flat_load|buffer_load|global_atomic|flat_atomic)")


def poll_loop_loads(text):
    """[(kernel, instruction)] of vector loads or vmcnt waits between an
    s_sleep and the next branch."""
    bad, func, inside = [], None, False
    for line in text.split("\n"):
        m = re.match(r"^[0-9a-f]+ <([^>]+)>:$", line)
        if m:
            func, inside = m.group(1), False
            continue
        ins = line.split("//")[0].strip()
        if not ins:
            continue
        op = ins.split()[0]
        if op == "s_sleep":
            inside = True
            continue
        if not inside:
            continue
        if op.startswith("s_cbranch") or op == "s_branch":
            inside = False
        elif VLOAD.match(op) or (op == "s_waitcnt" and "vmcnt" in ins):
            bad.append((func, ins))
    return bad


def test_scanner_finds_a_load_in_a_poll_loop():
    loop = ("0000 <k>:\n\ts_sleep 1\n\ts_memrealtime s[38:39]\n\tglobal_load_dwordx2 v[4:5], v0, s[8:9]\n"
            "\ts_waitcnt vmcnt(0)\n\ts_cbranch_vccnz 65527\n")
    assert poll_loop_loads(loop) == [("k", "global_load_dwordx2 v[4:5], v0, s[8:9]"), ("k", "s_waitcnt vmcnt(0)")]
    good = loop.replace("\tglobal_load_dwordx2 v[4:5], v0, s[8:9]\n\ts_waitcnt vmcnt(0)\n", "\ts_waitcnt lgkmcnt(0)\n")
    assert poll_loop_loads(good) == []


@pytest.mark.skipif(not os.path.exists(HSACO), reason="code object not built")
def test_no_vector_load_in_a_poll_loop(tmp_path):
    co = str(tmp_path / "gfx950.co")
    subprocess.run([os.path.join(LLVM, "clang-offload-bundler"), "--unbundle", "--type=o",
                    "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", "--input=" + HSACO, "--output=" + co],
                   check=True, capture_output=True)
    dis = subprocess.run([os.path.join(LLVM, "llvm-objdump"), "-d", "--no-show-raw-insn", co], check=True,
                         capture_output=True, text=True).stdout
    assert dis.count("s_sleep") > 10, "the bounded waits are missing from the scan"
    bad = poll_loop_loads(dis)
    assert not bad, bad[:5]
