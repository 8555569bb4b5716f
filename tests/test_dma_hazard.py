"""No vector memory instruction reads an SGPR that a VALU instruction wrote
fewer than 5 wait states before it.

On gfx9 a VMEM instruction (global_*, buffer_*, flat_*, scratch_*) that
reads an SGPR -- its address base, or soffset -- needs 5 wait states after
a VALU instruction that wrote that SGPR (v_readfirstlane, v_readlane, a
v_cmp or carry-out with an SGPR destination). The compiler's hazard
recognizer inserts them for the instructions it emits, but not around an
asm statement: the LDS DMA helpers (kernels/mq.h mq_dma16, kernels/prefill.h
pf_dma16, pf_dma4) are asm whose base the compiler may have just moved from
VGPRs with v_readfirstlane, so they carry their own s_nop (SEPIA_DMA_WAIT).
With too few, the DMA reads a stale base and faults the GPU.

This test disassembles the built gfx950 code object with llvm-objdump and
scans every kernel, counting wait states as instructions issued (s_nop N:
N + 1) in program order; a write stays in the window across branches,
which can only report more. CPU only: it reads the build output, nothing
runs on a GPU.
"""
import os
import re
import subprocess

import pytest

from conftest import ROOT

LLVM = "/opt/rocm/llvm/bin"
HSACO = os.path.join(ROOT, "sepia_amd", "lib", "sepia_kernels.hsaco")
VMEM = re.compile(r"(global|buffer|flat|scratch)_")
NEED = 5


def sgprs(tok):
    m = re.match(r"s\[(\d+):(\d+)\]$", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"s(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def valu_sgpr_writes(op, args):
    if op.startswith(("v_readfirstlane", "v_readlane")):
        return sgprs(args[0])
    if op.startswith("v_cmp") and args and args[0].startswith("s"):
        return sgprs(args[0])
    # VOP3b carry-out / scale destinations: v_add_co_u32 v, s[..], ...
    if len(args) > 1 and re.match(r"v_(add|sub|addc|subb|mad_u64|mad_i64|div_scale)", op):
        return sgprs(args[1])
    return set()


def scan(text):
    """{kernel: [(instruction, wait states)]} of the hazards in a disassembly."""
    hits, func, recent = {}, None, []
    for line in text.split("\n"):
        m = re.match(r"^[0-9a-f]+ <([^>]+)>:$", line)
        if m:
            func, recent = m.group(1), []
            continue
        ins = line.split("//")[0].strip()
        if not ins or ins.endswith(":"):
            continue
        op = ins.split()[0]
        args = [a.strip().split()[0] for a in ins[len(op):].split(",") if a.strip()]
        if VMEM.match(op):
            read = set().union(*[sgprs(a) for a in args[1:]]) if len(args) > 1 else set()
            for regs, ws in recent:
                if regs & read and ws < NEED:
                    hits.setdefault(func, []).append((ins, ws))
        n = int(re.match(r"s_nop\s+(\S+)", ins).group(1), 0) + 1 if op == "s_nop" else 1
        recent = [(r, w + n) for r, w in recent if w + n < NEED]
        if op.startswith("v_"):
            w = valu_sgpr_writes(op, args)
            if w:
                recent.append((w, 0))
    return hits


def test_scanner_finds_the_hazard():
    """The scan itself: a v_readfirstlane of the base one wait state before
    the DMA is found; five wait states are not."""
    bad = ("0000 <k>:\n\tv_readfirstlane_b32 s11, v17\n\tv_readfirstlane_b32 s10, v18\n\ts_nop 0\n"
           "\tglobal_load_lds_dwordx4 v2, s[10:11]\n")
    good = bad.replace("s_nop 0", "s_nop 4")
    other = bad.replace("s[10:11]", "s[20:21]")
    # s11 two wait states before the DMA, s10 one
    assert scan(bad) == {"k": [("global_load_lds_dwordx4 v2, s[10:11]", 2), ("global_load_lds_dwordx4 v2, s[10:11]", 1)]}
    assert scan(good) == {} and scan(other) == {}


@pytest.mark.skipif(not os.path.exists(HSACO), reason="code object not built")
def test_no_vmem_reads_a_fresh_valu_sgpr(tmp_path):
    co = str(tmp_path / "gfx950.co")
    subprocess.run([os.path.join(LLVM, "clang-offload-bundler"), "--unbundle", "--type=o",
                    "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", "--input=" + HSACO, "--output=" + co],
                   check=True, capture_output=True)
    dis = subprocess.run([os.path.join(LLVM, "llvm-objdump"), "-d", "--no-show-raw-insn", co], check=True,
                         capture_output=True, text=True).stdout
    assert dis.count("global_load_lds_dwordx4") > 1000, "the LDS DMA kernels are missing from the scan"
    hits = scan(dis)
    assert not hits, {k: v[:3] for k, v in hits.items()}
