"""Checks on the gfx950 assembly of the attention kernels (CPU: hipcc cross-compiles).

The LDS-DMA helpers are inline asm that sets M0. Two properties keep them sound:
  * M0 is used by nothing but that asm (the compiler keeps no value in it);
  * no SCC value the compiler produced before an asm block that writes SCC is
    read after it. A 64-bit pointer increment split around an asm block that set
    M0 with s_add_u32 once lost its carry: a K/V buffer base 4 GiB off.
"""
import os
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "qwfn-hybrid_amd")
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

SCC_WRITERS = ("s_cmp", "s_add_u32", "s_sub_u32", "s_addc", "s_subb", "s_and_b", "s_or_b", "s_xor_b", "s_andn2",
               "s_orn2", "s_lshl", "s_lshr", "s_ashr", "s_bfe", "s_min", "s_max", "s_add_i32", "s_sub_i32", "s_addk",
               "s_bitcmp", "s_abs", "s_not", "s_nand", "s_nor", "s_xnor", "s_bcnt", "s_ff", "s_flbit", "s_quadmask",
               "s_wqm")
SCC_READERS = ("s_cselect", "s_cbranch_scc", "s_addc", "s_subb", "s_cmovk", "s_cmov")


def _op(line):
    t = line.strip()
    return t.split()[0] if t and not t.startswith((";", ".")) else ""


def asm_blocks(lines):
    """(start, end) line indices of each inline-asm block (ASMSTART .. ASMEND)."""
    out, start = [], None
    for i, l in enumerate(lines):
        if "ASMSTART" in l:
            start = i
        elif "ASMEND" in l and start is not None:
            out.append((start, i))
            start = None
    return out


def scc_carried_across(lines, blocks):
    """Blocks that write SCC while an SCC value written before them is read after."""
    inside = set()
    for a, b in blocks:
        inside.update(range(a, b + 1))
    bad = []
    for a, b in blocks:
        if not any(_op(lines[i]).startswith(SCC_WRITERS) for i in range(a + 1, b)):
            continue
        live = False
        for j in range(a - 1, -1, -1):                      # the last SCC writer before the block
            t = lines[j].strip()
            if t.startswith(".LBB") or _op(t).startswith(("s_branch", "s_cbranch")):
                break
            if j in inside:
                continue
            if _op(t).startswith(SCC_WRITERS):
                live = True
                break
        if not live:
            continue
        for k in range(b + 1, len(lines)):                  # is it read before it is written again?
            t = lines[k].strip()
            if t.startswith(".LBB"):
                break
            if k in inside:
                continue
            op = _op(t)
            if op.startswith(SCC_READERS):
                bad.append((a + 1, t))
                break
            if op.startswith(SCC_WRITERS) or op.startswith(("s_branch", "s_cbranch")):
                break
    return bad


@pytest.fixture(scope="module")
def fattn_asm():
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not available")
    with tempfile.TemporaryDirectory() as d:
        out = os.path.join(d, "fattn.s")
        subprocess.run([HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
                        "-packed-fp32-ops", "-I", os.path.join(PKG, "csrc"), "-I", os.path.join(ROOT, "include"),
                        "--cuda-device-only", "-S", os.path.join(PKG, "csrc", "fattn_q8_0.hip"), "-o", out],
                       check=True, capture_output=True, timeout=600)
        return open(out).read().split("\n")


def test_dma_asm_keeps_scc(fattn_asm):
    blocks = asm_blocks(fattn_asm)
    assert any("m0" in fattn_asm[a + 1] for a, _ in blocks), "the LDS-DMA asm sets M0"
    assert scc_carried_across(fattn_asm, blocks) == []


def test_m0_only_in_dma_asm(fattn_asm):
    inside = set()
    for a, b in asm_blocks(fattn_asm):
        inside.update(range(a, b + 1))
    uses = [l.strip() for i, l in enumerate(fattn_asm) if i not in inside and _op(l) and "m0" in l.split(";")[0]]
    assert uses == []


def test_scan_finds_a_split_carry():
    """The scan itself: a 64-bit add split around an SCC-writing asm block is found."""
    lines = ["\ts_add_u32 s16, s16, s18", "\t;;#ASMSTART", "\ts_add_u32 m0, s47, 0x1900",
             "\tbuffer_load_dwordx4 v150, s[4:7], 0 offen lds", "\t;;#ASMEND", "\ts_addc_u32 s17, s17, s19"]
    assert len(scc_carried_across(lines, asm_blocks(lines))) == 1
    lines[0] = "\ts_mov_b32 s16, s18"                        # no SCC writer before: nothing carried
    assert scc_carried_across(lines, asm_blocks(lines)) == []
