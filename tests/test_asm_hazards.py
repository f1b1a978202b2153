"""The inline-assembly loads of the HIP sources, checked in the gfx950 code
the build produces.

A vector memory instruction may read an SGPR only 5 wait states after a VALU
instruction wrote it (v_readlane restoring a spilled SGPR, v_readfirstlane,
a v_cmp mask).  The compiler pads the loads it generates but not inline
assembly, which is opaque to its hazard pass; a load that reads a stale
buffer descriptor fetches from the wrong place.  The sources pad each asm
load themselves; this test compiles them to device assembly with the build's
own flags and checks every vector memory instruction that comes from inline
assembly against the VALU SGPR writes before it (in program order, counting
s_nop N as N + 1 wait states).
"""

import re
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

from tinygiant_amd import build as B

SOURCES = ["tg_grouped.hip", "tg_grouped_k.hip", "tg_head.hip", "tg_decode.hip", "tg_decode_mx.hip", "tg_attn.hip"]
WAIT_STATES = 5
VMEM = ("buffer_", "global_", "flat_", "scratch_")


def _sgprs(text):
    out = set()
    for m in re.finditer(r"\bs\[(\d+):(\d+)\]|\bs(\d+)\b", text):
        if m.group(3):
            out.add(int(m.group(3)))
        else:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    return out


def _valu_sgpr_writes(ins):
    op, _, rest = ins.partition(" ")
    if not op.startswith("v_") or op.startswith("v_mfma"):
        return set()
    ops = [o.strip() for o in rest.split(",")]
    w = _sgprs(ops[0]) if ops else set()
    if ("_co_" in op or "div_scale" in op) and len(ops) > 1:
        w |= _sgprs(ops[1])   # the carry-out / scale-condition SGPR result
    return w


def scan(asm_text):
    """(line, load, writer) of every inline-asm vector memory instruction that
    reads an SGPR a VALU instruction wrote fewer than 5 wait states before."""
    instrs, inasm = [], False
    for n, line in enumerate(asm_text.splitlines(), 1):
        t = line.strip()
        if t == ";;#ASMSTART":
            inasm = True
            continue
        if t == ";;#ASMEND":
            inasm = False
            continue
        if not t or t[0] in ";." or t.endswith(":"):
            continue
        instrs.append((n, t.split(";")[0].strip(), inasm))
    bad = []
    for i, (n, t, a) in enumerate(instrs):
        if not (a and t.startswith(VMEM)):
            continue
        reads = _sgprs(t.partition(" ")[2])
        ws = 0
        for j in range(i - 1, -1, -1):
            if ws >= WAIT_STATES:
                break
            t2 = instrs[j][1]
            if _valu_sgpr_writes(t2) & reads:
                bad.append((n, t, t2))
                break
            parts = t2.split()
            ws += int(parts[1]) + 1 if parts[0] == "s_nop" else 1
    return bad


def test_scan_finds_the_hazard():
    """The scanner itself: a descriptor restored by v_readlane two
    instructions before an asm load is flagged; with s_nop 4 in between it
    is not; a compiler-generated load is not the check's business."""
    hazard = """
\tv_readlane_b32 s14, v219, 39
\tv_readlane_b32 s15, v219, 40
\t;;#ASMSTART
\tbuffer_load_dword v166, v18, s[12:15], 0 offen
\t;;#ASMEND
"""
    padded = hazard.replace("\t;;#ASMSTART\n", "\t;;#ASMSTART\n\ts_nop 4\n")
    compiler = hazard.replace("\t;;#ASMSTART\n", "").replace("\t;;#ASMEND\n", "")
    other = hazard.replace("s[12:15]", "s[16:19]")
    assert len(scan(hazard)) == 1
    assert scan(padded) == []
    assert scan(compiler) == []
    assert scan(other) == []
    # four wait states are one short
    short = hazard.replace("\t;;#ASMSTART\n", "\t;;#ASMSTART\n\ts_nop 2\n")
    assert len(scan(short)) == 1


@pytest.mark.skipif(not shutil.which(B.HIPCC) and not Path(B.HIPCC).exists(), reason="hipcc not installed")
def test_inline_asm_loads_are_padded(tmp_path):
    flags = [f for f in B.HIP_FLAGS if f not in ("-fPIC",)]

    def one(src):
        out = tmp_path / (src + ".s")
        cmd = [B.HIPCC, *flags, "--cuda-device-only", "-S", "-I", str(B.CSRC), str(B.CSRC / src), "-o", str(out)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-2000:]
        return src, scan(out.read_text())

    with ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        results = list(ex.map(one, SOURCES))
    problems = [(src, b) for src, bad in results for b in bad]
    assert not problems, problems[:5]
