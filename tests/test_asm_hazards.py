"""The inline-assembly loads of the HIP sources, checked in the gfx950 code
the build produces.  Two hazards that the compiler cannot see, because
inline assembly is opaque to it:

1. A vector memory instruction may read an SGPR only 5 wait states after a
   VALU instruction wrote it (v_readlane restoring a spilled SGPR,
   v_readfirstlane, a v_cmp mask).  The compiler pads the loads it generates
   but not inline assembly; a load that reads a stale buffer descriptor
   fetches from the wrong place.  Every vector memory instruction that comes
   from inline assembly is checked against the VALU SGPR writes before it
   (in program order, counting s_nop N as N + 1 wait states).

2. A load issued from inline assembly is not tracked by the compiler: it
   treats the destination registers as written when the statement ends,
   while the data arrives later.  Until an s_waitcnt vmcnt(N) retires the
   load (N smaller than the number of loads issued after it: a wave's loads
   complete in order), no instruction may read or write those registers; a
   late load would overwrite a value the compiler put there, or an
   instruction would read stale data.  This is checked by a dataflow over
   each kernel's control-flow graph: the state at an instruction is every
   untracked load that may still be in flight there, with the fewest loads
   issued after it on any path that reaches it; a wait retires the loads it
   covers on every path.  Direct-to-LDS copies (``... lds``) write no
   registers; they and the compiler's own loads count as loads issued after.
   Stores and atomics without return are not counted: they may complete out
   of order with the loads, so only loads make a wait cover an older load.
"""

import re
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

from tinygiant_amd import build as B

# every source whose kernels contain inline assembly
SOURCES = ["tg_grouped.hip", "tg_grouped_k.hip", "tg_head.hip", "tg_decode.hip", "tg_decode_mx.hip", "tg_attn.hip"]
WAIT_STATES = 5
VMEM = ("buffer_", "global_", "flat_", "scratch_")
VMEM_LOAD = ("buffer_load", "global_load", "flat_load", "scratch_load")
MAX_VMCNT = 63


def _sgprs(text):
    out = set()
    for m in re.finditer(r"\bs\[(\d+):(\d+)\]|\bs(\d+)\b", text):
        if m.group(3):
            out.add(int(m.group(3)))
        else:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    return out


def _vregs(text):
    """VGPRs and AGPRs named in an operand string, as ('v' | 'a', index)."""
    out = set()
    for m in re.finditer(r"\b([va])\[(\d+):(\d+)\]|\b([va])(\d+)\b", text):
        if m.group(1):
            out.update((m.group(1), r) for r in range(int(m.group(2)), int(m.group(3)) + 1))
        else:
            out.add((m.group(4), int(m.group(5))))
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


def _lines(asm_text):
    """(line number, instruction, from inline asm) of every instruction."""
    out, inasm = [], False
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
        out.append((n, t.split(";")[0].strip(), inasm))
    return out


def scan(asm_text):
    """(line, load, writer) of every inline-asm vector memory instruction that
    reads an SGPR a VALU instruction wrote fewer than 5 wait states before."""
    instrs = _lines(asm_text)
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


# ---- in-flight registers of untracked loads ----

def _functions(asm_text):
    """(name, body) per function; body items are ('label', name) or
    ('ins', text, from inline asm, line number)."""
    fn, body, inasm = None, [], False
    for n, line in enumerate(asm_text.splitlines(), 1):
        s = line.strip()
        m = re.match(r"^([A-Za-z_$][\w$.]*):", line)
        if m and not m.group(1).startswith(".L"):
            if fn:
                yield fn, body
            fn, body = m.group(1), []
            continue
        if fn is None:
            continue
        if s.startswith(".Lfunc_end"):
            yield fn, body
            fn, body = None, []
            continue
        if s == ";;#ASMSTART":
            inasm = True
            continue
        if s == ";;#ASMEND":
            inasm = False
            continue
        m = re.match(r"^(\.L[\w$.]+):", s)
        if m:
            body.append(("label", m.group(1)))
            continue
        if not s or s[0] in ";.":
            continue
        body.append(("ins", s.split(";")[0].strip(), inasm, n))
    if fn:
        yield fn, body


def _vmcnt(ins):
    """The vmcnt an s_waitcnt waits for, or None (no vector-memory wait)."""
    if ins.split()[0] != "s_waitcnt":
        return None
    m = re.search(r"vmcnt\((\d+)\)", ins)
    if m:
        return int(m.group(1))
    m = re.match(r"s_waitcnt\s+(0x[0-9a-fA-F]+|\d+)\s*$", ins)
    if m:   # raw simm16: vmcnt is bits 3:0 and 15:14
        v = int(m.group(1), 0)
        return (v & 0xF) | (((v >> 14) & 3) << 4)
    return None


def _is_lds_copy(ins):
    return ins.rstrip().endswith(" lds") or "_lds_" in ins.split()[0]


def inflight_touches(fn, body):
    """(load line, load, touching line, touching instruction) for every
    instruction that may read or write a register of an untracked load still
    in flight on some path to it."""
    ins, labels = [], {}
    for item in body:
        if item[0] == "label":
            labels[item[1]] = len(ins)
        else:
            ins.append(item[1:])
    n = len(ins)
    if n == 0:
        return []

    def succ(i):
        op, _, rest = ins[i][0].partition(" ")
        if op in ("s_endpgm", "s_setpc_b64", "s_trap"):
            out = []
        elif op == "s_branch":
            out = [labels[rest.strip()]]
        elif op.startswith("s_cbranch_"):
            out = [labels[rest.strip()], i + 1]
        else:
            out = [i + 1]
        return [s for s in out if s < n]

    dests = {}
    state = {0: {}}
    work = [0]
    found = {}
    while work:
        i = work.pop()
        st = dict(state[i])
        t, a, line = ins[i]
        op, _, rest = t.partition(" ")
        w = _vmcnt(t)
        if w is not None:
            st = {k: after for k, after in st.items() if after < w}
        else:
            mention = _vregs(rest)
            for k in st:
                if dests[k] & mention:
                    found.setdefault((k, i), None)
        if op.startswith(VMEM_LOAD):
            st = {k: min(MAX_VMCNT + 1, after + 1) for k, after in st.items()}
            if a and not _is_lds_copy(t):
                dests[i] = _vregs(rest.split(",")[0])
                st[i] = 0
        for s in succ(i):
            old = state.get(s)
            if old is None:
                state[s] = st
                work.append(s)
                continue
            new, changed = dict(old), False
            for k, after in st.items():
                if k not in new or after < new[k]:
                    new[k] = after
                    changed = True
            if changed:
                state[s] = new
                work.append(s)
    return [(ins[k][2], ins[k][0], ins[i][2], ins[i][0]) for (k, i) in sorted(found)]


def scan_inflight(asm_text):
    return [(fn, *hit) for fn, body in _functions(asm_text) for hit in inflight_touches(fn, body)]


def _kernel(body):
    return "\t.text\n_Z4testv:\n" + body + "\t.Lfunc_end0:\n"


def test_scan_finds_the_hazard():
    """The SGPR check itself: a descriptor restored by v_readlane two
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


# The loop exit of the row-group loop of the q6_K head as one build had it:
# the loads of the group past the last go out in the loop, the loop is left
# with them in flight, and the exit block computes a value into one of their
# registers (v35 of v[34:37]) before the wait that covers them.  A late load
# then overwrote it.
HEAD_EXIT = """
\t;;#ASMSTART
\tbuffer_load_dwordx4 v[40:43], v83, s[28:31], 0 offen offset:16
\tbuffer_load_dword v82, v60, s[28:31], 0 offen offset:206
\t;;#ASMEND
.LBB6_40:
\t;;#ASMSTART
\ts_nop 4
\tbuffer_load_dwordx4 v[34:37], v83, s[28:31], 0 offen offset:16
\tbuffer_load_dword v81, v60, s[28:31], 0 offen offset:206
\t;;#ASMEND
\t;;#ASMSTART
\ts_waitcnt vmcnt(2)
\t;;#ASMEND
\tv_add_u32_e32 v90, v40, v82
\ts_cmp_lt_i32 s4, s5
\ts_cbranch_scc0 .LBB6_42
\t;;#ASMSTART
\ts_nop 4
\tbuffer_load_dwordx4 v[40:43], v83, s[28:31], 0 offen offset:16
\tbuffer_load_dword v82, v60, s[28:31], 0 offen offset:206
\t;;#ASMEND
\t;;#ASMSTART
\ts_waitcnt vmcnt(2)
\t;;#ASMEND
\tv_add_u32_e32 v90, v34, v81
\ts_cmp_lt_i32 s4, s5
\ts_cbranch_scc1 .LBB6_40
\ts_branch .LBB6_44
.LBB6_42:
\tv_bfe_u32 v35, v0, 1, 3
\t;;#ASMSTART
\ts_waitcnt vmcnt(0)
\t;;#ASMEND
\tv_lshlrev_b32_e32 v35, 3, v35
.LBB6_44:
\ts_endpgm
"""


def test_inflight_register_write_is_flagged():
    """The head's exit case: the write of v35 before the covering wait is
    flagged (once, against the load that owns v35); with the wait first, or
    the value put in another register, nothing is."""
    hits = scan_inflight(_kernel(HEAD_EXIT))
    assert [(h[2], h[4]) for h in hits] == [
        ("buffer_load_dwordx4 v[34:37], v83, s[28:31], 0 offen offset:16", "v_bfe_u32 v35, v0, 1, 3")]
    fixed = HEAD_EXIT.replace("\tv_bfe_u32 v35, v0, 1, 3\n\t;;#ASMSTART\n\ts_waitcnt vmcnt(0)\n\t;;#ASMEND\n",
                              "\t;;#ASMSTART\n\ts_waitcnt vmcnt(0)\n\t;;#ASMEND\n\tv_bfe_u32 v35, v0, 1, 3\n")
    assert scan_inflight(_kernel(fixed)) == []
    other = HEAD_EXIT.replace("v_bfe_u32 v35", "v_bfe_u32 v90").replace("v_lshlrev_b32_e32 v35, 3, v35",
                                                                       "v_lshlrev_b32_e32 v90, 3, v90")
    assert scan_inflight(_kernel(other)) == []


def test_inflight_reads_counts_and_paths():
    """Reads are flagged as well as writes; a wait covers a load only when
    enough loads (the compiler's and direct-to-LDS copies included) were
    issued after it on every path; a path that skips a wait keeps the load
    in flight."""
    body = """
\t;;#ASMSTART
\tbuffer_load_dwordx4 v[4:7], v1, s[8:11], 0 offen
\t;;#ASMEND
\tbuffer_load_dword v20, v2, s[8:11], 0 offen
\t;;#ASMSTART
\tbuffer_load_dwordx4 v3, s[8:11], 0 offen lds
\ts_waitcnt vmcnt(2)
\t;;#ASMEND
\tv_add_u32_e32 v9, v5, v6
\ts_endpgm
"""
    assert scan_inflight(_kernel(body)) == []            # two loads after it: vmcnt(2) covers it
    under = body.replace("vmcnt(2)", "vmcnt(3)")
    hits = scan_inflight(_kernel(under))
    assert len(hits) == 1 and hits[0][4] == "v_add_u32_e32 v9, v5, v6"   # a read of v5, v6
    # a store after the load does not make the wait cover it
    store = body.replace("\tbuffer_load_dword v20, v2, s[8:11], 0 offen\n",
                         "\tbuffer_store_dword v20, v2, s[8:11], 0 offen\n")
    assert len(scan_inflight(_kernel(store))) == 1
    # the wait skipped on one path
    branchy = """
\t;;#ASMSTART
\tbuffer_load_dwordx4 v[4:7], v1, s[8:11], 0 offen
\t;;#ASMEND
\ts_cbranch_scc1 .LBB0_2
\t;;#ASMSTART
\ts_waitcnt vmcnt(0)
\t;;#ASMEND
.LBB0_2:
\tv_mov_b32_e32 v4, 0
\ts_endpgm
"""
    hits = scan_inflight(_kernel(branchy))
    assert len(hits) == 1 and hits[0][4] == "v_mov_b32_e32 v4, 0"
    # a loop that re-issues the load each turn and waits for it before the
    # back edge is clean; without the wait the re-issue itself is flagged
    loop = """
.LBB0_1:
\t;;#ASMSTART
\tbuffer_load_dwordx4 v[4:7], v1, s[8:11], 0 offen
\ts_waitcnt vmcnt(0)
\t;;#ASMEND
\tv_add_u32_e32 v1, v4, v1
\ts_cbranch_scc1 .LBB0_1
\ts_endpgm
"""
    assert scan_inflight(_kernel(loop)) == []
    assert len(scan_inflight(_kernel(loop.replace("\ts_waitcnt vmcnt(0)\n", "")))) >= 1


@pytest.fixture(scope="module")
def device_asm(tmp_path_factory):
    if not shutil.which(B.HIPCC) and not Path(B.HIPCC).exists():
        pytest.skip("hipcc not installed")
    tmp = tmp_path_factory.mktemp("asm")
    flags = [f for f in B.HIP_FLAGS if f not in ("-fPIC",)]

    def one(src):
        out = tmp / (src + ".s")
        cmd = [B.HIPCC, *flags, *B.HIP_EXTRA.get(src, []), "--cuda-device-only", "-S", "-I", str(B.CSRC),
               str(B.CSRC / src), "-o", str(out)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-2000:]
        return src, out.read_text()

    with ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        return dict(ex.map(one, SOURCES))


def test_inline_asm_loads_are_padded(device_asm):
    problems = [(src, b) for src, text in device_asm.items() for b in scan(text)]
    assert not problems, problems[:5]


def test_no_register_of_an_untracked_load_is_touched_in_flight(device_asm):
    problems = [(src, h) for src, text in device_asm.items() for h in scan_inflight(text)]
    assert not problems, problems[:5]
