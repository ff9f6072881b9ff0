"""Device assembly scan (CPU, no GPU): no 12- or 16-byte vector-memory store is followed within two
instructions by a VALU write of its data registers.

gfx950 needs two wait states between such a store and a VALU overwrite of its data; the compiler
inserts them (s_nop 1) for buffer stores with a constant scalar offset and for global stores, but
not for buffer stores whose scalar offset is a register. A partial-tile store in that form, with a
VALU write of its first data register right behind it, put that write's value in memory in place of
the store's first word (one column in eight of some K-split tiles came out wrong). The kernels keep
every buffer store's scalar offset at 0 (buf_store16); this scan catches the pattern in any source."""
import os
import re
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "..", "hilbert-pruned-8b_amd", "csrc")
ASM = os.path.join(HERE, "..", "hilbert-pruned-8b_amd", "_build", "asm")

STORE = re.compile(r"^\s*(?:buffer_store_(?:dwordx3|dwordx4|b96|b128)\s+"
                   r"|(?:global|flat)_store_(?:dwordx3|dwordx4|b96|b128)\s+v(?:\[\d+:\d+\]|\d+),\s*)v\[(\d+):(\d+)\]")
VALU = re.compile(r"^\s*(v_\S+)\s+v(?:(\d+)|\[(\d+):(\d+)\])\b")
NOT_VGPR_DEF = ("v_cmp", "v_cmpx", "v_readfirstlane", "v_readlane")


def hazards(lines):
    """(store, next) pairs: a wide store whose data registers a VALU instruction writes within the
    next two instructions, with no s_nop in between."""
    code = [l.strip() for l in lines if l.strip() and not l.strip().startswith((";", ".", "//"))
            and not l.strip().endswith(":")]
    out = []
    for i, line in enumerate(code):
        m = STORE.match(line)
        if not m:
            continue
        lo, hi = int(m.group(1)), int(m.group(2))
        for nxt in code[i + 1:i + 3]:
            if nxt.startswith("s_nop"):
                break
            v = VALU.match(nxt)
            if v and not v.group(1).startswith(NOT_VGPR_DEF):
                a = int(v.group(2) or v.group(3))
                b = int(v.group(2) or v.group(4))
                if a <= hi and b >= lo:
                    out.append((line, nxt))
    return out


def test_scanner_flags_the_pattern():
    bad = ["buffer_store_dwordx4 v[2:5], v1, s[4:7], s1 offen sc1", "v_or_b32_e32 v2, 0x200, v0"]
    ok = ["buffer_store_dwordx4 v[2:5], v1, s[4:7], 0 offen sc1", "s_nop 1", "v_or_b32_e32 v2, 0x200, v0"]
    addr = ["global_store_dwordx4 v[2:3], v[12:15], off", "v_mov_b32_e32 v2, 0"]
    far = ["buffer_store_dwordx4 v[2:5], v1, s[4:7], s1 offen sc1", "s_waitcnt lgkmcnt(0)",
           "buffer_store_dwordx4 v[6:9], v1, s[4:7], s1 offen offset:16 sc1", "v_mov_b32_e32 v2, 0"]
    assert len(hazards(bad)) == 1
    assert hazards(ok) == [] and hazards(addr) == [] and hazards(far) == []
    assert len(hazards(["global_store_dwordx4 v[2:3], v[12:15], off", "v_mov_b32_e32 v13, 0"])) == 1


@pytest.mark.timeout(900)
def test_no_store_data_hazard_in_device_code():
    if subprocess.run(["which", "hipcc"], capture_output=True).returncode and not os.path.exists("/opt/rocm/bin/hipcc"):
        pytest.skip("hipcc not available")
    jobs = str(min(8, os.cpu_count() or 1))
    subprocess.run(["make", "-s", "-C", CSRC, "asm", "-j" + jobs], check=True, capture_output=True)
    files = sorted(f for f in os.listdir(ASM) if f.endswith(".s"))
    assert len(files) >= 10
    found = {}
    for f in files:
        with open(os.path.join(ASM, f)) as fh:
            h = hazards(fh.readlines())
        if h:
            found[f] = h[:3]
    assert not found, found
