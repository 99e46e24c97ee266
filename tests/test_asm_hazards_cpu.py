"""The LDS-DMA issue paths obey the gfx9 wait-state rules that the compiler cannot add itself.

The kernels issue ``global_load_lds_dwordx4`` from inline asm (so that the compiler's
wait-count pass does not serialise ring reads behind it), and the hazard recognizer does not
look inside inline asm. Two rules then fall to the source, and this test checks them on the
device assembly of every kernel source, built here for gfx950 (no GPU needed):

* a vector-ALU write of an SGPR (``v_readfirstlane_b32`` of a DMA base address) needs 5 wait
  states before a memory instruction reads that SGPR -- a stale base reads a wild address;
* a scalar write of M0 needs 1 wait state before an LDS DMA reads M0.
"""

from __future__ import annotations

import glob
import os
import re
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "mini-sglang_amd"))
import build  # noqa: E402  (mini-sglang_amd/build.py: the flags the library is built with)

HIPCC = build.HIPCC
SOURCES = sorted(glob.glob(os.path.join(build.CSRC, "*.hip")))


def _device_asm(src: str, out_dir: str) -> str:
    out = os.path.join(out_dir, os.path.basename(src) + ".s")
    cmd = [HIPCC, *build.FLAGS, *build.SOURCE_FLAGS.get(os.path.basename(src), []), "--cuda-device-only", "-S",
           src, "-o", out]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    with open(out) as f:
        return f.read()


def _instructions(asm: str):
    out = []
    for line in asm.splitlines():
        t = line.split(";")[0].strip()
        if t and not t.startswith(".") and not t.endswith(":"):
            out.append(t)
    return out


def _sgprs(text: str) -> set:
    regs = set()
    for m in re.finditer(r"s\[(\d+):(\d+)\]", text):
        regs.update(f"s{r}" for r in range(int(m.group(1)), int(m.group(2)) + 1))
    regs.update(f"s{m.group(1)}" for m in re.finditer(r"\bs(\d+)\b", text))
    return regs


def find_hazards(asm: str):
    """(VALU SGPR write -> VMEM read within 5 wait states, SALU M0 write -> LDS DMA) instances."""
    ins = _instructions(asm)
    sgpr_hazards, m0_hazards = [], []
    for i, line in enumerate(ins):
        op = line.split()[0]
        if not op.startswith(("global_", "buffer_", "flat_", "scratch_")):
            continue
        reads = _sgprs(" ".join(line.split()[1:]))
        waits = 0
        for j in range(i - 1, max(-1, i - 12), -1):
            prev = ins[j]
            pop = prev.split()[0]
            if pop.startswith("v_") and len(prev.split()) > 1 and _sgprs(prev.split()[1].rstrip(",")) & reads:
                if waits < 5:
                    sgpr_hazards.append((prev, line))
                break
            waits += int(prev.split()[1], 0) + 1 if pop == "s_nop" else 1
            if waits >= 5:
                break
        if "_lds_" in op:
            prev = ins[i - 1]
            if prev.startswith("s_") and not prev.startswith("s_nop") and prev.split()[1].rstrip(",") == "m0":
                m0_hazards.append((prev, line))
    return sgpr_hazards, m0_hazards


def test_checker_catches_a_readfirstlane_feeding_a_dma():
    asm = """
        v_readfirstlane_b32 s1, v3
        v_readfirstlane_b32 s0, v2
        s_mov_b32 m0, s6
        global_load_lds_dwordx4 v253, s[0:1]
        s_nop 4
        s_add_i32 m0, s6, 0x1000
        s_nop 0
        global_load_lds_dwordx4 v252, s[0:1]
    """
    sgpr, m0 = find_hazards(asm)
    assert len(sgpr) == 1 and "v_readfirstlane_b32 s0" in sgpr[0][0]
    assert len(m0) == 1 and "s_mov_b32 m0" in m0[0][0]


@pytest.mark.skipif(shutil.which(HIPCC) is None and not os.path.exists(HIPCC), reason="hipcc not available")
@pytest.mark.parametrize("src", [os.path.basename(s) for s in SOURCES])
def test_no_dma_hazards(src, tmp_path):
    sgpr, m0 = find_hazards(_device_asm(os.path.join(build.CSRC, src), str(tmp_path)))
    assert not sgpr, f"VALU-written SGPR read by a memory instruction too early: {sgpr[:3]}"
    assert not m0, f"M0 written right before an LDS DMA: {m0[:3]}"
