"""The LDS-DMA issue paths obey the gfx9 wait-state rules that the compiler cannot add itself.

The kernels issue ``global_load_lds_dwordx4`` from inline asm (so that the compiler's
wait-count pass does not serialise ring reads behind it), and the hazard recognizer does not
look inside inline asm. Two rules then fall to the source, and this test checks them on the
device assembly of every kernel source, built here for gfx950 (no GPU needed):

* a vector-ALU write of an SGPR (``v_readfirstlane_b32`` of a DMA base address, a compare's
  lane mask, a carry-out) needs 5 wait states before a memory instruction reads that SGPR -- a
  stale base reads a wild address;
* a scalar write of M0 needs 1 wait state before an LDS DMA reads M0.

The check follows the control flow: each kernel's assembly is split into basic blocks (labels,
branches, ``s_endpgm``), and from every memory instruction it walks back over every path into
it -- fall-through, branch targets and loop back-edges -- until the wait states add up.
"""

from __future__ import annotations

import glob
import os
import re
import shutil
import subprocess
import sys
from typing import Dict, List, Set, Tuple

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "mini-sglang_amd"))
import build  # noqa: E402  (mini-sglang_amd/build.py: the flags the library is built with)

HIPCC = build.HIPCC
SOURCES = sorted(glob.glob(os.path.join(build.CSRC, "*.hip")))

VALU_SGPR_WAITS = 5  # VALU writes an SGPR -> a VMEM instruction reads it
M0_WAITS = 1  # SALU writes M0 -> an LDS DMA reads it


def _device_asm(src: str, out_dir: str) -> str:
    out = os.path.join(out_dir, os.path.basename(src) + ".s")
    cmd = [HIPCC, *build.FLAGS, *build.SOURCE_FLAGS.get(os.path.basename(src), []), "--cuda-device-only", "-S",
           src, "-o", out]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    with open(out) as f:
        return f.read()


def _sgprs(text: str) -> Set[str]:
    regs = set()
    for m in re.finditer(r"\bs\[(\d+):(\d+)\]", text):
        regs.update(f"s{r}" for r in range(int(m.group(1)), int(m.group(2)) + 1))
    regs.update(f"s{m.group(1)}" for m in re.finditer(r"\bs(\d+)\b", text))
    for m in re.finditer(r"\b(vcc|m0|exec)(_lo|_hi)?\b", text):
        regs.add(m.group(1))
    return regs


def _operands(line: str) -> List[str]:
    parts = line.split(None, 1)
    return [o.strip() for o in parts[1].split(",")] if len(parts) > 1 else []


# VOP3 forms whose second operand is a scalar destination (carry-out / lane mask)
_SDST2 = re.compile(r"^v_(add|sub|subrev)_co_(ci_)?u32_e64$|^v_(addc|subb|subbrev)_co_u32_e64$|"
                    r"^v_div_scale_f(32|64)|^v_mad_(u|i)64_(u|i)32")


def valu_sgpr_dests(line: str) -> Set[str]:
    """Scalar registers a vector-ALU instruction writes (empty for other instructions)."""
    op = line.split()[0]
    if not op.startswith("v_"):
        return set()
    ops = _operands(line)
    if not ops:
        return set()
    if op.startswith(("v_readfirstlane", "v_readlane")) or (op.startswith("v_cmp") and op.endswith("_e64")):
        return _sgprs(ops[0])
    if _SDST2.match(op) and len(ops) > 1:
        return _sgprs(ops[1])
    if op.startswith("v_cmp") or re.match(r"^v_(add|sub|subrev)_co_u32_e32$|^v_(addc|subb)_co_u32_e32$", op):
        return {"vcc"}  # e32 compares and carries write VCC
    return set()


# scalar-ALU and scalar-load opcodes whose first operand is their destination
_SALU_DST = re.compile(r"^s_(mov|movk|cmov|cmovk|cselect|add|addc|addk|sub|subb|mul|mulk|mul_hi|lshl|lshr|ashr|"
                       r"lshl[1-4]_add|and|or|xor|andn2|orn2|nand|nor|xnor|not|bfe|bfm|min|max|abs|absdiff|brev|"
                       r"ff0|ff1|flbit|bcnt0|bcnt1|sext|pack|getpc|load|buffer_load)(_|$)")


def sgpr_dests(line: str) -> Set[str]:
    """Scalar registers any instruction writes, as far as the checker needs to know: vector-ALU
    scalar destinations and the destinations of scalar-ALU ops and scalar loads."""
    op = line.split()[0]
    if op.startswith("v_"):
        return valu_sgpr_dests(line)
    ops = _operands(line)
    if ops and _SALU_DST.match(op):
        return _sgprs(ops[0])
    return set()


def _is_vmem(op: str) -> bool:
    return op.startswith(("global_", "buffer_", "flat_", "scratch_"))


def _waits_of(line: str) -> int:
    op = line.split()[0]
    if op == "s_nop":
        return int(_operands(line)[0], 0) + 1
    return 1


class Function:
    """One kernel's instructions as basic blocks: blocks[i] = list of instructions; preds[i]."""

    def __init__(self, name: str, lines: List[str]):
        self.name = name
        blocks: List[List[str]] = [[]]
        labels: Dict[str, int] = {}
        ends_flow: List[bool] = []
        targets: List[List[str]] = []
        cur_targets: List[str] = []
        for raw in lines:
            t = raw.split(";")[0].strip()
            if not t:
                continue
            if t.endswith(":") and not t.startswith("s_"):
                if blocks[-1] or cur_targets:
                    ends_flow.append(False)
                    targets.append(cur_targets)
                    blocks.append([])
                    cur_targets = []
                labels[t[:-1]] = len(blocks) - 1
                continue
            if t.startswith("."):
                continue
            blocks[-1].append(t)
            op = t.split()[0]
            if op.startswith("s_branch") or op.startswith("s_cbranch"):
                cur_targets = [_operands(t)[0]]
                ends_flow.append(op.startswith("s_branch"))
                targets.append(cur_targets)
                blocks.append([])
                cur_targets = []
            elif op in ("s_endpgm", "s_setpc_b64"):
                ends_flow.append(True)
                targets.append([])
                blocks.append([])
                cur_targets = []
        ends_flow.append(True)
        targets.append(cur_targets)
        self.blocks = blocks
        self.preds: List[List[int]] = [[] for _ in blocks]
        for i in range(len(blocks)):
            if not ends_flow[i] and i + 1 < len(blocks):
                self.preds[i + 1].append(i)
            for lab in targets[i]:
                if lab in labels:
                    self.preds[labels[lab]].append(i)

    def writers_within(self, block: int, index: int, regs: Set[str], budget: int, pick) -> List[str]:
        """Instructions on any path into (block, index) that ``pick(line) & regs`` and lie fewer
        than ``budget`` wait states before it, counting only the last write of each register on
        the path (a later write by any instruction, scalar ALU included, hides an earlier one)."""
        found: List[str] = []
        seen: Set[Tuple[int, int, frozenset]] = set()

        def walk(b: int, i: int, left: int, live: frozenset):
            if (b, left, live) in seen:
                return
            seen.add((b, left, live))
            ins = self.blocks[b]
            for j in range(i - 1, -1, -1):
                if pick(ins[j]) & live:
                    found.append(ins[j])
                    return
                live = live - sgpr_dests(ins[j])
                if not live:
                    return
                left -= _waits_of(ins[j])
                if left <= 0:
                    return
            for p in self.preds[b]:
                walk(p, len(self.blocks[p]), left, live)

        walk(block, index, budget, frozenset(regs))
        return found


def functions(asm: str) -> List[Function]:
    """The code symbols of ``asm`` (``.type <name>,@function``: kernels and device functions), each
    up to its .Lfunc_end."""
    code = set(re.findall(r"\.type\s+([\w.$]+),@function", asm))
    out, name, body = [], None, []
    for line in asm.splitlines():
        m = re.match(r"^([A-Za-z_][\w.$]*):(\s|;|$)", line)
        if m and m.group(1) in code:
            if name is not None:
                out.append(Function(name, body))
            name, body = m.group(1), []
            continue
        if name is not None:
            if line.startswith(".Lfunc_end"):
                out.append(Function(name, body))
                name, body = None, []
            else:
                body.append(line)
    if name is not None:
        out.append(Function(name, body))
    return out


def _m0_write(line: str) -> Set[str]:
    op = line.split()[0]
    ops = _operands(line)
    if op.startswith("s_") and not op.startswith(("s_nop", "s_waitcnt", "s_cbranch", "s_branch")) and ops:
        return {"m0"} if ops[0] == "m0" else set()
    return set()


def find_hazards(asm: str):
    """(VALU SGPR write -> VMEM read within 5 wait states, SALU M0 write -> LDS DMA) instances,
    over every control-flow path of every function in ``asm``."""
    sgpr_hazards, m0_hazards = [], []
    for fn in functions(asm):
        for b, ins in enumerate(fn.blocks):
            for i, line in enumerate(ins):
                op = line.split()[0]
                if not _is_vmem(op):
                    continue
                reads = _sgprs(" ".join(_operands(line))) - {"exec"}
                if "_lds_" in op:
                    reads.add("m0")
                if reads:
                    for w in fn.writers_within(b, i, reads, VALU_SGPR_WAITS, valu_sgpr_dests):
                        sgpr_hazards.append((fn.name, w, line))
                if "_lds_" in op:
                    for w in fn.writers_within(b, i, {"m0"}, M0_WAITS, _m0_write):
                        m0_hazards.append((fn.name, w, line))
    dedup = lambda hs: list(dict.fromkeys(hs))  # noqa: E731  (one entry per writer and reader)
    return dedup(sgpr_hazards), dedup(m0_hazards)


def test_checker_catches_a_readfirstlane_feeding_a_dma():
    asm = """
        .type k,@function
k:
        v_readfirstlane_b32 s1, v3
        v_readfirstlane_b32 s0, v2
        s_mov_b32 m0, s6
        global_load_lds_dwordx4 v253, s[0:1]
        s_nop 4
        s_add_i32 m0, s6, 0x1000
        s_nop 0
        global_load_lds_dwordx4 v252, s[0:1]
        s_endpgm
.Lfunc_end0:
    """
    sgpr, m0 = find_hazards(asm)
    assert len(sgpr) == 1 and "v_readfirstlane_b32 s0" in sgpr[0][1]
    assert len(m0) == 1 and "s_mov_b32 m0" in m0[0][1]


def test_checker_follows_loop_back_edges_and_branches():
    """A readfirstlane at the bottom of a loop feeds the DMA at its top (the back-edge), a compare's
    lane mask and a carry-out feed DMAs across a branch; the same code with enough wait states on
    every path is clean."""
    bad = """
        .type k,@function
k:
        s_mov_b32 s4, 0
.LBB0_1:
        s_mov_b32 m0, s5
        s_nop 0
        global_load_lds_dwordx4 v10, s[0:1]
        v_mfma_f32_16x16x32_bf16 v[20:23], v[2:5], v[6:9], v[20:23]
        s_add_i32 s4, s4, 1
        s_cmp_lt_i32 s4, 8
        v_readfirstlane_b32 s0, v12
        s_cbranch_scc1 .LBB0_1
        v_cmp_gt_i32_e64 s[8:9], v1, v2
        s_cbranch_vccz .LBB0_3
        s_nop 1
.LBB0_3:
        global_load_dword v3, v4, s[8:9]
        v_add_co_u32_e64 v5, s[10:11], v6, v7
        s_branch .LBB0_4
.LBB0_4:
        global_load_dword v3, v4, s[10:11]
        s_endpgm
.Lfunc_end0:
    """
    sgpr, m0 = find_hazards(bad)
    got = sorted(h[1].split()[0] + " -> " + h[2].split()[-1] for h in sgpr)
    assert got == ["v_add_co_u32_e64 -> s[10:11]", "v_cmp_gt_i32_e64 -> s[8:9]", "v_readfirstlane_b32 -> s[0:1]"]
    assert not m0
    good = bad.replace("s_cbranch_scc1 .LBB0_1", "s_nop 4\n        s_cbranch_scc1 .LBB0_1").replace(
        "s_cbranch_vccz .LBB0_3\n        s_nop 1", "s_nop 4\n        s_cbranch_vccz .LBB0_3\n        s_nop 1").replace(
        "v_add_co_u32_e64 v5, s[10:11], v6, v7", "v_add_co_u32_e64 v5, s[10:11], v6, v7\n        s_nop 4")
    assert find_hazards(good) == ([], [])


def test_checker_counts_the_last_write_only():
    """A spilled address restored with readlanes and then rebuilt by scalar adds is read by the DMA
    from the scalar writes: no hazard. Rebuilding only its low half leaves the readlane of the high
    half as the last write: a hazard."""
    asm = """
        .type k,@function
k:
        v_readlane_b32 s4, v239, 10
        s_add_u32 s4, s4, s8
        v_readlane_b32 s5, v239, 11
        s_addc_u32 s5, s5, s3
        s_mov_b32 m0, s3
        s_nop 0
        global_load_lds_dwordx4 v4, s[4:5]
        s_endpgm
.Lfunc_end0:
    """
    assert find_hazards(asm) == ([], [])
    half = asm.replace("s_addc_u32 s5, s5, s3", "s_nop 0")
    sgpr, m0 = find_hazards(half)
    assert len(sgpr) == 1 and "v_readlane_b32 s5" in sgpr[0][1] and not m0


def test_checker_m0_across_a_branch():
    asm = """
        .type k,@function
k:
        s_cbranch_execz .LBB0_2
        s_mov_b32 m0, s3
.LBB0_2:
        global_load_lds_dwordx4 v1, s[0:1]
        s_endpgm
.Lfunc_end0:
    """
    sgpr, m0 = find_hazards(asm)
    assert not sgpr and len(m0) == 1


@pytest.mark.skipif(shutil.which(HIPCC) is None and not os.path.exists(HIPCC), reason="hipcc not available")
@pytest.mark.parametrize("src", [os.path.basename(s) for s in SOURCES])
def test_no_dma_hazards(src, tmp_path):
    path = os.path.join(build.CSRC, src)
    asm = _device_asm(path, str(tmp_path))
    with open(path) as f:
        has_kernels = "__global__" in f.read()
    assert bool(functions(asm)) == has_kernels, "kernel symbols not found in the device assembly"
    sgpr, m0 = find_hazards(asm)
    assert not sgpr, f"VALU-written SGPR read by a memory instruction too early: {sgpr[:3]}"
    assert not m0, f"M0 written right before an LDS DMA: {m0[:3]}"
