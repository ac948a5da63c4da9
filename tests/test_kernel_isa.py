"""Checks on the gfx950 assembly of the hand-scheduled one-wave-per-SIMD
kernels, dK/dV and the forward (CPU only: hipcc cross-compiles them).

Both issue their accumulating MFMAs from inline assembly, so the compiler's
hazard recognizer does not see those instructions.  Two orders need wait
states the code provides itself:
  * an instruction the compiler places that reads an accumulator (an AGPR
    copy where it keeps the accumulators in other registers, the final
    VALU reads) must come at least the MFMA's latency after the last MFMA
    writing it.  A read closer than that reads the value from before the
    MFMA, at random, and broke the bitwise repeatability of dK/dV once;
  * a VALU instruction (an AGPR copy at a control-flow join, an operand
    conversion) that writes a register an assembly MFMA reads must come a
    few cycles before it.  A copy one slot before the MFMA that read it as
    its accumulator gave wrong forward outputs once.
Both scans follow the control flow backwards: at a label they continue
from every branch that jumps there as well as from the instruction before
it (unless that is an unconditional branch), so a read at a loop head is
checked against the MFMAs at the end of the previous iteration.
"""
import os
import re
import shutil
import subprocess
from collections import defaultdict

import pytest

from cpuforge_amd import build as B

# Issue slots (instructions, s_nop N counting N + 1) between an MFMA that
# writes an AGPR and the next non-MFMA read of it: a 32x32x16 MFMA takes 8
# passes of 4 cycles, and the documented VALU-read wait for it is well
# below this bound.
MIN_SLOTS = 20


def _program(asm: str):
    """(instructions, preds): the instructions as (text, inside inline
    assembly) in order, and for each instruction index the indices of the
    instructions control can come from just before it (the previous one
    unless that is an unconditional branch or an end, and every branch whose
    target label sits right before it)."""
    ins, labels, pending, inasm = [], {}, [], False
    for line in asm.split("\n"):
        t = line.strip()
        if t.startswith(";;#ASMSTART"):
            inasm = True
            continue
        if t.startswith(";;#ASMEND"):
            inasm = False
            continue
        if t.endswith(":") and not t.startswith(";"):
            pending.append(t[:-1])
            continue
        if not t or t.startswith(";") or t.startswith("."):
            continue
        for name in pending:
            labels[name] = len(ins)
        pending = []
        ins.append((t, inasm))
    preds = defaultdict(list)
    for i, (t, _) in enumerate(ins):
        op = t.split()[0]
        if i + 1 < len(ins) and op not in ("s_branch", "s_endpgm", "s_setpc_b64"):
            preds[i + 1].append(i)
        if (op == "s_branch" or op.startswith("s_cbranch")) and len(t.split()) > 1 and t.split()[1] in labels:
            preds[labels[t.split()[1]]].append(i)
    return ins, preds


def _slots(line: str) -> int:
    """Issue slots an instruction takes: s_nop N counts N + 1."""
    parts = line.split()
    return int(parts[1]) + 1 if parts[0] == "s_nop" else 1


def _paths_back(preds, i, budget, visit):
    """Walks every control path back from instruction i.  visit(j, slots)
    sees instruction j with `slots` issue slots between it and i (j's own
    not counted) and returns True to stop that path (a finding), False to
    go on; a path also stops once its slots reach `budget`.  Returns the
    indices where visit stopped."""
    hits, seen = [], set()
    stack = [(j, 0) for j in preds.get(i, [])]
    while stack:
        j, slots = stack.pop()
        if (j, slots) in seen or slots >= budget:
            continue
        seen.add((j, slots))
        if visit(j, slots):
            hits.append(j)
            continue
        stack.extend((k, slots + visit.cost(j)) for k in preds.get(j, []))
    return hits


def _agprs(tok: str):
    regs = set()
    for m in re.finditer(r"\ba\[(\d+):(\d+)\]", tok):
        regs |= set(range(int(m.group(1)), int(m.group(2)) + 1))
    for m in re.finditer(r"\ba(\d+)\b", tok):
        regs.add(int(m.group(1)))
    return regs


class _Visit:
    def __init__(self, ins, fn):
        self.ins, self.fn = ins, fn

    def __call__(self, j, slots):
        return self.fn(self.ins[j][0], slots)

    def cost(self, j):
        return _slots(self.ins[j][0])


def early_agpr_reads(asm: str, min_slots: int = MIN_SLOTS):
    """(reader, writer) pairs where a non-MFMA instruction (or an MFMA's A/B
    operand) reads an AGPR fewer than min_slots issue slots after an MFMA
    that writes it, on any control path leading to the reader (the MFMA's
    own slot counted)."""
    ins, preds = _program(asm)
    found = []
    for i, (line, _) in enumerate(ins):
        op, *rest = line.split(None, 1)
        toks = [t.strip() for t in rest[0].split(",")] if rest else []
        reads = toks[1:3] if op.startswith("v_mfma") else toks[1:]
        src = set().union(*[_agprs(t) for t in reads]) if reads else set()
        if not src:
            continue

        def writes_src(prev, slots):
            # The MFMA's own slot counts: it issues `slots + 1` before the reader.
            return (prev.split()[0].startswith("v_mfma") and slots + 1 < min_slots
                    and bool(_agprs(prev.split()[1].rstrip(",")) & src))

        for j in _paths_back(preds, i, min_slots, _Visit(ins, writes_src)):
            found.append((line, ins[j][0]))
    return found


# Wait states (issue slots in between, s_nop N counting N + 1) a VALU write
# of a register needs before an MFMA reads it as an operand: the figure
# the compiler's hazard recognizer inserts ahead of its own MFMAs.
SRC_WAIT_STATES = 2


def _regs(tok: str):
    regs = set()
    for m in re.finditer(r"\b([va])\[(\d+):(\d+)\]", tok):
        regs |= {(m.group(1), i) for i in range(int(m.group(2)), int(m.group(3)) + 1)}
    for m in re.finditer(r"\b([va])(\d+)\b", tok):
        regs.add((m.group(1), int(m.group(2))))
    return regs


def late_operand_writes(asm: str, wait_states: int = SRC_WAIT_STATES):
    """(writer, mfma) pairs where a VALU instruction writes a source register
    (A, B or accumulator input) of an inline-assembly MFMA with fewer than
    wait_states issue slots between them, on any control path."""
    ins, preds = _program(asm)
    found = []
    for i, (line, inasm) in enumerate(ins):
        if not (inasm and line.startswith("v_mfma")):
            continue
        ops = [t.strip() for t in line.split(None, 1)[1].split(",")]
        srcs = set().union(*[_regs(t) for t in ops[1:4]])

        def writes_src(prev, slots):
            pop, *prest = prev.split(None, 1)
            return (pop.startswith("v_") and not pop.startswith("v_mfma") and bool(prest)
                    and bool(_regs(prest[0].split(",")[0]) & srcs))

        for j in _paths_back(preds, i, wait_states, _Visit(ins, writes_src)):
            found.append((ins[j][0], line))
    return found


def test_checker_flags_a_write_right_before_an_mfma():
    asm = "\n".join([
        "v_accvgpr_mov_b32 a3, a200",
        ";;#ASMSTART",
        "v_mfma_f32_32x32x16_bf16 a[0:15], v[0:3], v[4:7], a[0:15]",
        ";;#ASMEND",
        "v_cvt_pk_bf16_f32 v9, v1, v2",
        "s_nop 1",
        ";;#ASMSTART",
        "v_mfma_f32_32x32x16_bf16 a[16:31], v[8:11], v[4:7], a[16:31]",
        ";;#ASMEND",
        "v_accvgpr_mov_b32 a33, a200",
        "s_nop 0",
        ";;#ASMSTART",
        "v_mfma_f32_32x32x16_bf16 a[32:47], v[0:3], v[4:7], a[32:47]",
        ";;#ASMEND",
        "v_cvt_pk_bf16_f32 v5, v1, v2",
        "v_mfma_f32_32x32x16_bf16 v[32:47], v[0:3], v[4:7], 0",  # compiler's own: its hazards are handled
    ])
    hits = late_operand_writes(asm)
    assert [h[0] for h in hits] == ["v_accvgpr_mov_b32 a3, a200", "v_accvgpr_mov_b32 a33, a200"]


def test_checker_flags_a_read_right_after_an_mfma():
    asm = "\n".join([
        "v_mfma_f32_32x32x16_bf16 a[0:15], v[0:3], v[4:7], a[0:15]",
        "s_nop 3",
        "v_accvgpr_mov_b32 a200, a15",
        "v_mfma_f32_32x32x16_bf16 a[16:31], v[0:3], v[4:7], a[16:31]",
        "s_nop 15", "s_nop 15", "s_nop 3",
        "v_accvgpr_read_b32 v9, a16",
        "v_mfma_f32_32x32x16_bf16 a[32:47], v[0:3], v[4:7], a[32:47]",
        "v_mfma_f32_32x32x16_bf16 a[32:47], v[0:3], v[4:7], a[32:47]",  # accumulating: not a read by VALU
    ])
    hits = early_agpr_reads(asm)
    assert [h[0] for h in hits] == ["v_accvgpr_mov_b32 a200, a15"]


def test_checkers_follow_loop_back_edges():
    """A read at a loop head right after the loop tail's MFMA, and a write at
    the tail right before the head's MFMA, are reached only over the branch
    back to the head; a straight-line scan does not see them."""
    loop = "\n".join([
        ".LBB0_1:",
        ";;#ASMSTART",
        "v_mfma_f32_32x32x16_bf16 a[0:15], v[0:3], v[4:7], a[0:15]",
        ";;#ASMEND",
        "v_accvgpr_read_b32 v9, a16",
        "s_nop 15", "s_nop 15", "s_nop 3",
        "v_mfma_f32_32x32x16_bf16 a[16:31], v[8:11], v[4:7], a[16:31]",
        "v_cvt_pk_bf16_f32 v3, v1, v2",
        "s_cbranch_scc1 .LBB0_1",
        "s_endpgm",
    ])
    assert [h[0] for h in early_agpr_reads(loop)] == ["v_accvgpr_read_b32 v9, a16"]
    assert [h[0] for h in late_operand_writes(loop)] == ["v_cvt_pk_bf16_f32 v3, v1, v2"]
    # The same instructions with the loop's branch gone: no path, no finding.
    straight = loop.replace("s_cbranch_scc1 .LBB0_1", "s_nop 0")
    assert early_agpr_reads(straight) == [] and late_operand_writes(straight) == []


def _kernel_asm(name, tmp_path):
    src = os.path.join(B.CSRC, name)
    out = tmp_path / (name + ".s")
    cmd = [B.hipcc(), *B.COMMON, *B.EXTRA.get(name, []), "--cuda-device-only", "-S", src, "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    asm = out.read_text()
    assert asm.count("v_mfma_f32_32x32x16_bf16") > 100
    return asm


@pytest.mark.skipif(not (shutil.which("hipcc") or os.path.exists("/opt/rocm/bin/hipcc")), reason="hipcc not found")
@pytest.mark.parametrize("name", ["attn_dkdv.hip", "attn_fwd_q64.hip"])
def test_kernel_reads_no_accumulator_before_its_mfma_completes(name, tmp_path):
    hits = early_agpr_reads(_kernel_asm(name, tmp_path))
    assert not hits, "\n".join(f"{a}   <- {b}" for a, b in hits[:10])


@pytest.mark.skipif(not (shutil.which("hipcc") or os.path.exists("/opt/rocm/bin/hipcc")), reason="hipcc not found")
@pytest.mark.parametrize("name", ["attn_dkdv.hip", "attn_fwd_q64.hip"])
def test_kernel_writes_no_mfma_operand_right_before_it(name, tmp_path):
    hits = late_operand_writes(_kernel_asm(name, tmp_path))
    assert not hits, "\n".join(f"{a}   -> {b}" for a, b in hits[:10])
