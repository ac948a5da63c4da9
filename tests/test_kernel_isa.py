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
"""
import os
import re
import shutil
import subprocess

import pytest

from cpuforge_amd import build as B

# Issue slots (instructions, s_nop N counting N + 1) between an MFMA that
# writes an AGPR and the next non-MFMA read of it: a 32x32x16 MFMA takes 8
# passes of 4 cycles, and the documented VALU-read wait for it is well
# below this bound.
MIN_SLOTS = 20


def _instructions(asm: str):
    out = []
    for line in asm.split("\n"):
        t = line.strip()
        if not t or t.startswith(";") or t.startswith(".") or t.endswith(":"):
            continue
        out.append(t)
    return out


def _agprs(tok: str):
    regs = set()
    for m in re.finditer(r"\ba\[(\d+):(\d+)\]", tok):
        regs |= set(range(int(m.group(1)), int(m.group(2)) + 1))
    for m in re.finditer(r"\ba(\d+)\b", tok):
        regs.add(int(m.group(1)))
    return regs


def early_agpr_reads(asm: str, min_slots: int = MIN_SLOTS):
    """(reader, writer) pairs where a non-MFMA instruction (or an MFMA's A/B
    operand) reads an AGPR fewer than min_slots issue slots after an MFMA
    that writes it, scanning the instruction stream backwards in order."""
    ins = _instructions(asm)
    found = []
    for i, line in enumerate(ins):
        op, *rest = line.split(None, 1)
        toks = [t.strip() for t in rest[0].split(",")] if rest else []
        reads = toks[1:3] if op.startswith("v_mfma") else toks[1:]
        src = set().union(*[_agprs(t) for t in reads]) if reads else set()
        if not src:
            continue
        slots = 0
        for j in range(i - 1, max(-1, i - 4 * min_slots), -1):
            prev = ins[j]
            pop = prev.split()[0]
            slots += int(prev.split()[1]) + 1 if pop == "s_nop" else 1
            if slots >= min_slots:
                break
            if pop.startswith("v_mfma") and _agprs(prev.split()[1].rstrip(",")) & src:
                found.append((line, prev))
                break
    return found


# Wait states (issue slots in between, s_nop N counting N + 1) a VALU write
# of a register needs before an MFMA reads it as an operand: the figure
# the compiler's hazard recognizer inserts ahead of its own MFMAs.
SRC_WAIT_STATES = 2


def _asm_instructions(asm: str):
    """(instruction, inside inline assembly) in order."""
    out, inasm = [], False
    for line in asm.split("\n"):
        t = line.strip()
        if t.startswith(";;#ASMSTART"):
            inasm = True
            continue
        if t.startswith(";;#ASMEND"):
            inasm = False
            continue
        if not t or t.startswith(";") or t.startswith(".") or t.endswith(":"):
            continue
        out.append((t, inasm))
    return out


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
    wait_states issue slots between them."""
    ins = _asm_instructions(asm)
    found = []
    for i, (line, inasm) in enumerate(ins):
        if not (inasm and line.startswith("v_mfma")):
            continue
        ops = [t.strip() for t in line.split(None, 1)[1].split(",")]
        srcs = set().union(*[_regs(t) for t in ops[1:4]])
        slots = 0
        for j in range(i - 1, max(-1, i - 4 * wait_states - 4), -1):
            prev = ins[j][0]
            pop, *prest = prev.split(None, 1)
            if slots >= wait_states:
                break
            if pop.startswith("v_") and not pop.startswith("v_mfma") and prest:
                if _regs(prest[0].split(",")[0]) & srcs:
                    found.append((prev, line))
                    break
            slots += int(prest[0]) + 1 if pop == "s_nop" else 1
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
