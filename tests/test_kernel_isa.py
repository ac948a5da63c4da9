"""Checks on the gfx950 assembly of the hand-scheduled dK/dV kernel (CPU only:
hipcc cross-compiles it).

The kernel issues its dK/dV accumulating MFMAs from inline assembly, so the
compiler's hazard recognizer does not know those instructions write the
accumulator registers.  Any instruction the compiler places that reads such
a register (an AGPR copy when it keeps the accumulators in other registers
in another loop, the final VALU reads) must come at least the MFMA's
latency after the last MFMA writing it; the kernel provides that with
explicit waits (acc_settle / acc_drain).  A read closer than that reads the
value from before the MFMA, at random, and broke the bitwise repeatability
of dK/dV once.
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


@pytest.mark.skipif(not (shutil.which("hipcc") or os.path.exists("/opt/rocm/bin/hipcc")), reason="hipcc not found")
def test_dkdv_kernel_reads_no_accumulator_before_its_mfma_completes(tmp_path):
    src = os.path.join(B.CSRC, "attn_dkdv.hip")
    out = tmp_path / "attn_dkdv.s"
    cmd = [B.hipcc(), *B.COMMON, *B.EXTRA.get("attn_dkdv.hip", []), "--cuda-device-only", "-S", src, "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    asm = out.read_text()
    assert asm.count("v_mfma_f32_32x32x16_bf16") > 100
    hits = early_agpr_reads(asm)
    assert not hits, "\n".join(f"{a}   <- {b}" for a, b in hits[:10])
