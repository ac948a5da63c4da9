"""Builds cpuforge_amd/libcfattn.so (gfx950 HIP kernels + C ABI) in-tree.

    python -m cpuforge_amd.build        # or cpuforge_amd.build.build()

Every HIP source is compiled for gfx950 only, with packed-FP32 instruction
selection disabled (the kernels' f32 arithmetic stays scalar), then linked
into one shared library next to this file.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
OBJDIR = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libcfattn.so")

HIP_SOURCES = ["attn_fwd.hip", "attn_fwd_q64.hip", "attn_bwd.hip", "attn_dkdv.hip", "attn_f32.hip", "prologue.hip", "layer_ops.hip", "lora.hip",
               "io_kernels.hip", "noalloc.hip", "probe.hip", "cfattn_capi.cpp", "cfops_capi.cpp", "cfio_capi.cpp", "host_stage.cpp"]
ARCH = "gfx950"
COMMON = ["-std=c++17", "-fPIC", "-O3", f"--offload-arch={ARCH}", f"-I{INCLUDE}", f"-I{CSRC}",
          "-Wall", "-Wno-unused-result",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
# Per-file additions.  attn_dkdv.hip: MFMA results in the architectural VGPR
# form (its score products are read by VALU code; its long-lived
# accumulators are kept in AGPRs by inline assembly).  Left to choose, the
# compiler puts every MFMA of that one-wave-per-SIMD kernel in the AGPR form
# and copies the scores and accumulators between the two files each step.
EXTRA = {"attn_dkdv.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
         "attn_fwd_q64.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (os.path.sep not in cand or os.path.exists(cand)):
            return cand
    return "hipcc"


def _filter(out: str) -> str:
    # hipcc's host pass warns that it does not know the packed-fp32 target
    # feature; that is expected and harmless.
    keep = [ln for ln in out.splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
    return "\n".join(keep)


def build(verbose: bool = False) -> str:
    os.makedirs(OBJDIR, exist_ok=True)
    cc = hipcc()
    procs = []
    objs = []
    for src in HIP_SOURCES:
        obj = os.path.join(OBJDIR, os.path.splitext(src)[0] + ".o")
        objs.append(obj)
        cmd = [cc, *COMMON, *EXTRA.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
    failed = []
    for src, p in procs:
        out, _ = p.communicate()
        msg = _filter(out)
        if p.returncode != 0:
            failed.append(f"{src}:\n{msg}")
        elif msg and verbose:
            print(msg)
    if failed:
        raise RuntimeError("hipcc failed:\n" + "\n".join(failed))
    tmp = LIB + ".tmp"
    # hipBLASLt runs the plain f32 GEMMs of the layer ops (matmul_*, Linear).
    cmd = [cc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp, "-L/opt/rocm/lib", "-lhipblaslt",
           "-pthread"]
    out = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if out.returncode != 0:
        raise RuntimeError("link failed:\n" + _filter(out.stdout))
    # A kernel the host pass failed to emit links fine and only fails when
    # the library is loaded (an undefined launch stub): refuse it here.
    und = subprocess.run(["nm", "-u", tmp], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    stubs = [ln.split()[-1] for ln in und.stdout.splitlines() if "__device_stub__" in ln]
    if stubs:
        raise RuntimeError("kernel launch stubs missing from the host pass: " + ", ".join(stubs))
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
