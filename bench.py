"""Benchmark of the causal GQA attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config C5] [--mode bf16]

One step is one forward + backward of cpuforge's attention op
(crates/core/src/ops/attention.rs:42-262) over one batch of the configuration:
cfattn_fwd (O, lse overwritten) then cfattn_bwd (dQ, dK, dV accumulated), on
device-resident inputs.  The default workload is BASELINE.json's Llama-3-8B
layer shape (batch 1, seq 8192, 32 query / 8 KV heads, head_dim 128, bf16
inputs with fp32 accumulation), the configuration the target figure is
quoted on.  Q and K are produced once, before timing, by the library's RoPE
prologue (theta 500000) from synthetic N(0,1) data.

Printed: one JSON line with the whole-step throughput (algorithmic TFLOP/s,
7*B*Hq*D*S*(S+1) per step), a `roofline` object for the kernel that takes the
most time (its algorithmic FLOPs per launch / its mean launch time, measured
with hipEvents on its stream over the timed steps) and a `cpu_baseline`
object: the oracle's restatement of the reference CPU algorithm timed on a
bounded sample of the same workload on the host cores.  Beside them:
`f32`, the same step at the reference's own precision (C2, f32 inputs, fp32
MFMA; roofline against the fp32 matrix peak); `fused`, the Layer-level step
of the headline config (q/k prologue + attention forward and backward through
cfattn_fused_fwd/bwd); and `smollm_train`, the SmolLM-135M LoRA train step.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

# MI355X published dense peaks (TFLOP/s) and HBM bandwidth (GB/s).
PEAK_TFLOPS = {"bf16": 2516.6, "f32": 157.3}
PEAK_HBM_GBS = 8000.0

# name: (batch, seq, n_heads, n_kv, head_dim, theta, llama3 scaling, qk norm)
CONFIGS = {
    "C1": (1, 512, 9, 3, 64, 1e4, None, False),
    "C2": (8, 2048, 9, 3, 64, 1e4, None, False),
    "C3": (4, 4096, 32, 8, 64, 5e5, (32.0, 1.0, 4.0, 8192.0), False),
    "C4": (4, 4096, 16, 8, 128, 1e6, None, True),
    "C5": (1, 8192, 32, 8, 128, 5e5, None, False),
}
WORKLOAD = {
    "C1": "SmolLM-135M attention layer (B1 S512 9q/3kv D64)",
    "C2": "SmolLM-135M attention, training batch (B8 S2048 9q/3kv D64)",
    "C3": "Llama-3.2-1B attention layer (B4 S4096 32q/8kv D64, llama3 rope)",
    "C4": "Qwen3-0.6B attention layer (B4 S4096 16q/8kv D128, q/k rmsnorm)",
    "C5": "Llama-3-8B attention layer (B1 S8192 32q/8kv D128)",
}

# Contractions each kernel performs that the algorithmic count includes
# (units of B*Hq*D*S*(S+1) FLOPs): forward QK^T and PV; dK/dV kernel the
# recomputed QK^T, dP = dO V^T, dV and dK; dQ kernel dQ only (it also
# recomputes QK^T and dP, which the algorithmic count does not credit).
ALGO_UNITS = {"attn_fwd": 2.0, "attn_bwd_dkdv": 4.0, "attn_bwd_dq": 1.0}


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="C5", choices=sorted(CONFIGS))
    ap.add_argument("--mode", default=None, choices=["bf16", "f32"], help="default: bf16 (f32 for C1)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the cpu_baseline leg")
    ap.add_argument("--cpu-heads", type=int, default=16, help="query heads of sequence 0 in the CPU sample")
    ap.add_argument("--cpu-single-heads", type=int, default=4,
                    help="query heads of sequence 0 in the single-thread CPU sample (0 skips it)")
    ap.add_argument("--no-train", action="store_true", help="skip the SmolLM-135M train tok/s leg")
    ap.add_argument("--train-steps", type=int, default=10)
    ap.add_argument("--no-f32", action="store_true", help="skip the f32 (C2) sub-object")
    ap.add_argument("--no-fused", action="store_true", help="skip the fused Layer-level sub-object")
    ap.add_argument("--sub-steps", type=int, default=20, help="timed steps of the f32 and fused sub-objects")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="run one plain device copy of MIB MiB before timing (calibrates rocprofv3 byte counters)")
    ap.add_argument("--host-slices", action="store_true",
                    help="time the drop-in host-slice entry points instead (PCIe-inclusive; not the headline value)")
    ap.add_argument("--fused", action="store_true",
                    help="time the Layer-level path instead: q/k prologue (RoPE, Qwen3 norm) + attention, forward "
                         "and backward (cfattn_fused_fwd/bwd); prints its own JSON line")
    ap.add_argument("--io", action="store_true",
                    help="time the on-disk formats (include/cfio.h) at SmolLM-135M scale instead")
    ap.add_argument("--ops", action="store_true",
                    help="time the layer ops (include/cfops.h) at the SmolLM-135M train shape and the train step "
                         "with and without them; prints its own JSON line")
    ap.add_argument("--peak", action="store_true",
                    help="measure the on-board bf16 MFMA ceiling only (cfattn_probe_mfma_peak on pseudo-random and "
                         "on zero operands); prints its own JSON line")
    ap.add_argument("--fwd-dist", action="store_true",
                    help="time the C5 bf16 forward on score distributions that move the running max (and count "
                         "the wave-tiles whose row-sum guard settles); prints its own JSON line")
    ap.add_argument("--power", type=float, default=0.0, metavar="SECONDS",
                    help="board power and GFX clocks (amd-smi) while the --config forward, backward and whole step "
                         "(--mode, bf16 by default) each run back to back for SECONDS; prints its own JSON line")
    ap.add_argument("--zero-inputs", action="store_true",
                    help="diagnostic: q, k, v, dO all zero (the same kernels and instructions with the least bit "
                         "activity, to show what the board's power limit costs); not a benchmark figure")
    ap.add_argument("--energy", type=float, default=0.0, metavar="SECONDS",
                    help="board power (amd-smi) while loops of one instruction class run back to back for SECONDS "
                         "each (LDS reads, v_fma_f32, bf16 MFMA on random and zero operands, an HBM copy) and at "
                         "idle; prints its own JSON line")
    ap.add_argument("--sweep", action="store_true",
                    help="per-kernel times of the bf16 step at the --config heads and head_dim, the tokens held at "
                         "the config's batch x seq and the sequence halved from 4x seq (B shrinking to match) down "
                         "to seq/4, with a least-squares split of each backward kernel's time into a per-step and a "
                         "per-workgroup part; prints its own JSON line")
    ap.add_argument("--ds-limit", type=int, default=None, metavar="BYTES",
                    help="stored-dS scratch limit of the context (0: dQ recomputes the softmax instead)")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the C2/C3/C4 bf16 sub-objects of the default run")
    ap.add_argument("--traffic-file", default=None,
                    help="rocprofv3 traffic summary to read `traffic` from (default: profiles/ match)")
    return ap.parse_args()


def _host_cpu():
    """Host CPU model name and logical CPU count, as lscpu and nproc show them."""
    name = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    name = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"model": name, "nproc": os.cpu_count()}


def cpu_baseline(cfg_name, mode, heads, single_heads):
    """The oracle (a C restatement of attention_forward_blocked /
    attention_backward_blocked with an OpenMP GEMM) timed on query heads
    [0, heads) of one sequence of the workload with all its threads, and on
    query heads [0, single_heads) with one thread.  Runs on the host only."""
    import numpy as np

    from oracle import oracle as O
    B, S, Hq, Hk, D = CONFIGS[cfg_name][:5]
    grp = Hq // Hk

    def whole_groups(n):
        n = max(grp, min(n, Hq))
        return n - n % grp

    heads, single_heads = whole_groups(heads), whole_groups(single_heads)
    q = O.rand(S * Hq * D, 1, 1.0)
    k = O.rand(S * Hk * D, 2, 1.0)
    v = O.rand(S * Hk * D, 3, 1.0)
    g = O.rand(S * Hq * D, 4, 1.0)
    if mode == "bf16":
        q, k, v, g = (O.round_bf16(x) for x in (q, k, v, g))

    def run(nh):
        o = np.zeros_like(q)
        lse = np.zeros(Hq * S, np.float32)
        dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
        t0 = time.perf_counter()
        O.attention_forward_blocked(q, k, v, o, lse, S, Hq, Hk, D, 128, heads=(0, nh))
        O.attention_backward_blocked(g, q, k, v, o, lse, dq, dk, dv, S, Hq, Hk, D, 128, heads=(0, nh))
        dt = time.perf_counter() - t0
        return 7.0 * nh * D * S * (S + 1), dt

    threads = O.gemm_threads()
    flops, dt = run(heads)
    out = {
        "value": flops / dt / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle fwd+bwd (q_block 128, f32 arithmetic) over query heads 0..{heads} of one sequence "
                   f"of {cfg_name} (S={S}, D={D}); {dt:.2f} s for {flops / 1e9:.1f} GFLOP"),
        "host": _host_cpu(),
    }
    if single_heads > 0:
        O.set_gemm_threads(1)
        try:
            flops1, dt1 = run(single_heads)
        finally:
            O.set_gemm_threads(threads)
        out["single_core"] = {
            "value": flops1 / dt1 / 1e12,
            "unit": "TFLOP/s",
            "cores": 1,
            "sample": f"query heads 0..{single_heads} of the same sequence; {dt1:.2f} s for {flops1 / 1e9:.1f} GFLOP",
        }
    return out


def peak_probe(ctx, runs=3, iters=40000):
    """On-board bf16 MFMA ceiling (cfattn_probe_mfma_peak): a loop of
    32x32x16 MFMAs on every SIMD after one warm-up run, on pseudo-random
    operands (the bit activity of the attention inputs) and on zeros.  The
    board's power limit sets the clock under such a load, so the random
    figure, not the 2.4 GHz spec, is what a kernel can reach."""
    out = {}
    for kind, zeros in (("random", False), ("zeros", True)):
        ctx.probe_mfma_peak(zeros, iters)  # warm-up: lets the clock settle under the load
        vals = sorted(ctx.probe_mfma_peak(zeros, iters) for _ in range(runs))
        out[kind] = round(vals[len(vals) // 2], 1)
    return out


def mfma_shape_probe(ctx, runs=3, iters=40000):
    """The 16x16x32 bf16 MFMA loop (cfattn_probe_loop kind "mfma16") against
    the 32x32x16 one on the same pseudo-random operands, alternating, median
    TFLOP/s of each: which shape does more FLOPs under the board's power
    limit."""
    ctx.probe_mfma_peak(False, iters)  # warm-up
    r32, r16 = [], []
    for _ in range(runs):
        r32.append(ctx.probe_mfma_peak(False, iters))
        r16.append(ctx.probe_loop("mfma16", iters) / 1e12)
    return {"mfma_32x32x16_random": round(sorted(r32)[runs // 2], 1),
            "mfma_16x16x32_random": round(sorted(r16)[runs // 2], 1)}


def fwd_distributions(a):
    """The C5 bf16 forward (attn_fwd_q64_kernel) on inputs whose scores move
    the running max, against N(0,1) inputs.  The kernel forms P against the
    running max as it stands and settles a wave-tile (exact row max, lazy
    rescale, P formed again) only when the tile's row sums show that the max
    may have moved; the first key tile of every wave always settles.
    Distributions (q, k, v ~ N(0,1) before the changes):
      normal   as is (scores ~ N(0,1) after the 1/sqrt(D) scale);
      growing  keys scaled x1 at token 0 to x12 at the end (the running max
               moves many times along every row; test_bf16_running_max_moves);
      std4     q and k doubled: scores ~ N(0, 4^2);
      diag     k_j = 0.5 q_j (the first query head of the group) + 0.87 noise:
               every row's largest score sits on its diagonal, the last tile.
    Per distribution: the forward's mean time over `steps` launches
    (hipEvents), the settled wave-tiles of one launch over all its
    wave-tiles, and the largest lse."""
    import torch

    import cpuforge_amd as cf
    B, S, Hq, Hk, D = CONFIGS["C5"][:5]
    grp = Hq // Hk
    nqt = (S + 63) // 64
    wave_tiles = B * Hq * nqt * (nqt + 1) // 2  # a 64-query wave walks key tiles 0 .. its diagonal
    ctx = cf.Context(0)
    from cpuforge_amd import device as dev
    out = {}
    for dist in ("normal", "growing", "std4", "diag"):
        g = torch.Generator(device="cuda")
        g.manual_seed(77)
        q = torch.randn(B, S, Hq, D, device="cuda", generator=g)
        k = torch.randn(B, S, Hk, D, device="cuda", generator=g)
        v = torch.randn(B, S, Hk, D, device="cuda", generator=g).to(torch.bfloat16)
        if dist == "growing":
            k = k * (1.0 + 11.0 * torch.arange(S, device="cuda", dtype=torch.float32) / S).view(1, S, 1, 1)
        elif dist == "std4":
            q, k = 2.0 * q, 2.0 * k
        elif dist == "diag":
            k = 0.5 * q[:, :, ::grp, :] + 0.87 * k
        q, k = q.to(torch.bfloat16), k.to(torch.bfloat16)
        o = torch.empty(B, S, Hq, D, device="cuda")
        lse = torch.empty(B, Hq, S, device="cuda")
        for _ in range(max(3, a.warmup)):
            dev.fwd(q, k, v, o, lse, ctx=ctx)
        torch.cuda.synchronize()
        ctx.fwd_stats_enable(True)
        dev.fwd(q, k, v, o, lse, ctx=ctx)
        settles = ctx.fwd_stats_read()
        ctx.fwd_stats_enable(False)
        ctx.profile_select(["attn_fwd"])
        ctx.profile_enable(True)
        for _ in range(a.steps):
            dev.fwd(q, k, v, o, lse, ctx=ctx)
        ms, n = ctx.profile_read()["attn_fwd"]
        ctx.profile_enable(False)
        ctx.profile_select(None)
        out[dist] = {"fwd_ms": round(ms / n, 4), "settles": settles, "wave_tiles": wave_tiles,
                     "settle_frac": round(settles / wave_tiles, 5), "lse_max": round(float(lse.max()), 3),
                     "tflops": round(2.0 * B * Hq * D * S * (S + 1) / (ms / n * 1e-3) / 1e12, 1)}
        del q, k, v, o, lse
        print(f"bench: fwd {dist}: {out[dist]}", file=sys.stderr, flush=True)
    ctx.close()
    base = out["normal"]["fwd_ms"]
    print(json.dumps({"metric": "C5 bf16 forward on score distributions that move the running max",
                      "value": max(out[d]["fwd_ms"] / base - 1.0 for d in out), "unit": "worst slowdown vs N(0,1)",
                      "higher_is_better": False, "dtype": "bf16", "steps": a.steps,
                      "config": {"workload": WORKLOAD["C5"], "config": "C5", "kernel": "attn_fwd_q64_kernel"},
                      "data": "synthetic (torch.randn, seed 77), changed per distribution as documented",
                      "distributions": out,
                      "slowdown_vs_normal": {d: round(out[d]["fwd_ms"] / base - 1.0, 4) for d in out}}), flush=True)


def shape_sweep(a):
    """Per-kernel times (the library's hipEvents around every launch, 10
    steps after 3 warm-up ones) of the bf16 step at the heads and head_dim of
    a.config with batch x seq fixed, and for each backward kernel of the
    one-workgroup-per-CU grids the least-squares fit
        time = step_us x (steps per CU) + wg_us x (workgroups per CU).
    The dK/dV grid has one workgroup per 128 keys of a KV head, walking
    group x (query tiles of 64 from its key tile to the end) steps; the
    stored-dS dQ grid one workgroup per (KV head, tile of 8 query blocks),
    walking the key tiles of 64 up to its last query.  Both run one workgroup
    per CU, so the workgroups (steps) per CU are the grid's (its steps) / CUs.
    Inputs are N(0,1) without RoPE."""
    import numpy as np
    import torch

    import cpuforge_amd as cf
    from cpuforge_amd import device as dev
    B0, S0, Hq, Hk, D = CONFIGS[a.config][:5]
    tokens = B0 * S0
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    group = Hq // Hk
    ctx = cf.Context(0)
    rows = []
    for S in (4 * S0, 2 * S0, S0, S0 // 2, S0 // 4):
        if S < 256 or tokens % S:
            continue
        B = tokens // S
        g = torch.Generator(device="cuda")
        g.manual_seed(1234)
        q = torch.randn(B, S, Hq, D, device="cuda", generator=g).to(torch.bfloat16)
        k = torch.randn(B, S, Hk, D, device="cuda", generator=g).to(torch.bfloat16)
        v = torch.randn(B, S, Hk, D, device="cuda", generator=g).to(torch.bfloat16)
        d_o = torch.randn(B, S, Hq, D, device="cuda", generator=g).to(torch.bfloat16)
        o, lse = torch.empty(B, S, Hq, D, device="cuda"), torch.empty(B, Hq, S, device="cuda")
        dq, dk, dv = torch.zeros_like(o), torch.zeros(B, S, Hk, D, device="cuda"), torch.zeros(B, S, Hk, D, device="cuda")

        def step():
            dev.fwd(q, k, v, o, lse, ctx=ctx)
            dev.bwd(d_o, q, k, v, o, lse, dq, dk, dv, ctx=ctx)

        for _ in range(3):
            step()
        torch.cuda.synchronize()
        ctx.profile_select(None)
        ctx.profile_enable(True)
        for _ in range(10):
            step()
        torch.cuda.synchronize()
        ms = {n: round(t / c, 4) for n, (t, c) in ctx.profile_read().items() if c}
        ctx.profile_enable(False)
        nqt, nkt = S // 64, S // 128
        # dK/dV: key tile j of a head walks group * (nqt - 2j) steps.
        kv_wgs = B * Hk * nkt
        kv_steps = B * Hk * group * sum(nqt - 2 * j for j in range(nkt))
        # stored-dS dQ (head_dim 128): tiles of 8 query blocks over the group's
        # heads (hpw heads x 8 / hpw blocks); tile t walks key tiles up to its end.
        hpw = 4 if group % 4 == 0 else 2 if group % 2 == 0 else 1
        tq = 32 * (8 // hpw)
        ntt = S // tq
        q_wgs = B * Hk * (group // hpw) * ntt
        q_steps = B * Hk * (group // hpw) * sum(((t + 1) * tq + 63) // 64 for t in range(ntt))
        rows.append({"batch": B, "seq": S, "kernels_ms": ms,
                     "dkdv": {"steps_per_cu": kv_steps / cus, "wgs_per_cu": kv_wgs / cus},
                     "dq": {"steps_per_cu": q_steps / cus, "wgs_per_cu": q_wgs / cus}})
        print(f"bench: sweep B{B} S{S} {ms}", file=sys.stderr, flush=True)
        del q, k, v, d_o, o, lse, dq, dk, dv
        torch.cuda.empty_cache()
    fits = {}
    for kern, key in (("attn_bwd_dkdv", "dkdv"), ("attn_bwd_dq", "dq")):
        A = np.array([[r[key]["steps_per_cu"], r[key]["wgs_per_cu"]] for r in rows])
        y = np.array([r["kernels_ms"].get(kern, 0.0) * 1e3 for r in rows])
        if len(rows) >= 2 and D == 128:
            coef = np.linalg.lstsq(A, y, rcond=None)[0]
            fits[kern] = {"step_us": round(float(coef[0]), 3), "wg_us": round(float(coef[1]), 2),
                          "max_residual_us": round(float(np.max(np.abs(A @ coef - y))), 2)}
    ctx.close()
    print(json.dumps({"metric": f"per-kernel times across sequence lengths at {a.config}'s heads and head_dim",
                      "value": None, "unit": "ms", "dtype": "bf16", "tokens": tokens, "n_heads": Hq, "n_kv": Hk,
                      "head_dim": D, "cus": cus, "data": "synthetic (torch.randn, seed 1234, no RoPE)",
                      "config": {"workload": WORKLOAD[a.config], "config": a.config}, "rows": rows,
                      "fit": fits}), flush=True)


def _smi_sampler(stop, out):
    """amd-smi samples (time, board power W, median XCD GFX clock MHz) into
    `out` until `stop` is set."""
    import re
    import shutil
    import subprocess
    smi = shutil.which("amd-smi") or "/opt/rocm/bin/amd-smi"
    while not stop.is_set():
        t = subprocess.run([smi, "metric", "-g", "0", "-p", "-c"], capture_output=True, text=True).stdout
        pw = re.search(r"SOCKET_POWER:\s*([0-9.]+)\s*W", t)
        clk = [int(c) for c in re.findall(r"GFX_\d+:\s*\n\s*CLK:\s*(\d+)\s*MHz", t)]
        if pw and clk:
            out.append((time.perf_counter(), float(pw.group(1)), sorted(clk)[len(clk) // 2]))


def energy_probes(a):
    """Board power per instruction class: each loop (cfattn_probe_loop,
    cfattn_probe_mfma_peak, torch's device copy) runs back to back for
    a.energy seconds while amd-smi is sampled (samples of the first 0.7 s
    dropped), and the board is read idle.  Per class: median power and
    clock, the loop's rate, and (power - idle power) / rate, an upper bound
    of the energy per unit (it also carries the clocked-but-idle power,
    which grows with the clock)."""
    import threading

    import torch

    import cpuforge_amd as cf
    ctx = cf.Context(0)

    def run_for(fn):
        samples, stop = [], threading.Event()
        th = threading.Thread(target=_smi_sampler, args=(stop, samples), daemon=True)
        t0 = time.perf_counter()
        th.start()
        rates = []
        while time.perf_counter() - t0 < a.energy:
            rates.append(fn())
        torch.cuda.synchronize()
        stop.set()
        th.join()
        kept = [(w, c) for ts, w, c in samples if ts - t0 > 0.7]
        ws, cs = sorted(w for w, _ in kept), sorted(c for _, c in kept)
        rs = sorted(r for r in rates if r)
        return (ws[len(ws) // 2] if ws else None, cs[len(cs) // 2] if cs else None,
                rs[len(rs) // 2] if rs else None, len(kept))

    samples, stop = [], threading.Event()
    th = threading.Thread(target=_smi_sampler, args=(stop, samples), daemon=True)
    t0 = time.perf_counter()
    th.start()
    time.sleep(a.energy)
    stop.set()
    th.join()
    idle = sorted(w for ts, w, _ in samples if ts - t0 > 0.5)
    idle_w = idle[len(idle) // 2] if idle else None
    x = torch.empty(1 << 28, device="cuda")
    y = torch.empty_like(x)
    x.normal_()
    cp_bytes = 2.0 * x.numel() * 4

    def copy_rate():
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        y.copy_(x)
        e1.record()
        e1.synchronize()
        return cp_bytes / (e0.elapsed_time(e1) * 1e-3)

    classes = {
        "lds_read": (lambda: ctx.probe_loop("lds"), "B/s", "pJ/B"),
        "valu_fma_f32": (lambda: ctx.probe_loop("valu"), "lane-op/s", "pJ/lane-op"),
        "mfma_bf16_random": (lambda: ctx.probe_mfma_peak(False, 20000) * 1e12 / 32768.0, "MFMA/s", "pJ/MFMA"),
        "mfma_bf16_zeros": (lambda: ctx.probe_mfma_peak(True, 20000) * 1e12 / 32768.0, "MFMA/s", "pJ/MFMA"),
        "hbm_copy": (copy_rate, "B/s", "pJ/B"),
    }
    out = {}
    for name, (fn, unit, eunit) in classes.items():
        fn()
        pw, ck, rate, n = run_for(fn)
        e = round((pw - idle_w) / rate * 1e12, 3) if pw and idle_w and rate else None
        out[name] = {"power_w": pw, "clock_mhz": ck, "rate": rate, "unit": unit, "samples": n,
                     "over_idle": e, "over_idle_unit": eunit}
        print(f"bench: energy {name}: {out[name]}", file=sys.stderr, flush=True)
    ctx.close()
    print(json.dumps({"metric": "board power per instruction class (amd-smi)", "value": idle_w, "unit": "W idle",
                      "higher_is_better": False, "seconds_per_class": a.energy, "idle_w": idle_w,
                      "data": "loop probes (cfattn_probe_loop, cfattn_probe_mfma_peak) and torch's device copy",
                      "classes": out}), flush=True)


def power_clock(a, mode="bf16"):
    """Board power (SOCKET_POWER) and the GFX clocks of the 8 XCDs, read with
    amd-smi every ~0.1 s while the forward, backward or whole step of config
    a.config (C5 by default; q, k, v, dO drawn from N(0,1), no RoPE) in
    `mode` (bf16 or f32) runs back to back for a.power seconds each.  Samples
    from the first 0.5 s of each run (the clock settling) are dropped.
    Reports per phase the median power, median XCD clock and the kernels'
    mean time."""
    import re
    import shutil
    import subprocess
    import threading

    import torch

    import cpuforge_amd as cf
    from cpuforge_amd import device as dev
    smi = shutil.which("amd-smi") or "/opt/rocm/bin/amd-smi"
    B, S, Hq, Hk, D = CONFIGS[a.config][:5]
    ctx = cf.Context(0)
    g = torch.Generator(device="cuda")
    g.manual_seed(1234)
    tdt = torch.bfloat16 if mode == "bf16" else torch.float32
    q = torch.randn(B, S, Hq, D, device="cuda", generator=g).to(tdt)
    k = torch.randn(B, S, Hk, D, device="cuda", generator=g).to(tdt)
    v = torch.randn(B, S, Hk, D, device="cuda", generator=g).to(tdt)
    d_o = torch.randn(B, S, Hq, D, device="cuda", generator=g).to(tdt)
    o, lse = torch.empty(B, S, Hq, D, device="cuda"), torch.empty(B, Hq, S, device="cuda")
    dq, dk, dv = torch.zeros_like(o), torch.zeros(B, S, Hk, D, device="cuda"), torch.zeros(B, S, Hk, D, device="cuda")
    dev.fwd(q, k, v, o, lse, ctx=ctx)
    torch.cuda.synchronize()

    def sample(stop, out):
        while not stop.is_set():
            r = subprocess.run([smi, "metric", "-g", "0", "-p", "-c"], capture_output=True, text=True)
            t = r.stdout
            pw = re.search(r"SOCKET_POWER:\s*([0-9.]+)\s*W", t)
            clk = [int(c) for c in re.findall(r"GFX_\d+:\s*\n\s*CLK:\s*(\d+)\s*MHz", t)]
            if pw and clk:
                out.append((time.perf_counter(), float(pw.group(1)), sorted(clk)[len(clk) // 2]))

    phases = {"fwd": lambda: dev.fwd(q, k, v, o, lse, ctx=ctx),
              "bwd": lambda: dev.bwd(d_o, q, k, v, o, lse, dq, dk, dv, ctx=ctx),
              "step": lambda: (dev.fwd(q, k, v, o, lse, ctx=ctx), dev.bwd(d_o, q, k, v, o, lse, dq, dk, dv, ctx=ctx))}
    out = {}
    for name, fn in phases.items():
        samples, stop = [], threading.Event()
        th = threading.Thread(target=sample, args=(stop, samples), daemon=True)
        t0 = time.perf_counter()
        th.start()
        n = 0
        while time.perf_counter() - t0 < a.power:
            for _ in range(10):
                fn()
            torch.cuda.synchronize()
            n += 10
        dt = time.perf_counter() - t0
        stop.set()
        th.join()
        kept = [(w, c) for ts, w, c in samples if ts - t0 > 0.5]
        ws, cs = sorted(w for w, _ in kept), sorted(c for _, c in kept)
        out[name] = {"ms": round(dt / n * 1e3, 4), "samples": len(kept),
                     "power_w_median": ws[len(ws) // 2] if ws else None,
                     "power_w_range": [ws[0], ws[-1]] if ws else None,
                     "gfx_clock_mhz_median": cs[len(cs) // 2] if cs else None,
                     "gfx_clock_mhz_range": [cs[0], cs[-1]] if cs else None}
        print(f"bench: power {name}: {out[name]}", file=sys.stderr, flush=True)
    ctx.close()
    print(json.dumps({"metric": f"board power and GFX clock under the {a.config} {mode} kernels (amd-smi)",
                      "value": out["step"]["power_w_median"], "unit": "W", "higher_is_better": False,
                      "dtype": mode, "seconds_per_phase": a.power,
                      "config": {"workload": WORKLOAD[a.config], "config": a.config},
                      "data": "synthetic (torch.randn, seed 1234)", "phases": out}), flush=True)


def read_traffic(path, kernel, workload_key):
    """HBM bytes per launch of `kernel` from a committed rocprofv3 summary:
    a line `traffic_bytes <kernel> <workload_key> <bytes>`."""
    if not path or not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            parts = line.split()
            if len(parts) == 4 and parts[0] == "traffic_bytes" and parts[1] == kernel and parts[2] == workload_key:
                return float(parts[3])
    return None


def host_slices(a, mode):
    """Times cfattn_attention_forward + cfattn_attention_backward on host
    float32 buffers (the reference's calling convention: every operand crosses
    PCIe both ways on every call).  Prints its own JSON line."""
    import numpy as np

    import cpuforge_amd as cf
    B, S, Hq, Hk, D = CONFIGS[a.config][:5]
    rng = np.random.default_rng(5)
    q, g = (rng.standard_normal(S * Hq * D, dtype=np.float32) for _ in range(2))
    k, v = (rng.standard_normal(S * Hk * D, dtype=np.float32) for _ in range(2))
    o = np.zeros_like(q)
    lse = np.zeros(Hq * S, np.float32)
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    ctx = cf.Context(0)
    ctx.set_mode(mode)
    s = cf.AttnShape(S, Hq, Hk, D)

    def step():
        for _ in range(B):  # the trainer's B sequential single-sequence calls
            cf.attention_forward(q, k, v, o, lse, s, ctx)
            cf.attention_backward(g, q, k, v, o, lse, dq, dk, dv, s, ctx)

    for _ in range(a.warmup):
        step()
    t0 = time.perf_counter()
    for _ in range(a.steps):
        step()
    per = (time.perf_counter() - t0) / a.steps
    flops = 7.0 * B * Hq * D * S * (S + 1)
    ctx.close()
    print(json.dumps({"metric": "attention fwd+bwd TFLOP/s through the host-slice drop-in (PCIe-inclusive)",
                      "value": round(flops / per / 1e12, 3), "unit": "TFLOP/s", "ms_per_step": round(per * 1e3, 3),
                      "steps": a.steps, "warmup": a.warmup, "dtype": mode, "higher_is_better": True,
                      "config": {"workload": WORKLOAD[a.config], "config": a.config, "host_buffers": "numpy float32"}}),
          flush=True)


def fused_layer(a, mode):
    """Prints the JSON line of `fused_timing` for --config/--mode."""
    r = fused_timing(a.config, mode, a.steps, a.warmup)
    print(json.dumps({"metric": "Layer attention fwd+bwd (prologue + attention) TFLOP/s, attention FLOPs only",
                      "value": r["value"], "unit": "TFLOP/s", "ms_per_step": r["ms_per_step"],
                      "steps": a.steps, "warmup": a.warmup, "dtype": mode, "higher_is_better": True,
                      "kernels_ms": r["kernels_ms"],
                      "config": {"workload": WORKLOAD[a.config], "config": a.config, "path": "cfattn_fused_fwd/bwd"}}),
          flush=True)


def fused_timing(cfg, mode, steps, warmup):
    """Times cfattn_fused_fwd + cfattn_fused_bwd: Layer::forward/backward's
    attention part (crates/model/src/layer.rs:104-121, 183-206): pre-RoPE
    q/k in f32 -> [q/k RMSNorm] -> RoPE -> attention, and back to dq_pre,
    dk_pre, dv (and the norm-gain gradients).  Returns ms per step, the
    attention-FLOP TFLOP/s and the time of each kernel."""
    import torch

    import cpuforge_amd as cf
    from cpuforge_amd import device as dev
    B, S, Hq, Hk, D, theta, scaling, qk_norm = CONFIGS[cfg]
    ctx = cf.Context(0)
    torch.manual_seed(1234)
    dt = torch.bfloat16 if mode == "bf16" else torch.float32
    q_pre = torch.randn(B, S, Hq, D, device="cuda")
    k_pre = torch.randn(B, S, Hk, D, device="cuda")
    v = torch.randn(B, S, Hk, D, device="cuda").to(dt)
    d_o = torch.randn(B, S, Hq, D, device="cuda").to(dt)
    sc = cf.Llama3Scaling(*scaling) if scaling else None
    qn = kn = None
    if qk_norm:
        qn = (1.0 + 0.02 * torch.randn(D, device="cuda")).float()
        kn = (1.0 + 0.02 * torch.randn(D, device="cuda")).float()
    pr = dev.DeviceRope(cf.RopeCache(D, S, theta, sc), "cuda", 0, qn, kn, 1e-6)
    dq_pre, dk_pre = torch.zeros_like(q_pre), torch.zeros_like(k_pre)
    dv = torch.zeros(B, S, Hk, D, device="cuda")

    def step():
        o, lse, q, k, qr, kr = dev.fused_fwd(q_pre, k_pre, v, pr, ctx=ctx)
        dev.fused_bwd(d_o, q_pre, k_pre, q, k, v, o, lse, qr, kr, pr, dq_pre, dk_pre, dv, ctx=ctx)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    # Per-kernel times over untimed steps, each kernel bracketed alone; the
    # timed steps bracket the dK/dV kernel only, as the attention step's
    # timing does.
    kernels = {n: round(ms, 4) for n, (ms, _) in kernel_times(ctx, step, steps).items()}
    ctx.profile_select(["attn_bwd_dkdv"])
    ctx.profile_enable(True)
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    per = (time.perf_counter() - t0) / steps
    ctx.profile_enable(False)
    ctx.close()
    del q_pre, k_pre, v, d_o, dq_pre, dk_pre, dv, pr
    torch.cuda.empty_cache()
    flops = 7.0 * B * Hq * D * S * (S + 1)
    return {"value": round(flops / per / 1e12, 3), "unit": "TFLOP/s", "ms_per_step": round(per * 1e3, 4),
            "kernels_ms": kernels}


def layer_ops(a):
    """Times the layer ops of include/cfops.h at the SmolLM-135M training
    shape of the train tok/s metric (batch 8 x seq 512 = 4096 tokens, hidden
    576, FFN 1536, vocab 49152; crates/cli/src/cmd_bench.rs:43-99) and the
    train step itself with every op in libcfattn.so (backend "cfops") and
    with torch ops (backend "torch").  Each op's `achieved` is its
    algorithmic bytes (HBM-bound ops) or FLOPs (GEMM-bound ops) per call over
    its mean time, measured with HIP events on the stream the ops run on.
    Prints its own JSON line."""
    import torch

    from cpuforge_amd import ops as P
    from cpuforge_amd.train_bench import SMOLLM_135M, train_tok_s
    c = SMOLLM_135M
    t, d, f, V, r = 8 * 512, c["d"], c["ffn"], c["vocab"], 16
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    rn = lambda *s_, std=1.0: torch.randn(*s_, generator=g, device="cuda") * std  # noqa: E731
    x, w, y, rstd = rn(t, d), 1 + rn(d, std=0.1), torch.empty(t, d, device="cuda"), torch.empty(t, device="cuda")
    dx, dw = torch.zeros(t, d, device="cuda"), torch.zeros(d, device="cuda")
    gg, uu, hh = rn(t, f, std=2.0), rn(t, f), torch.empty(t, f, device="cuda")
    dg, du = torch.zeros(t, f, device="cuda"), torch.zeros(t, f, device="cuda")
    logits = rn(t, V, std=3.0)
    dl = torch.empty_like(logits)
    tg = torch.randint(0, V, (t,), generator=g, device="cuda")
    head = rn(V, d, std=0.02)
    dhn = torch.empty(t, d, device="cuda")
    wq, la, lb = rn(d, d, std=0.02), rn(r, d, std=0.04), rn(d, r, std=0.1)
    yq, xs = torch.empty(t, d, device="cuda"), torch.empty(t, r, device="cuda")
    ga, gb = torch.zeros(r, d, device="cuda"), torch.zeros(d, r, device="cuda")
    n_opt = 1 << 24
    pp, pg, pm, pv = rn(n_opt), rn(n_opt), torch.zeros(n_opt, device="cuda"), torch.zeros(n_opt, device="cuda")
    F = 4
    cases = {
        # name: (call, bytes or flops per call, bound)
        "rmsnorm_forward": (lambda: P.rmsnorm_forward(x, w, y, rstd, t, d, 1e-5), F * (2 * t * d + d + t), "hbm"),
        "rmsnorm_backward": (lambda: P.rmsnorm_backward(y, x, w, rstd, dx, dw, t, d), F * (4 * t * d + 2 * d + t),
                             "hbm"),
        "silu_mul_forward": (lambda: P.silu_mul_forward(gg, uu, hh), F * 3 * t * f, "hbm"),
        "silu_mul_backward": (lambda: P.silu_mul_backward(hh, gg, uu, dg, du), F * 7 * t * f, "hbm"),
        "cross_entropy_fwd_bwd": (lambda: P.cross_entropy_fwd_bwd(logits, tg, dl, t, V), F * 2 * t * V, "hbm"),
        "adamw_update": (lambda: P.adamw_update(pp, pg, pm, pv, 1, 1e-3, 0.9, 0.95, 1e-8, 0.1), F * 7 * n_opt,
                         "hbm"),
        "linear_forward_lora": (lambda: P.linear_forward(x, wq, t, d, d, yq, la, lb, 2.0, xs),
                                2.0 * t * d * (d + 2 * r), "mfma"),
        "linear_backward_lora": (lambda: P.linear_backward(x, xs, yq, wq, t, d, d, dx, None, ga, gb, la, lb, 2.0),
                                 2.0 * t * (d * d + 3 * d * r + r * d), "mfma"),
        "lm_head_ce": (lambda: P.lm_head_ce(x, head, tg, t, d, V, dhn), 2.0 * 2 * t * d * V, "mfma"),
    }
    out = {}
    for name, (fn, amount, bound) in cases.items():
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        n = 20
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / n
        if bound == "hbm":
            ach = amount / (ms * 1e-3) / 1e9
            out[name] = {"ms": round(ms, 4), "achieved": round(ach, 1), "unit": "GB/s", "peak": PEAK_HBM_GBS,
                         "frac": round(ach / PEAK_HBM_GBS, 4), "bytes": int(amount)}
        else:
            ach = amount / (ms * 1e-3) / 1e12
            out[name] = {"ms": round(ms, 4), "achieved": round(ach, 2), "unit": "TFLOP/s",
                         "peak": PEAK_TFLOPS["f32"], "frac": round(ach / PEAK_TFLOPS["f32"], 4), "flops": amount}
    del x, y, dx, gg, uu, hh, dg, du, logits, dl, head, pp, pg, pm, pv
    torch.cuda.empty_cache()
    train = {}
    for backend in ("cfops", "torch"):
        tr = train_tok_s(batch=8, seq=512, steps=a.train_steps, backend=backend)
        train[backend] = {"tok_s": round(tr["value"], 1), "ms_per_step": round(tr["ms_per_step"], 3),
                          "first_loss": round(tr["first_loss"], 5)}
    print(json.dumps({"metric": "SmolLM-135M train tok/s with the layer ops in libcfattn.so; per-op roofline",
                      "value": train["cfops"]["tok_s"], "unit": "tok/s", "higher_is_better": True,
                      "data": "synthetic (torch.randn / randint)", "dtype": "f32",
                      "config": {"workload": "SmolLM-135M LoRA r=16 train step, batch 8 x seq 512, 30 layers",
                                 "tokens": t, "hidden": d, "ffn": f, "vocab": V},
                      "train": train, "ops": out}), flush=True)


def _smollm_tensors():
    """(name, shape) of every SmolLM-135M parameter in visit_params order
    (crates/model/src/model.rs:179-208; tied embeddings, no LM head)."""
    from cpuforge_amd.train_bench import SMOLLM_135M as c
    d, f, hd = c["d"], c["ffn"], c["head_dim"]
    qd, kvd = c["heads"] * hd, c["kv_heads"] * hd
    out = [("model.embed_tokens.weight", (c["vocab"], d))]
    for i in range(30):
        p = f"model.layers.{i}"
        out += [(f"{p}.input_layernorm.weight", (d,)), (f"{p}.self_attn.q_proj.weight", (qd, d)),
                (f"{p}.self_attn.k_proj.weight", (kvd, d)), (f"{p}.self_attn.v_proj.weight", (kvd, d)),
                (f"{p}.self_attn.o_proj.weight", (d, qd)), (f"{p}.post_attention_layernorm.weight", (d,)),
                (f"{p}.mlp.gate_proj.weight", (f, d)), (f"{p}.mlp.up_proj.weight", (f, d)),
                (f"{p}.mlp.down_proj.weight", (d, f))]
    return out + [("model.norm.weight", (d,))]


def io_formats(a):
    """Times the on-disk formats of include/cfio.h at SmolLM-135M scale:
    the bf16 -> f32 widening kernel against HBM bandwidth (6 algorithmic
    bytes per element), loading the model's bf16 checkpoint into f32 HBM
    tensors (read_safetensors, crates/io/src/st.rs:19-45) and saving / loading
    a full-training state of it (p, m, v of every parameter, f32;
    train/src/state.rs) through the pinned staging chunks.  File throughput
    is quoted against the measured pinned-host <-> HBM copy rate, the ceiling
    of a page-cache-resident file.  cpu_baseline: the same load and save on
    host memory with the safetensors crate the reference links (0.8.0, through
    its Python binding) and the oracle's dtype.rs widening.  Prints its own
    JSON line."""
    import shutil
    import tempfile

    import numpy as np
    import torch

    from cpuforge_amd import st as S
    from oracle import oracle as O
    from safetensors.numpy import load_file as np_load_file
    from safetensors.numpy import save_file as np_save_file
    from safetensors.torch import save_file as torch_save_file

    def timed(fn, n):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        w0 = time.perf_counter()
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return max(e0.elapsed_time(e1), (time.perf_counter() - w0) * 1e3) / n

    def fresh_saves(save, n, tag):
        """Mean seconds of `n` saves, each to a new path (replacing an existing
        file adds the filesystem's replace-on-rename writeback to either
        writer); the files are removed outside the timed region."""
        total = 0.0
        for i in range(n):
            p = os.path.join(tmp, f"{tag}{i}.safetensors")
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            save(p)
            total += time.perf_counter() - t0
            os.remove(p)
        return total / n

    out = {}
    # 1. the widening kernel, HBM-resident in and out, and torch's own
    # bf16 -> f32 copy of the same tensor as a practical ceiling
    n = 1 << 28
    src = torch.randint(-32768, 32767, (n,), dtype=torch.int16, device="cuda")
    dst = torch.empty(n, dtype=torch.float32, device="cuda")
    for kind, fn in (("bf16", S.bf16_to_f32), ("f16", S.f16_to_f32)):
        ms = timed(lambda: fn(src, dst), 20)
        gbs = 6.0 * n / (ms * 1e-3) / 1e9
        out[f"widen_{kind}"] = {"ms": round(ms, 4), "achieved": round(gbs, 1), "unit": "GB/s", "peak": PEAK_HBM_GBS,
                                "frac": round(gbs / PEAK_HBM_GBS, 4), "bytes": 6 * n, "elements": n}
    ms = timed(lambda: dst.copy_(src.view(torch.bfloat16)), 20)
    out["torch_copy_bf16_to_f32"] = {"ms": round(ms, 4), "achieved": round(6.0 * n / (ms * 1e-3) / 1e9, 1)}
    del src, dst
    # 2. pinned host <-> HBM copy rates (the staging pipeline's ceiling)
    nb = 256 << 20
    hbuf = torch.empty(nb, dtype=torch.uint8, pin_memory=True)
    dbuf = torch.empty(nb, dtype=torch.uint8, device="cuda")
    h2d = nb / (timed(lambda: dbuf.copy_(hbuf, non_blocking=True), 10) * 1e-3) / 1e9
    d2h = nb / (timed(lambda: hbuf.copy_(dbuf, non_blocking=True), 10) * 1e-3) / 1e9
    del hbuf, dbuf
    out["pinned_copy_gbs"] = {"h2d": round(h2d, 1), "d2h": round(d2h, 1)}

    names = _smollm_tensors()
    g = torch.Generator().manual_seed(3)
    tmp = tempfile.mkdtemp(prefix="cfio_bench_")
    try:
        # 3. bf16 checkpoint -> f32 HBM tensors
        ck = os.path.join(tmp, "model.safetensors")
        host_bf16 = {nm: (torch.randn(shape, generator=g) * 0.02).to(torch.bfloat16) for nm, shape in names}
        torch_save_file(host_bf16, ck)
        ck_bytes = os.path.getsize(ck)
        numel = sum(t.numel() for t in host_bf16.values())
        del host_bf16
        load_ms = timed(lambda: S.read_safetensors(ck), 3)
        out["load_bf16_checkpoint"] = {"ms": round(load_ms, 2), "file_bytes": ck_bytes, "params": numel,
                                       "file_gbs": round(ck_bytes / (load_ms * 1e-3) / 1e9, 2),
                                       "frac_of_h2d": round(ck_bytes / (load_ms * 1e-3) / 1e9 / h2d, 3)}
        # 4. full-training state, f32 p / m / v
        dev_ts = [(f"{k}.{nm}", list(shape), torch.randn(shape, generator=g).cuda())
                  for nm, shape in names for k in ("p", "m", "v")]
        stp = os.path.join(tmp, "state.safetensors")
        meta = {"step": "100", "consumed": "800", "opt_step": "100"}
        S.write_safetensors(stp, dev_ts, meta)
        st_bytes = os.path.getsize(stp)
        save_s = fresh_saves(lambda p: S.write_safetensors(p, dev_ts, meta), 3, "ours")
        ld = S.read_safetensors(stp)
        ok = all(torch.equal(ld.tensors[nm], t) for nm, _, t in dev_ts)
        del ld
        read_ms = timed(lambda: S.read_safetensors(stp), 3)
        out["state_f32"] = {"tensors": len(dev_ts), "file_bytes": st_bytes, "roundtrip_bitwise": ok,
                            "save_ms": round(save_s * 1e3, 2), "save_gbs": round(st_bytes / save_s / 1e9, 2),
                            "save_frac_of_d2h": round(st_bytes / save_s / 1e9 / d2h, 3),
                            "load_ms": round(read_ms, 2), "load_gbs": round(st_bytes / (read_ms * 1e-3) / 1e9, 2),
                            "load_frac_of_h2d": round(st_bytes / (read_ms * 1e-3) / 1e9 / h2d, 3)}
        host_state = {nm: t.cpu().numpy() for nm, _, t in dev_ts}
        del dev_ts
        torch.cuda.empty_cache()
        # 5. cpu baseline: the crate on host memory, the oracle's widening
        cpu = {}
        if not a.no_cpu:
            from safetensors import safe_open

            def crate_load():
                with safe_open(ck, "pt") as f:
                    tensors = {k: f.get_tensor(k) for k in f.keys()}
                return {k: O.bf16_to_f32(v.view(torch.int16).numpy().view(np.uint16)) for k, v in tensors.items()}

            crate_load()
            t0 = time.perf_counter()
            for _ in range(3):
                crate_load()
            cpu_load_s = (time.perf_counter() - t0) / 3
            cpu_save_s = fresh_saves(lambda p: np_save_file(host_state, p, metadata=meta), 3, "crate")
            t0 = time.perf_counter()
            for _ in range(3):
                np_load_file(stp)
            cpu_read_s = (time.perf_counter() - t0) / 3
            cpu = {"value": round(ck_bytes / cpu_load_s / 1e9, 3), "unit": "GB/s (bf16 checkpoint load)",
                   "cores": 1, "kind": "port",
                   "sample": "whole workload, mean of 3: SmolLM-135M bf16 checkpoint read by the safetensors crate "
                             "0.8.0 (the reference's, via its Python binding) and widened by the oracle's dtype.rs "
                             "restatement; the f32 state saved (fresh paths) and read on host memory",
                   "state_save_gbs": round(st_bytes / cpu_save_s / 1e9, 3),
                   "state_load_gbs": round(st_bytes / cpu_read_s / 1e9, 3)}
        del host_state
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    w = out["widen_bf16"]
    traffic = read_traffic(os.path.join(ROOT, "profiles", "hbm_traffic_io_widen.md"), "widen4_kernel<bf16>", "io")
    print(json.dumps({"metric": "SmolLM-135M bf16 checkpoint load into f32 HBM tensors, GB/s of file",
                      "value": out["load_bf16_checkpoint"]["file_gbs"], "unit": "GB/s", "n_gpus": 1,
                      "higher_is_better": True, "vs_baseline": None, "dtype": "bf16->f32",
                      "data": "synthetic (torch.randn), files in the box's temp dir (page cache)",
                      "config": {"workload": "SmolLM-135M checkpoint and full-training state (cfio)",
                                 "params": out["load_bf16_checkpoint"]["params"]},
                      "roofline": {"bound": "hbm", "kernel": "widen4_kernel<bf16>", "achieved": w["achieved"],
                                   "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": w["frac"], "traffic": traffic},
                      "io": out, "cpu_baseline": cpu or None}), flush=True)


def kernel_times(ctx, step, steps, dominant=False):
    """{kernel: (ms per launch, launches)} from the library's hipEvents.  A
    pass with every launch bracketed names the kernels; each bracket adds
    queue time around its kernel, so each kernel is then timed in a pass of
    `steps` steps of its own in which only it is bracketed.  With `dominant`
    the kernel of the most time (among ALGO_UNITS) keeps the first pass's
    figure: the caller times it in its timed steps."""
    import torch

    ctx.profile_select(None)
    ctx.profile_enable(True)
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    every = {n: (t / c, c) for n, (t, c) in ctx.profile_read().items() if c}
    ctx.profile_enable(False)
    skip = None
    if dominant:
        skip = max((n for n in every if n in ALGO_UNITS), key=lambda n: every[n][0] * every[n][1])
    for n in list(every):
        if n == skip:
            continue
        ctx.profile_select([n])
        ctx.profile_enable(True)
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
        t, c = ctx.profile_read().get(n, (0.0, 0))
        ctx.profile_enable(False)
        if c:
            every[n] = (t / c, c)
    ctx.profile_select(None)
    return every


def attn_timing(cfg, mode, steps, warmup, ctx, traffic_file, copy_probe, zero_inputs=False):
    """Times `steps` attention steps (cfattn_fwd then cfattn_bwd on
    device-resident tensors) of config `cfg` after `warmup` untimed ones.
    Returns the step time (the larger of the hipEvent span and the host wall
    clock, over the steps), the whole-step TFLOP/s and the roofline of the
    kernel that takes the most time."""
    import torch

    import cpuforge_amd as cf
    from cpuforge_amd import device as dev
    B, S, Hq, Hk, D, theta, scaling, qk_norm = CONFIGS[cfg]
    torch.manual_seed(1234)
    dt = torch.bfloat16 if mode == "bf16" else torch.float32
    # Synthetic pre-RoPE q/k, v and upstream gradient, N(0,1).
    q_pre = torch.randn(B, S, Hq, D, device="cuda", dtype=torch.float32)
    k_pre = torch.randn(B, S, Hk, D, device="cuda", dtype=torch.float32)
    v = torch.randn(B, S, Hk, D, device="cuda", dtype=torch.float32).to(dt)
    d_o = torch.randn(B, S, Hq, D, device="cuda", dtype=torch.float32).to(dt)
    sc = cf.Llama3Scaling(*scaling) if scaling else None
    rope = cf.RopeCache(D, S, theta, sc)
    qn = kn = None
    if qk_norm:
        qn = (1.0 + 0.02 * torch.randn(D, device="cuda")).float()
        kn = (1.0 + 0.02 * torch.randn(D, device="cuda")).float()
    pr = dev.DeviceRope(rope, "cuda", 0, qn, kn, 1e-6)
    q, k, _, _ = dev.prologue_fwd(q_pre, k_pre, pr, dtype=dt, ctx=ctx)
    del q_pre, k_pre
    if zero_inputs:
        for t in (q, k, v, d_o):
            t.zero_()
    o = torch.empty(B, S, Hq, D, device="cuda", dtype=torch.float32)
    lse = torch.empty(B, Hq, S, device="cuda", dtype=torch.float32)
    dq = torch.zeros(B, S, Hq, D, device="cuda", dtype=torch.float32)
    dk = torch.zeros(B, S, Hk, D, device="cuda", dtype=torch.float32)
    dv = torch.zeros(B, S, Hk, D, device="cuda", dtype=torch.float32)

    def step():
        dev.fwd(q, k, v, o, lse, ctx=ctx)
        dev.bwd(d_o, q, k, v, o, lse, dq, dk, dv, ctx=ctx)

    if copy_probe:
        src = torch.empty(copy_probe << 18, device="cuda", dtype=torch.float32).fill_(1.0)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    print(f"bench: {cfg} {mode} warmup done ({warmup} steps)", file=sys.stderr, flush=True)

    # Per-kernel times, each kernel bracketed alone; the kernel that takes
    # the most time (the roofline's) is bracketed in the timed steps.
    every = kernel_times(ctx, step, steps, dominant=True)
    dom = max((n for n in every if n in ALGO_UNITS), key=lambda n: every[n][0] * every[n][1])
    ctx.profile_select([dom])
    ctx.profile_enable(True)
    stream = torch.cuda.current_stream()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    prof = ctx.profile_read()
    ctx.profile_enable(False)
    ctx.profile_select(None)
    gpu_ms = ev0.elapsed_time(ev1)
    ms_per_step = max(gpu_ms, wall * 1e3) / steps
    flops = 7.0 * B * Hq * D * S * (S + 1)
    tflops = flops / (ms_per_step * 1e-3) / 1e12
    print(f"bench: {cfg} {mode} timed {steps} steps, {ms_per_step:.3f} ms/step", file=sys.stderr, flush=True)

    kernels = dict(every)
    kernels[dom] = (prof[dom][0] / prof[dom][1], prof[dom][1])  # from the timed steps
    dom_ms = kernels[dom][0]
    dom_flops = ALGO_UNITS[dom] * B * Hq * D * S * (S + 1)
    achieved = dom_flops / (dom_ms * 1e-3) / 1e12
    peak = PEAK_TFLOPS[mode]
    tpath = traffic_file or os.path.join(ROOT, "profiles", f"hbm_traffic_{cfg}_{mode}.md")
    traffic = read_traffic(tpath, dom, f"{cfg}-{mode}")
    del q, k, v, d_o, o, lse, dq, dk, dv, pr
    torch.cuda.empty_cache()
    return {"value": round(tflops, 3), "ms_per_step": round(ms_per_step, 4),
            "pct_peak": round(100.0 * tflops / peak, 2),
            "kernels_ms": {n: round(m, 4) for n, (m, _) in kernels.items()},
            "roofline": {"bound": "mfma", "kernel": dom, "achieved": round(achieved, 3), "peak": peak,
                         "unit": "TFLOP/s", "frac": round(achieved / peak, 4), "traffic": traffic}}


def main():
    a = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if a.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: the attention op runs on a single MI355X here and this build has no "
              f"multi-GPU path (asked for --gpus {a.gpus}, WORLD_SIZE={world}).", file=sys.stderr)
        sys.exit(2)
    mode = a.mode or ("f32" if a.config == "C1" else "bf16")
    B, S, Hq, Hk, D, theta, scaling, qk_norm = CONFIGS[a.config]
    if a.host_slices:
        host_slices(a, mode)
        return
    if a.fused:
        fused_layer(a, mode)
        return
    if a.ops:
        layer_ops(a)
        return
    if a.io:
        io_formats(a)
        return
    if a.fwd_dist:
        fwd_distributions(a)
        return
    if a.power > 0:
        power_clock(a, mode)
        return
    if a.sweep:
        shape_sweep(a)
        return
    if a.energy > 0:
        energy_probes(a)
        return
    if a.peak:
        import cpuforge_amd as cf
        ctx = cf.Context(0)
        pk = peak_probe(ctx, runs=5)
        shapes = mfma_shape_probe(ctx, runs=5)
        ctx.close()
        print(json.dumps({"metric": "on-board bf16 MFMA ceiling (loop of v_mfma_f32_32x32x16_bf16, two waves per "
                                    "SIMD, every CU)", "value": pk["random"], "unit": "TFLOP/s", "n_gpus": 1,
                          "higher_is_better": True, "dtype": "bf16", "spec_peak": PEAK_TFLOPS["bf16"],
                          "frac_of_spec": round(pk["random"] / PEAK_TFLOPS["bf16"], 4), "zero_operands": pk["zeros"],
                          "mfma_shapes": shapes,
                          "data": "pseudo-random bf16 operands in registers (median of 5 runs of ~20 ms after a "
                                  "warm-up); zero_operands: the same loop on zeros; mfma_shapes: the 32x32x16 and "
                                  "16x16x32 loops alternating on the same operands"}), flush=True)
        return

    import torch

    import cpuforge_amd as cf

    if not torch.cuda.is_available():
        print("bench.py needs a GPU (torch.cuda.is_available() is False)", file=sys.stderr)
        sys.exit(1)
    ctx = cf.Context(0)
    if a.ds_limit is not None:
        ctx.ds_limit = a.ds_limit
    r = attn_timing(a.config, mode, a.steps, a.warmup, ctx, a.traffic_file, a.copy_probe, a.zero_inputs)
    pk = peak_probe(ctx) if mode == "bf16" else None
    out = {
        "metric": "attention fwd+bwd TFLOP/s + % MFMA peak at 1 MI355X; SmolLM-135M train tok/s",
        "value": r["value"],
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": r["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": mode,
        "data": ("ZERO inputs (diagnostic, not a benchmark figure)" if a.zero_inputs else
                 "synthetic (torch.randn N(0,1), RoPE prologue applied before timing)"),
        "config": {"workload": WORKLOAD[a.config], "config": a.config, "batch": B, "seq": S, "n_heads": Hq,
                   "n_kv": Hk, "head_dim": D, "mode": mode, "causal": True},
        "pct_peak": r["pct_peak"],
        "kernels_ms": r["kernels_ms"],
        "roofline": r["roofline"],
    }
    if pk:
        # The measured ceiling beside the spec peak (the roofline's `peak`).
        out["roofline"]["practical_peak"] = pk["random"]
        out["roofline"]["frac_practical"] = round(out["roofline"]["achieved"] / pk["random"], 4)
        out["roofline"]["practical_peak_zero_operands"] = pk["zeros"]
        out["pct_practical_peak"] = round(100.0 * r["value"] / pk["random"], 2)
    if not a.no_f32:
        # The reference's own precision: C2 (SmolLM-135M training batch) with
        # f32 inputs through the fp32 MFMA kernels.
        print("bench: C2 f32 ...", file=sys.stderr, flush=True)
        f = attn_timing("C2", "f32", a.sub_steps, 3, ctx, None, 0)
        out["f32"] = {"config": "C2", "workload": WORKLOAD["C2"], "dtype": "f32", "value": f["value"],
                      "unit": "TFLOP/s", "ms_per_step": f["ms_per_step"], "steps": a.sub_steps,
                      "pct_peak": f["pct_peak"], "kernels_ms": f["kernels_ms"], "roofline": f["roofline"]}
    if not a.no_configs and a.config == "C5" and mode == "bf16":
        # The other bf16 configurations of BASELINE.json, each its own step
        # of the same kind (cfattn_fwd + cfattn_bwd on device-resident
        # inputs); C4 also with its Layer-level step (q/k RMSNorm + RoPE).
        out["configs"] = {}
        for cfg in ("C4", "C3", "C2"):
            print(f"bench: {cfg} bf16 ...", file=sys.stderr, flush=True)
            c = attn_timing(cfg, "bf16", a.sub_steps, 3, ctx, None, 0)
            e = {"workload": WORKLOAD[cfg], "dtype": "bf16", "value": c["value"], "unit": "TFLOP/s",
                 "ms_per_step": c["ms_per_step"], "steps": a.sub_steps, "pct_peak": c["pct_peak"],
                 "kernels_ms": c["kernels_ms"], "roofline": c["roofline"]}
            if pk:
                e["pct_practical_peak"] = round(100.0 * c["value"] / pk["random"], 2)
                e["roofline"]["frac_practical"] = round(c["roofline"]["achieved"] / pk["random"], 4)
            if cfg == "C4" and not a.no_fused:
                fz = fused_timing(cfg, "bf16", a.sub_steps, 3)
                e["fused"] = {"path": "cfattn_fused_fwd/bwd", "ms_per_step": fz["ms_per_step"],
                              "over_attention_ms": round(fz["ms_per_step"] - c["ms_per_step"], 4),
                              "kernels_ms": fz["kernels_ms"]}
            out["configs"][cfg] = e
    if not a.no_fused:
        # The Layer-level step of the same config: the q/k prologue (RoPE,
        # and the Qwen3 norm where the config has it) forward and backward
        # around the attention.
        print(f"bench: {a.config} fused layer ...", file=sys.stderr, flush=True)
        fz = fused_timing(a.config, mode, a.sub_steps, 3)
        out["fused"] = {"config": a.config, "dtype": mode, "path": "cfattn_fused_fwd/bwd",
                        "value": fz["value"], "unit": "TFLOP/s (attention FLOPs only)",
                        "ms_per_step": fz["ms_per_step"], "steps": a.sub_steps,
                        "over_attention_ms": round(fz["ms_per_step"] - r["ms_per_step"], 4),
                        "kernels_ms": fz["kernels_ms"]}
    if not a.no_train:
        # SmolLM-135M LoRA r=16 train step (cmd_bench.rs:52-99), seq 512, batch 8,
        # f32 like the reference, attention through the fused GPU path.
        # The step is timed as replays of a HIP graph of it (the same kernels
        # in the same order, bitwise the eager step's results:
        # tests/test_gpu_train_graph.py), and eagerly beside it.
        from cpuforge_amd.train_bench import train_tok_s
        print("bench: SmolLM-135M train step ...", file=sys.stderr, flush=True)
        tr = train_tok_s(batch=8, seq=512, steps=a.train_steps, graph=True)
        ea = train_tok_s(batch=8, seq=512, steps=a.train_steps)
        tr["eager"] = {"value": round(ea["value"], 3), "ms_per_step": round(ea["ms_per_step"], 3)}
        tr["reference_tok_s"] = 122.0  # README.md:95, 2-core CPU, batch 1, same shape and LoRA
        out["smollm_train"] = {k: (round(v, 3) if isinstance(v, float) else v) for k, v in tr.items()}
    if not a.no_cpu:
        print("bench: cpu baseline ...", file=sys.stderr, flush=True)
        out["cpu_baseline"] = cpu_baseline(a.config, mode, a.cpu_heads, a.cpu_single_heads)
    else:
        out["cpu_baseline"] = None
    ctx.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
