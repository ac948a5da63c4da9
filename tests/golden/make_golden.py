"""Writes the golden fixtures in tests/golden/ (run from the repo root:
`python tests/golden/make_golden.py`).

cpuforge ships no stored vectors (its tests generate data from seeds), so
these fixtures are computed here, independently of the C oracle:
  * rng.json   -- the reference RNG (crates/core/src/rng.rs:10-36) restated in
                  pure Python integers; Box-Muller uses the C library's
                  logf/cosf/sqrtf through ctypes, as Rust's f32 ln/cos/sqrt
                  do on Linux.
  * attn_cases.npz -- the reference's attention CASES (attention.rs:321-322)
                  with its seeds (forward 10+i, backward 50+i, upstream
                  gradient 70+i; attention.rs:325-326, 373-374): inputs from
                  the Python RNG, expected O, lse, dQ, dK, dV from torch
                  float64 (scaled_dot_product_attention, is_causal, GQA
                  heads repeated h -> h // group, autograd).
  * rope.npz   -- cos/sin tables in float64 closed form rounded to float32
                  (rope.rs:46-63), plain and Llama-3-scaled
                  (factor 32, low 1, high 4, original 8192; rope.rs:26-38).
"""
from __future__ import annotations

import ctypes
import ctypes.util
import json
import math
import os
import struct

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
M64 = (1 << 64) - 1

_libm = ctypes.CDLL(ctypes.util.find_library("m"))
for _fn in ("logf", "cosf", "sqrtf"):
    getattr(_libm, _fn).restype = ctypes.c_float
    getattr(_libm, _fn).argtypes = [ctypes.c_float]


def f32(x: float) -> float:
    return struct.unpack("f", struct.pack("f", x))[0]


class PyRng:
    def __init__(self, seed: int):
        self.state = ((seed ^ 0x9E3779B97F4A7C15) | 1) & M64

    def next_u64(self) -> int:
        x = self.state
        x ^= x >> 12
        x ^= (x << 25) & M64
        x ^= x >> 27
        self.state = x
        return (x * 0x2545F4914F6CDD1D) & M64

    def uniform(self) -> float:
        return f32(float(self.next_u64() >> 40) / float(1 << 24))

    def normal(self) -> float:
        u1 = max(self.uniform(), f32(1e-12))
        u2 = self.uniform()
        two_pi = f32(2.0 * f32(math.pi))
        a = _libm.sqrtf(f32(-2.0 * _libm.logf(u1)))
        b = _libm.cosf(f32(two_pi * u2))
        return f32(a * b)


def rand(n: int, seed: int, std: float = 1.0) -> np.ndarray:
    r = PyRng(seed)
    return np.array([f32(r.normal() * std) for _ in range(n)], dtype=np.float32)


CASES = [(8, 4, 2, 6, 3), (10, 3, 1, 4, 4), (7, 2, 2, 8, 100), (13, 6, 2, 4, 5), (1, 2, 1, 4, 4)]


def torch_attention(q, k, v, seq, nh, nkv, hd):
    """float64 causal GQA attention in torch; returns (o, lse) as tensors with graph."""
    group = nh // nkv
    qt = q.view(seq, nh, hd).transpose(0, 1)
    kt = k.view(seq, nkv, hd).transpose(0, 1).repeat_interleave(group, dim=0)
    vt = v.view(seq, nkv, hd).transpose(0, 1).repeat_interleave(group, dim=0)
    o = torch.nn.functional.scaled_dot_product_attention(qt.unsqueeze(0), kt.unsqueeze(0), vt.unsqueeze(0),
                                                         is_causal=True)[0]
    scores = (qt @ kt.transpose(1, 2)) / math.sqrt(hd)
    mask = torch.ones(seq, seq, dtype=torch.bool).tril()
    lse = torch.logsumexp(scores.masked_fill(~mask, float("-inf")), dim=-1)
    return o.transpose(0, 1).reshape(-1), lse.reshape(-1)


def make_rng():
    out = {}
    for seed in (0, 1, 7, 10, 42, 1000, 2**63 + 5):
        r = PyRng(seed)
        u64 = [r.next_u64() for _ in range(8)]
        r = PyRng(seed)
        uni = [r.uniform() for _ in range(8)]
        r = PyRng(seed)
        nor = [r.normal() for _ in range(8)]
        out[str(seed)] = {
            "u64": [str(x) for x in u64],
            "uniform_bits": [struct.unpack("I", struct.pack("f", x))[0] for x in uni],
            "normal_bits": [struct.unpack("I", struct.pack("f", x))[0] for x in nor],
        }
    with open(os.path.join(HERE, "rng.json"), "w") as f:
        json.dump(out, f, indent=1)


def make_attn():
    arrays = {}
    for i, (seq, nh, nkv, hd, qb) in enumerate(CASES):
        for kind, seed in (("fwd", 10 + i), ("bwd", 50 + i)):
            q = rand(seq * nh * hd, seed)
            k = rand(seq * nkv * hd, seed + 1)
            v = rand(seq * nkv * hd, seed + 2)
            tq, tk, tv = (torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in (q, k, v))
            o, lse = torch_attention(tq, tk, tv, seq, nh, nkv, hd)
            pre = f"c{i}_{kind}_"
            arrays[pre + "q"], arrays[pre + "k"], arrays[pre + "v"] = q, k, v
            arrays[pre + "o"] = o.detach().numpy()
            arrays[pre + "lse"] = lse.detach().numpy()
            if kind == "bwd":
                g = rand(seq * nh * hd, 70 + i)
                (o * torch.tensor(g, dtype=torch.float64)).sum().backward()
                arrays[pre + "g"] = g
                arrays[pre + "dq"] = tq.grad.numpy()
                arrays[pre + "dk"] = tk.grad.numpy()
                arrays[pre + "dv"] = tv.grad.numpy()
    np.savez_compressed(os.path.join(HERE, "attn_cases.npz"), **arrays)


def llama3(inv_freq, factor, low, high, orig):
    wavelen = 2.0 * math.pi / inv_freq
    lo_w, hi_w = orig / low, orig / high
    if wavelen < hi_w:
        return inv_freq
    if wavelen > lo_w:
        return inv_freq / factor
    smooth = (orig / wavelen - low) / (high - low)
    return (1.0 - smooth) * inv_freq / factor + smooth * inv_freq


def make_rope():
    arrays = {}
    for name, hd, max_pos, theta, sc in (("plain", 16, 32, 10000.0, None), ("llama3", 64, 40, 500000.0,
                                                                            (32.0, 1.0, 4.0, 8192.0))):
        half = hd // 2
        cos = np.zeros((max_pos, half), np.float32)
        sin = np.zeros((max_pos, half), np.float32)
        for pos in range(max_pos):
            for i in range(half):
                f = theta ** (-(2.0 * i) / hd)
                if sc:
                    f = llama3(f, *sc)
                cos[pos, i] = np.float32(math.cos(pos * f))
                sin[pos, i] = np.float32(math.sin(pos * f))
        arrays[name + "_cos"] = cos
        arrays[name + "_sin"] = sin
    np.savez_compressed(os.path.join(HERE, "rope.npz"), **arrays)


if __name__ == "__main__":
    make_rng()
    make_attn()
    make_rope()
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith((".json", ".npz"))))
