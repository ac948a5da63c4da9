"""Shared test data: the reference's attention test cases and the benchmark
configurations, with inputs drawn from the reference's RNG (restated in the
oracle).  Imported by the tests and by bench.py's cpu_baseline leg only.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from oracle import oracle as O

# (seq, heads, kv heads, head_dim, q_block): multiple blocks, ragged last
# block, GQA, MHA, MQA -- crates/core/src/ops/attention.rs:321-322.
CASES = [(8, 4, 2, 6, 3), (10, 3, 1, 4, 4), (7, 2, 2, 8, 100), (13, 6, 2, 4, 5), (1, 2, 1, 4, 4)]


def case(seq, n_heads, n_kv, hd, seed):
    """`case()` of attention.rs:310-318: q, k, v from seeds s, s+1, s+2, std 1."""
    return (O.rand(seq * n_heads * hd, seed, 1.0), O.rand(seq * n_kv * hd, seed + 1, 1.0),
            O.rand(seq * n_kv * hd, seed + 2, 1.0))


@dataclass(frozen=True)
class Config:
    name: str
    batch: int
    seq: int
    n_heads: int
    n_kv: int
    head_dim: int
    std: float
    theta: float
    modes: tuple
    scaling: tuple | None = None  # (factor, low, high, original_max_position)
    qk_norm: bool = False
    eps: float = 1e-6
    extra: dict = field(default_factory=dict)

    @property
    def group(self):
        return self.n_heads // self.n_kv

    def flops(self):
        return 7.0 * self.batch * self.n_heads * self.head_dim * self.seq * (self.seq + 1)


# BASELINE.json configs[0..4]
CONFIGS = {
    "C1": Config("C1", 1, 512, 9, 3, 64, 0.5, 1e4, ("f32",)),
    "C2": Config("C2", 8, 2048, 9, 3, 64, 0.5, 1e4, ("f32", "bf16")),
    "C3": Config("C3", 4, 4096, 32, 8, 64, 1.0, 5e5, ("bf16",), scaling=(32.0, 1.0, 4.0, 8192.0)),
    "C4": Config("C4", 4, 4096, 16, 8, 128, 1.0, 1e6, ("bf16",), qk_norm=True),
    "C5": Config("C5", 1, 8192, 32, 8, 128, 1.0, 5e5, ("bf16",)),
}


def seq_inputs(cfg: Config, b: int, base: int = 1000):
    """Sequence b's pre-prologue q, k, v, dO: seeds base+16b+{0,1,2,3}, std cfg.std."""
    s, hq, hk, d = cfg.seq, cfg.n_heads, cfg.n_kv, cfg.head_dim
    sd = base + 16 * b
    return (O.rand(s * hq * d, sd + 0, cfg.std), O.rand(s * hk * d, sd + 1, cfg.std), O.rand(s * hk * d, sd + 2, cfg.std),
            O.rand(s * hq * d, sd + 3, cfg.std))


def norm_gains(cfg: Config, base: int = 1000):
    """C4's q/k RMSNorm gains 1 + 0.02 N(0,1) from seeds base+4, base+5."""
    d = cfg.head_dim
    return (1.0 + O.rand(d, base + 4, 0.02)).astype(np.float32), (1.0 + O.rand(d, base + 5, 0.02)).astype(np.float32)


def rope_tables(cfg: Config, max_pos=None):
    return O.rope_table(cfg.head_dim, max_pos or cfg.seq, cfg.theta, cfg.scaling)


def rel_err(a, r) -> float:
    """max|a - r| / max|r| (the bf16 parity metric)."""
    a = np.asarray(a, dtype=np.float64)
    r = np.asarray(r, dtype=np.float64)
    den = np.abs(r).max()
    return float(np.abs(a - r).max() / (den if den > 0 else 1.0))


def grad_metric(a, r) -> float:
    """max |a - r| / (1 + |r|): the reference's gradcheck metric
    (crates/core/src/gradcheck.rs:31-48), reported beside rel_err for bf16."""
    a = np.asarray(a, dtype=np.float64)
    r = np.asarray(r, dtype=np.float64)
    return float((np.abs(a - r) / (1.0 + np.abs(r))).max())


def max_abs(a, r) -> float:
    return float(np.abs(np.asarray(a, dtype=np.float64) - np.asarray(r, dtype=np.float64)).max())
