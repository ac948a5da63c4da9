"""RoPE tables for the fused attention prologue (crates/core/src/ops/rope.rs).

`RopeCache(head_dim, max_pos, theta, scaling)` builds the reference's cos/sin
tables [max_pos, head_dim/2] (computed in f64, rounded to f32; rope.rs:46-63)
through libcfattn's host helper; the rotation itself runs on the GPU inside
the prologue kernels.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _lib


@dataclass(frozen=True)
class Llama3Scaling:
    """rope.rs:16-22; `apply` is Llama3Scaling::apply (rope.rs:26-38)."""
    factor: float
    low_freq_factor: float
    high_freq_factor: float
    original_max_position: float

    def c(self) -> _lib.Llama3ScalingC:
        return _lib.Llama3ScalingC(self.factor, self.low_freq_factor, self.high_freq_factor,
                                   self.original_max_position)

    def apply(self, inv_freq: float) -> float:
        sc = self.c()
        return _lib.lib().cfattn_llama3_scale(C.byref(sc), float(inv_freq))


class RopeCache:
    """rope.rs:6-12 / 41-63: cos and sin as float32 arrays [max_pos, head_dim/2]."""

    def __init__(self, head_dim: int, max_pos: int, theta: float, scaling: Llama3Scaling | None = None):
        if head_dim % 2 != 0:
            raise _lib.ShapeError(_lib.ERR_SHAPE, "head_dim must be even")
        self.head_dim = head_dim
        self.half = head_dim // 2
        self.max_pos = max_pos
        self.theta = theta
        self.scaling = scaling
        self.cos = np.empty((max_pos, self.half), dtype=np.float32)
        self.sin = np.empty((max_pos, self.half), dtype=np.float32)
        sc = scaling.c() if scaling is not None else None
        rc = _lib.lib().cfattn_rope_table(head_dim, max_pos, float(theta), C.byref(sc) if sc is not None else None,
                                          self.cos.ctypes.data, self.sin.ctypes.data)
        _lib.check(rc)

    @classmethod
    def new(cls, head_dim: int, max_pos: int, theta: float) -> "RopeCache":
        return cls(head_dim, max_pos, theta)

    @classmethod
    def with_scaling(cls, head_dim: int, max_pos: int, theta: float, scaling: Llama3Scaling | None) -> "RopeCache":
        return cls(head_dim, max_pos, theta, scaling)
