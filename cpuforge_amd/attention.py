"""Host-side mirror of cpuforge's attention op (crates/core/src/ops/attention.rs).

Same names, argument order, layouts and conventions as the reference:

    attention_forward(q, k, v, o, lse, s)                       # attention.rs:42-44
    attention_forward_blocked(q, k, v, o, lse, s, q_block)      # attention.rs:46-54
    attention_backward(d_o, q, k, v, o, lse, dq, dk, dv, s)     # attention.rs:126-139
    attention_backward_blocked(..., s, q_block)                 # attention.rs:142-154

Buffers are float32 numpy arrays (the reference's `&[f32]` / `&mut [f32]`):
q, o, d_o, dq hold [seq, n_heads, head_dim]; k, v, dk, dv hold
[seq, n_kv, head_dim]; lse holds [n_heads, seq].  The forward overwrites o
and lse; the backward accumulates (+=) into dq, dk, dv.  A length mismatch
raises ShapeError (an AssertionError), where the reference panics.

The arithmetic runs on the GPU through libcfattn.so's host-slice entry
points; `set_mode("bf16")` switches the default context to bf16 inputs with
fp32 accumulation.  Results do not depend on q_block.
"""
from __future__ import annotations

import ctypes as C
import threading
from dataclasses import dataclass

import numpy as np

from . import _lib

DEFAULT_Q_BLOCK = 128  # attention.rs:18


@dataclass(frozen=True)
class AttnShape:
    """attention.rs:20-26."""
    seq: int
    n_heads: int
    n_kv: int
    head_dim: int

    def c(self) -> _lib.Shape:
        return _lib.Shape(self.seq, self.n_heads, self.n_kv, self.head_dim)


class Context:
    """One libcfattn context: a HIP device, a stream and a buffer pool."""

    def __init__(self, device: int = 0):
        self._lib = _lib.lib()
        h = C.c_void_p()
        rc = self._lib.cfattn_create(device, C.byref(h))
        if rc != _lib.OK:
            raise _lib.CfattnError(rc, f"cfattn_create(device={device}) failed (no usable HIP device?)")
        self.handle = h
        self.device = device

    def close(self):
        if self.handle:
            self._lib.cfattn_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_mode(self, mode: str):
        _lib.check(self._lib.cfattn_set_mode(self.handle, _dtype_code(mode)), self.handle)

    @property
    def mode(self) -> str:
        return "bf16" if self._lib.cfattn_get_mode(self.handle) == _lib.BF16 else "f32"

    def synchronize(self):
        _lib.check(self._lib.cfattn_synchronize(self.handle), self.handle)

    @property
    def stream(self) -> int:
        return self._lib.cfattn_stream(self.handle) or 0

    @property
    def ds_limit(self) -> int:
        """Bytes of device scratch the bf16 backward may keep to store dS, so
        that dQ needs no softmax recompute; 0 disables that path."""
        return int(self._lib.cfattn_get_ds_limit(self.handle))

    @ds_limit.setter
    def ds_limit(self, nbytes: int) -> None:
        _lib.check(self._lib.cfattn_set_ds_limit(self.handle, int(nbytes)), self.handle)

    def profile_enable(self, on: bool = True) -> None:
        """Bracket every kernel this context queues with hipEvents on its
        stream (enabling again resets the totals)."""
        _lib.check(self._lib.cfattn_profile_enable(self.handle, int(bool(on))), self.handle)

    def profile_select(self, names=None) -> None:
        """Bracket only the named kernels ("attn_bwd_dkdv", ...) while
        profiling; None selects every kernel."""
        if names is None:
            mask = 0xFFFFFFFF
        else:
            ids = {self._lib.cfattn_kernel_name(k).decode(): k for k in range(self._lib.cfattn_kernel_count())}
            mask = 0
            for n in names:
                if n not in ids:
                    raise ValueError(f"unknown kernel {n!r}")
                mask |= 1 << ids[n]
        _lib.check(self._lib.cfattn_profile_select(self.handle, mask), self.handle)

    def fwd_stats_enable(self, on: bool = True) -> None:
        """Count the bf16 head_dim-128 forward's settled wave-tiles from now
        on (enabling again restarts the count); off frees the counter."""
        _lib.check(self._lib.cfattn_fwd_stats_enable(self.handle, int(bool(on))), self.handle)

    def fwd_stats_read(self) -> int:
        """Settled wave-tiles since cfattn_fwd_stats_enable."""
        n = C.c_longlong()
        _lib.check(self._lib.cfattn_fwd_stats_read(self.handle, C.byref(n)), self.handle)
        return n.value

    def probe_mfma_peak(self, zeros: bool = False, iters: int = 40000) -> float:
        """TFLOP/s of a loop of bf16 32x32x16 MFMAs on every SIMD, on
        pseudo-random operands (or zeros): the on-board ceiling of the bf16
        roofline (cfattn_probe_mfma_peak)."""
        out = C.c_double()
        _lib.check(self._lib.cfattn_probe_mfma_peak(self.handle, int(bool(zeros)), int(iters), C.byref(out)),
                   self.handle)
        return out.value

    def probe_loop(self, kind: str, iters: int = 20000) -> float:
        """Rate of a loop of one instruction class on every SIMD
        (cfattn_probe_loop): "lds" (16-byte LDS reads, bytes/s), "valu"
        (v_fma_f32, lane operations/s) or "mfma16" (bf16 16x16x32 MFMAs on
        pseudo-random operands, FLOP/s)."""
        code = {"lds": 0, "valu": 1, "mfma16": 2}[kind]
        out = C.c_double()
        _lib.check(self._lib.cfattn_probe_loop(self.handle, code, int(iters), C.byref(out)), self.handle)
        return out.value

    def profile_read(self) -> dict:
        """{kernel name: (total ms, launches)} since profiling was enabled."""
        out = {}
        for kid in range(self._lib.cfattn_kernel_count()):
            ms = C.c_double()
            n = C.c_longlong()
            _lib.check(self._lib.cfattn_profile_read(self.handle, kid, C.byref(ms), C.byref(n)), self.handle)
            out[self._lib.cfattn_kernel_name(kid).decode()] = (ms.value, n.value)
        return out


def _dtype_code(mode) -> int:
    if mode in ("f32", "fp32", "float32", _lib.F32):
        return _lib.F32
    if mode in ("bf16", "bfloat16", _lib.BF16):
        return _lib.BF16
    raise ValueError(f"unknown mode {mode!r} (f32 or bf16)")


_default = None
_default_lock = threading.Lock()


def default_context() -> Context:
    """The process-wide context the reference-shaped functions use (device 0)."""
    global _default
    if _default is None:
        with _default_lock:
            if _default is None:
                _default = Context(0)
    return _default


def set_mode(mode: str) -> None:
    """Arithmetic of the reference-shaped functions: "f32" or "bf16"."""
    default_context().set_mode(mode)


def _slice(x, name: str, writable: bool):
    if not isinstance(x, np.ndarray) or x.dtype != np.float32:
        raise TypeError(f"{name} must be a float32 numpy array")
    if not x.flags.c_contiguous:
        raise TypeError(f"{name} must be C-contiguous")
    if writable and not x.flags.writeable:
        raise TypeError(f"{name} must be writable")
    return x.ctypes.data, x.size


def attention_forward(q, k, v, o, lse, s: AttnShape, ctx: Context | None = None) -> None:
    attention_forward_blocked(q, k, v, o, lse, s, DEFAULT_Q_BLOCK, ctx)


def attention_forward_blocked(q, k, v, o, lse, s: AttnShape, q_block: int, ctx: Context | None = None) -> None:
    ctx = ctx or default_context()
    args = [*_slice(q, "q", False), *_slice(k, "k", False), *_slice(v, "v", False), *_slice(o, "o", True),
            *_slice(lse, "lse", True)]
    rc = ctx._lib.cfattn_attention_forward_blocked(ctx.handle, *args, s.c(), q_block)
    _lib.check(rc, ctx.handle)


def attention_backward(d_o, q, k, v, o, lse, dq, dk, dv, s: AttnShape, ctx: Context | None = None) -> None:
    attention_backward_blocked(d_o, q, k, v, o, lse, dq, dk, dv, s, DEFAULT_Q_BLOCK, ctx)


def attention_backward_blocked(d_o, q, k, v, o, lse, dq, dk, dv, s: AttnShape, q_block: int,
                               ctx: Context | None = None) -> None:
    ctx = ctx or default_context()
    args = [*_slice(d_o, "d_o", False), *_slice(q, "q", False), *_slice(k, "k", False), *_slice(v, "v", False),
            *_slice(o, "o", False), *_slice(lse, "lse", False), *_slice(dq, "dq", True), *_slice(dk, "dk", True),
            *_slice(dv, "dv", True)]
    rc = ctx._lib.cfattn_attention_backward_blocked(ctx.handle, *args, s.c(), q_block)
    _lib.check(rc, ctx.handle)


def flops_fwd_bwd(s: AttnShape, batch: int = 1) -> float:
    """Algorithmic FLOPs of one forward + backward: 7*B*Hq*D*S*(S+1)."""
    return _lib.lib().cfattn_flops_fwd_bwd(s.c(), batch)
