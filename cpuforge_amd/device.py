"""Device-tensor entry points over libcfattn's batched C ABI.

torch is used only for device memory and the current HIP stream: tensors are
handed to the kernels by pointer.  Layouts (contiguous, row-major):
    q, o, d_o, dq : [B, S, n_heads, D]      k, v, dk, dv : [B, S, n_kv, D]
    lse           : [B, n_heads, S]
q/k/v/d_o are float32 (fp32 parity mode) or bfloat16 (bf16 inputs, fp32
accumulation); o, lse and all gradients are float32.  Forward overwrites o
and lse; backward accumulates into dq, dk, dv (crates/core/src/ops/mod.rs:1-6).
"""
from __future__ import annotations

import ctypes as C

import torch

from . import _lib
from .attention import AttnShape, Context, default_context
from .rope import RopeCache


def _code(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return _lib.F32
    if t.dtype == torch.bfloat16:
        return _lib.BF16
    raise TypeError(f"unsupported dtype {t.dtype} (float32 or bfloat16)")


def _need(t: torch.Tensor, name: str, shape=None, dtype=None) -> None:
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError(f"{name} must be a device tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise _lib.ShapeError(_lib.ERR_SHAPE, f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
    if dtype is not None and t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")


def _batched(q: torch.Tensor, k: torch.Tensor):
    if q.dim() == 3:
        q, k = q.unsqueeze(0), k.unsqueeze(0)
    if q.dim() != 4 or k.dim() != 4:
        raise _lib.ShapeError(_lib.ERR_SHAPE, "q, k must be [B, S, H, D] or [S, H, D]")
    B, S, H, D = q.shape
    if k.shape[0] != B or k.shape[1] != S or k.shape[3] != D:
        raise _lib.ShapeError(_lib.ERR_SHAPE, f"k shape {tuple(k.shape)} does not match q {tuple(q.shape)}")
    return B, AttnShape(S, H, k.shape[2], D)


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def fwd(q, k, v, o=None, lse=None, ctx: Context | None = None):
    """Causal GQA attention forward; returns (o, lse)."""
    ctx = ctx or default_context()
    B, s = _batched(q, k)
    dt = _code(q)
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _need(t, n, dtype=q.dtype)
    if v.shape != k.shape:
        raise _lib.ShapeError(_lib.ERR_SHAPE, "v must have k's shape")
    oshape = (B, s.seq, s.n_heads, s.head_dim) if q.dim() == 4 else (s.seq, s.n_heads, s.head_dim)
    lshape = (B, s.n_heads, s.seq) if q.dim() == 4 else (s.n_heads, s.seq)
    if o is None:
        o = torch.empty(oshape, dtype=torch.float32, device=q.device)
    if lse is None:
        lse = torch.empty(lshape, dtype=torch.float32, device=q.device)
    _need(o, "o", oshape, torch.float32)
    _need(lse, "lse", lshape, torch.float32)
    rc = ctx._lib.cfattn_fwd(ctx.handle, s.c(), B, dt, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                             lse.data_ptr(), _stream())
    _lib.check(rc, ctx.handle)
    return o, lse


def bwd(d_o, q, k, v, o, lse, dq=None, dk=None, dv=None, ctx: Context | None = None):
    """Backward; accumulates into dq, dk, dv (zero-initialised if None)."""
    ctx = ctx or default_context()
    B, s = _batched(q, k)
    dt = _code(q)
    for t, n in ((d_o, "d_o"), (q, "q"), (k, "k"), (v, "v")):
        _need(t, n, dtype=q.dtype)
    _need(d_o, "d_o", q.shape)
    _need(o, "o", q.shape, torch.float32)
    _need(lse, "lse", (B, s.n_heads, s.seq) if q.dim() == 4 else (s.n_heads, s.seq), torch.float32)
    if dq is None:
        dq = torch.zeros(q.shape, dtype=torch.float32, device=q.device)
    if dk is None:
        dk = torch.zeros(k.shape, dtype=torch.float32, device=q.device)
    if dv is None:
        dv = torch.zeros(k.shape, dtype=torch.float32, device=q.device)
    _need(dq, "dq", q.shape, torch.float32)
    _need(dk, "dk", k.shape, torch.float32)
    _need(dv, "dv", k.shape, torch.float32)
    rc = ctx._lib.cfattn_bwd(ctx.handle, s.c(), B, dt, d_o.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                             o.data_ptr(), lse.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), _stream())
    _lib.check(rc, ctx.handle)
    return dq, dk, dv


class DeviceRope:
    """A RopeCache's tables on the device, plus the prologue's settings."""

    def __init__(self, rope: RopeCache, device="cuda", pos0: int = 0, q_norm=None, k_norm=None, eps: float = 1e-6):
        self.rope = rope
        self.cos = torch.from_numpy(rope.cos).to(device)
        self.sin = torch.from_numpy(rope.sin).to(device)
        self.pos0 = pos0
        self.q_norm = q_norm
        self.k_norm = k_norm
        self.eps = eps

    def c(self) -> _lib.PrologueC:
        return _lib.PrologueC(self.cos.data_ptr(), self.sin.data_ptr(), self.rope.max_pos, self.pos0,
                              self.q_norm.data_ptr() if self.q_norm is not None else None,
                              self.k_norm.data_ptr() if self.k_norm is not None else None, float(self.eps))


def prologue_fwd(q_pre, k_pre, pr: DeviceRope, dtype=torch.float32, ctx: Context | None = None):
    """Layer::forward's prologue (layer.rs:104-116); returns (q, k, q_rstd, k_rstd)."""
    ctx = ctx or default_context()
    B, s = _batched(q_pre, k_pre)
    _need(q_pre, "q_pre", dtype=torch.float32)
    _need(k_pre, "k_pre", dtype=torch.float32)
    q = torch.empty(q_pre.shape, dtype=dtype, device=q_pre.device)
    k = torch.empty(k_pre.shape, dtype=dtype, device=q_pre.device)
    q_rstd = k_rstd = None
    if pr.q_norm is not None:
        q_rstd = torch.empty(B * s.seq * s.n_heads, dtype=torch.float32, device=q_pre.device)
        k_rstd = torch.empty(B * s.seq * s.n_kv, dtype=torch.float32, device=q_pre.device)
    prc = pr.c()
    rc = ctx._lib.cfattn_prologue_fwd(ctx.handle, s.c(), B, _code(q), C.byref(prc), q_pre.data_ptr(),
                                      k_pre.data_ptr(), q.data_ptr(), k.data_ptr(),
                                      q_rstd.data_ptr() if q_rstd is not None else None,
                                      k_rstd.data_ptr() if k_rstd is not None else None, _stream())
    _lib.check(rc, ctx.handle)
    return q, k, q_rstd, k_rstd


def prologue_bwd(dq, dk, q_pre, k_pre, q_rstd, k_rstd, pr: DeviceRope, dq_pre=None, dk_pre=None, dq_norm=None,
                 dk_norm=None, ctx: Context | None = None):
    """Layer::backward after attention (layer.rs:191-206); accumulates into
    dq_pre, dk_pre (and the norm-gain gradients); returns them."""
    ctx = ctx or default_context()
    B, s = _batched(dq, dk)
    dev = dq.device
    if dq_pre is None:
        dq_pre = torch.zeros(dq.shape, dtype=torch.float32, device=dev)
    if dk_pre is None:
        dk_pre = torch.zeros(dk.shape, dtype=torch.float32, device=dev)
    if pr.q_norm is not None:
        if dq_norm is None:
            dq_norm = torch.zeros(s.head_dim, dtype=torch.float32, device=dev)
        if dk_norm is None:
            dk_norm = torch.zeros(s.head_dim, dtype=torch.float32, device=dev)
    ptr = lambda t: t.data_ptr() if t is not None else None  # noqa: E731
    prc = pr.c()
    rc = ctx._lib.cfattn_prologue_bwd(ctx.handle, s.c(), B, C.byref(prc), dq.data_ptr(), dk.data_ptr(), ptr(q_pre),
                                      ptr(k_pre), ptr(q_rstd), ptr(k_rstd), dq_pre.data_ptr(), dk_pre.data_ptr(),
                                      ptr(dq_norm), ptr(dk_norm), _stream())
    _lib.check(rc, ctx.handle)
    return dq_pre, dk_pre, dq_norm, dk_norm


def fused_fwd(q_pre, k_pre, v, pr: DeviceRope, ctx: Context | None = None):
    """Prologue + attention forward in one library call.  v's dtype selects
    the mode.  Returns (o, lse, q, k, q_rstd, k_rstd)."""
    ctx = ctx or default_context()
    B, s = _batched(q_pre, k_pre)
    dev = q_pre.device
    q = torch.empty(q_pre.shape, dtype=v.dtype, device=dev)
    k = torch.empty(k_pre.shape, dtype=v.dtype, device=dev)
    o = torch.empty(q_pre.shape, dtype=torch.float32, device=dev)
    lse = torch.empty((B, s.n_heads, s.seq) if q_pre.dim() == 4 else (s.n_heads, s.seq), dtype=torch.float32,
                      device=dev)
    q_rstd = k_rstd = None
    if pr.q_norm is not None:
        q_rstd = torch.empty(B * s.seq * s.n_heads, dtype=torch.float32, device=dev)
        k_rstd = torch.empty(B * s.seq * s.n_kv, dtype=torch.float32, device=dev)
    ptr = lambda t: t.data_ptr() if t is not None else None  # noqa: E731
    prc = pr.c()
    rc = ctx._lib.cfattn_fused_fwd(ctx.handle, s.c(), B, _code(v), C.byref(prc), q_pre.data_ptr(), k_pre.data_ptr(),
                                   v.data_ptr(), q.data_ptr(), k.data_ptr(), ptr(q_rstd), ptr(k_rstd), o.data_ptr(),
                                   lse.data_ptr(), _stream())
    _lib.check(rc, ctx.handle)
    return o, lse, q, k, q_rstd, k_rstd


def fused_bwd(d_o, q_pre, k_pre, q, k, v, o, lse, q_rstd, k_rstd, pr: DeviceRope, dq_pre=None, dk_pre=None, dv=None,
              dq_norm=None, dk_norm=None, ctx: Context | None = None):
    """Attention backward + prologue backward; accumulates and returns
    (dq_pre, dk_pre, dv, dq_norm, dk_norm)."""
    ctx = ctx or default_context()
    B, s = _batched(q_pre, k_pre)
    dev = q_pre.device
    z = lambda shape: torch.zeros(shape, dtype=torch.float32, device=dev)  # noqa: E731
    dq_pre = z(q_pre.shape) if dq_pre is None else dq_pre
    dk_pre = z(k_pre.shape) if dk_pre is None else dk_pre
    dv = z(k_pre.shape) if dv is None else dv
    if pr.q_norm is not None:
        dq_norm = z(s.head_dim) if dq_norm is None else dq_norm
        dk_norm = z(s.head_dim) if dk_norm is None else dk_norm
    ptr = lambda t: t.data_ptr() if t is not None else None  # noqa: E731
    prc = pr.c()
    rc = ctx._lib.cfattn_fused_bwd(ctx.handle, s.c(), B, _code(q), C.byref(prc), d_o.data_ptr(), q_pre.data_ptr(),
                                   k_pre.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                   lse.data_ptr(), ptr(q_rstd), ptr(k_rstd), dq_pre.data_ptr(), dk_pre.data_ptr(),
                                   dv.data_ptr(), ptr(dq_norm), ptr(dk_norm), _stream())
    _lib.check(rc, ctx.handle)
    return dq_pre, dk_pre, dv, dq_norm, dk_norm


class CausalGQAAttention(torch.autograd.Function):
    """torch autograd wrapper: o = attention(q, k, v); backward through the
    HIP kernels.  q/k/v [B,S,H,D] float32 or bfloat16; o is float32."""

    @staticmethod
    def forward(fctx, q, k, v):
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        o, lse = fwd(q, k, v)
        fctx.save_for_backward(q, k, v, o, lse)
        return o

    @staticmethod
    def backward(fctx, g):
        q, k, v, o, lse = fctx.saved_tensors
        d_o = g.contiguous().to(q.dtype)
        dq, dk, dv = bwd(d_o, q, k, v, o, lse)
        return dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype)


def attention(q, k, v):
    return CausalGQAAttention.apply(q, k, v)
