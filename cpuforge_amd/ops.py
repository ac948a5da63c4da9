"""Device-tensor entry points of the layer ops (include/cfops.h).

Each function keeps the reference op's argument meaning and its overwrite /
accumulate (+=) contract, on contiguous float32 device tensors; torch is only
the holder of device memory and the current HIP stream:

    matmul_nn / matmul_nt / matmul_tn   crates/core/src/matmul.rs:127-147
    rmsnorm_forward / rmsnorm_backward  crates/core/src/ops/rmsnorm.rs
    silu_mul_forward / silu_mul_backward crates/core/src/ops/swiglu.rs
    cross_entropy_fwd_bwd               crates/core/src/ops/loss.rs:9-55
    lm_head_ce                          crates/model/src/model.rs:436-457
      (lm_head_ce_dev: the same, its loss left in device memory)
    linear_forward / linear_backward    crates/model/src/linear.rs:56-91
    adamw_update                        crates/train/src/optim.rs:9-30

Misuse the reference would panic on raises `ShapeError` (an AssertionError);
library failures raise `CfattnError`.
"""
from __future__ import annotations

import ctypes as C

import torch

from . import _lib
from .attention import Context, default_context

IGNORE_INDEX = _lib.IGNORE_INDEX


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _f32(t: torch.Tensor, name: str, numel: int | None = None) -> int:
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError(f"{name} must be a device tensor")
    if t.dtype != torch.float32:
        raise TypeError(f"{name} must be float32, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if numel is not None and t.numel() != numel:
        raise _lib.ShapeError(_lib.ERR_SHAPE,
                              f"assertion `left == right` failed: {name}.len() = {t.numel()}, expected {numel}")
    return t.data_ptr()


def _opt(t, name, numel=None):
    return None if t is None else _f32(t, name, numel)


def _targets(t: torch.Tensor, rows: int) -> int:
    if not isinstance(t, torch.Tensor) or not t.is_cuda or t.dtype != torch.int64 or not t.is_contiguous():
        raise TypeError("targets must be a contiguous int64 device tensor")
    if t.numel() != rows:
        raise _lib.ShapeError(_lib.ERR_SHAPE, f"assertion `left == right` failed: targets.len() = {t.numel()}, "
                                              f"expected {rows}")
    return t.data_ptr()


def _call(ctx: Context, name: str, *args) -> None:
    _lib.check(getattr(ctx._lib, name)(ctx.handle, *args), ctx.handle)


# --------------------------------------------------------------- matmul
def _matmul(kind, a, b, c, m, k, n, acc, ctx):
    ctx = ctx or default_context()
    ka, kb = (m * k, k * n) if kind == _lib.NN else (m * k, n * k) if kind == _lib.NT else (k * m, k * n)
    _call(ctx, "cfops_matmul", kind, _f32(a, "a", ka), _f32(b, "b", kb), _f32(c, "c", m * n), m, k, n, int(acc),
          _stream())
    return c


def matmul_nn(a, b, c, m, k, n, acc=False, ctx: Context | None = None):
    """C[m,n] (+)= A[m,k] . B[k,n]"""
    return _matmul(_lib.NN, a, b, c, m, k, n, acc, ctx)


def matmul_nt(a, b, c, m, k, n, acc=False, ctx: Context | None = None):
    """C[m,n] (+)= A[m,k] . B[n,k]^T"""
    return _matmul(_lib.NT, a, b, c, m, k, n, acc, ctx)


def matmul_tn(a, b, c, m, k, n, acc=False, ctx: Context | None = None):
    """C[m,n] (+)= A[k,m]^T . B[k,n]"""
    return _matmul(_lib.TN, a, b, c, m, k, n, acc, ctx)


# -------------------------------------------------------------- RMSNorm
def rmsnorm_forward(x, w, y, rstd, rows, dim, eps, ctx: Context | None = None):
    """rmsnorm.rs:4-28: overwrites y [rows, dim] and rstd [rows]."""
    ctx = ctx or default_context()
    _call(ctx, "cfops_rmsnorm_forward", _f32(x, "x", rows * dim), _f32(w, "w", dim), _f32(y, "y", rows * dim),
          _f32(rstd, "rstd", rows), rows, dim, float(eps), _stream())


def rmsnorm_backward(dy, x, w, rstd, dx, dw, rows, dim, ctx: Context | None = None):
    """rmsnorm.rs:33-67: accumulates into dx and dw (dw None: frozen gain)."""
    ctx = ctx or default_context()
    _call(ctx, "cfops_rmsnorm_backward", _f32(dy, "dy", rows * dim), _f32(x, "x", rows * dim), _f32(w, "w", dim),
          _f32(rstd, "rstd", rows), _f32(dx, "dx", rows * dim), _opt(dw, "dw", dim), rows, dim, _stream())


# --------------------------------------------------------------- SwiGLU
def silu_mul_forward(g, u, h, ctx: Context | None = None):
    """swiglu.rs:10-16: h = silu(g) * u (overwritten)."""
    ctx = ctx or default_context()
    n = g.numel()
    _call(ctx, "cfops_silu_mul_forward", _f32(g, "g"), _f32(u, "u", n), _f32(h, "h", n), n, _stream())


def silu_mul_backward(dh, g, u, dg, du, ctx: Context | None = None):
    """swiglu.rs:18-30: accumulates into dg and du."""
    ctx = ctx or default_context()
    n = g.numel()
    _call(ctx, "cfops_silu_mul_backward", _f32(dh, "dh", n), _f32(g, "g"), _f32(u, "u", n), _f32(dg, "dg", n),
          _f32(du, "du", n), n, _stream())


# -------------------------------------------------------- cross-entropy
def cross_entropy_fwd_bwd(logits, targets, dlogits, rows, vocab, ctx: Context | None = None) -> float:
    """loss.rs:9-55: returns the mean loss; dlogits overwritten (may be
    logits itself).  Waits for the stream, as the reference returns the
    loss.  A target out of range raises CfattnError (the reference panics)."""
    ctx = ctx or default_context()
    loss = C.c_float(0.0)
    _call(ctx, "cfops_cross_entropy_fwd_bwd", _f32(logits, "logits", rows * vocab), _targets(targets, rows),
          _f32(dlogits, "dlogits", rows * vocab), rows, vocab, C.byref(loss), _stream())
    return loss.value


def lm_head_ce(hn, head, targets, t, d, vocab, dhn, dhead=None, ctx: Context | None = None) -> float:
    """The LM head and loss of Model::forward_backward (model.rs:436-457):
    logits = hn . head^T, mean cross-entropy, dhn = dlogits . head
    (overwritten) and dhead += dlogits^T . hn when dhead is given.  Returns
    the loss; the [t, vocab] logits are formed a chunk of rows at a time."""
    ctx = ctx or default_context()
    loss = C.c_float(0.0)
    _call(ctx, "cfops_lm_head_ce", _f32(hn, "hn", t * d), _f32(head, "head", vocab * d), _targets(targets, t), t, d,
          vocab, _f32(dhn, "dhn", t * d), _opt(dhead, "dhead", vocab * d), C.byref(loss), _stream())
    return loss.value


CE_RESULT_WORDS = 3  # cfops_ce_result: n_valid, bad_row (int32), loss (float32)
_NO_BAD_ROW = 2 ** 31 - 1


def ce_result_buffer(device) -> torch.Tensor:
    """A device block for lm_head_ce_dev's result (cfops_ce_result)."""
    return torch.empty(CE_RESULT_WORDS, dtype=torch.int32, device=device)


def ce_result_loss(result: torch.Tensor) -> torch.Tensor:
    """The loss of a cfops_ce_result block, as a 0-d float32 device tensor
    (a view of the block)."""
    return result.view(torch.float32)[2]


def lm_head_ce_dev(hn, head, targets, t, d, vocab, dhn, dhead, result, ctx: Context | None = None) -> None:
    """lm_head_ce queued on the current stream with no host wait: the loss
    block goes to `result` (ce_result_buffer), for a step captured in a HIP
    graph.  The target check is the caller's, after the stream drains
    (ce_check)."""
    ctx = ctx or default_context()
    if not isinstance(result, torch.Tensor) or not result.is_cuda or result.dtype != torch.int32 \
            or result.numel() < CE_RESULT_WORDS or not result.is_contiguous():
        raise TypeError("result must be a contiguous int32 device tensor of 3 words")
    _call(ctx, "cfops_lm_head_ce_dev", _f32(hn, "hn", t * d), _f32(head, "head", vocab * d), _targets(targets, t), t,
          d, vocab, _f32(dhn, "dhn", t * d), _opt(dhead, "dhead", vocab * d), result.data_ptr(), _stream())


def ce_check(result: torch.Tensor, targets: torch.Tensor, vocab: int) -> None:
    """Waits for `result` (a cfops_ce_result written by lm_head_ce_dev) and
    raises, with lm_head_ce's error, for a target outside [0, vocab)."""
    bad = int(result[1].item())
    if bad != _NO_BAD_ROW:
        t = int(targets.reshape(-1)[bad].item())
        raise _lib.CfattnError(_lib.ERR_ARG, f"target {t} out of range for vocab {vocab}")


def set_head_chunk_limit(nbytes: int, ctx: Context | None = None) -> None:
    ctx = ctx or default_context()
    _call(ctx, "cfops_set_head_chunk_limit", int(nbytes))


# --------------------------------------------------------------- Linear
def linear_forward(x, w, t, inn, out, y, lora_a=None, lora_b=None, lora_scale=1.0, xs=None, ctx: Context | None = None):
    """Linear::forward (linear.rs:56-71): y = x W^T (+ xs B^T with xs =
    scale * x A^T when an adapter is given); y and xs overwritten."""
    ctx = ctx or default_context()
    r = 0 if lora_a is None else lora_a.shape[0]
    _call(ctx, "cfops_linear_forward", _f32(x, "x", t * inn), _f32(w, "w", out * inn), _opt(lora_a, "lora_a", r * inn),
          _opt(lora_b, "lora_b", out * r), float(lora_scale), t, inn, out, r, _f32(y, "y", t * out),
          _opt(xs, "xs", t * r), _stream())


def linear_backward(x, xs, dy, w, t, inn, out, dx, gw=None, ga=None, gb=None, lora_a=None, lora_b=None,
                    lora_scale=1.0, ctx: Context | None = None):
    """Linear::backward (linear.rs:73-91): accumulates into dx and every
    gradient given (None: frozen)."""
    ctx = ctx or default_context()
    r = 0 if lora_a is None else lora_a.shape[0]
    _call(ctx, "cfops_linear_backward", _f32(x, "x", t * inn), _opt(xs, "xs", t * r), _f32(dy, "dy", t * out),
          _f32(w, "w", out * inn), _opt(lora_a, "lora_a", r * inn), _opt(lora_b, "lora_b", out * r),
          float(lora_scale), t, inn, out, r, _f32(dx, "dx", t * inn), _opt(gw, "gw", out * inn),
          _opt(ga, "ga", r * inn), _opt(gb, "gb", out * r), _stream())


# ---------------------------------------------------------------- AdamW
def adamw_update(p, g, m, v, t, lr, beta1, beta2, eps, weight_decay, ctx: Context | None = None):
    """optim.rs:9-30: one AdamW step (t 1-based), in place on p, m, v."""
    ctx = ctx or default_context()
    n = p.numel()
    _call(ctx, "cfops_adamw_update", _f32(p, "p"), _f32(g, "g", n), _f32(m, "m", n), _f32(v, "v", n), n, int(t),
          float(lr), float(beta1), float(beta2), float(eps), float(weight_decay), _stream())
