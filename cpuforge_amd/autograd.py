"""torch autograd functions over the layer ops of include/cfops.h, so a host
model can run cpuforge's Layer and LM head on the GPU with every hot op in
libcfattn.so.  Each backward keeps the reference's gradient contract (the
`Linear::backward` / `rmsnorm_backward` / `silu_mul_backward` formulas,
accumulating into fresh zero buffers); frozen tensors (requires_grad False)
get no gradient work, as an empty LinGrad vector does in the reference
(crates/model/src/linear.rs:22-27)."""
from __future__ import annotations

import torch

from . import ops as P


def _flat(x: torch.Tensor, cols: int) -> torch.Tensor:
    return x.contiguous().view(-1, cols)


def _zeros(*likes):
    """Zero-filled buffers shaped like `likes` (None entries stay None), cut
    from one allocation so they cost one fill launch."""
    sizes = [t.numel() if t is not None else 0 for t in likes]
    flat = torch.zeros(sum(sizes), device=next(t for t in likes if t is not None).device, dtype=torch.float32)
    out, off = [], 0
    for t, n in zip(likes, sizes):
        out.append(None if t is None else flat[off:off + n].view(t.shape))
        off += n
    return out


class RMSNormFn(torch.autograd.Function):
    """y = rmsnorm(x, w) over the last dim (crates/core/src/ops/rmsnorm.rs)."""

    @staticmethod
    def forward(ctx, x, w, eps: float):
        dim = x.shape[-1]
        x2 = _flat(x, dim)
        rows = x2.shape[0]
        y = torch.empty_like(x2)
        rstd = torch.empty(rows, device=x.device, dtype=torch.float32)
        P.rmsnorm_forward(x2, w, y, rstd, rows, dim, eps)
        ctx.save_for_backward(x2, w, rstd)
        return y.view(x.shape)

    @staticmethod
    def backward(ctx, dy):
        x2, w, rstd = ctx.saved_tensors
        rows, dim = x2.shape
        dx, dw = _zeros(x2, w if ctx.needs_input_grad[1] else None)
        P.rmsnorm_backward(_flat(dy, dim), x2, w, rstd, dx, dw, rows, dim)
        return dx.view(dy.shape), dw, None


class SiluMulFn(torch.autograd.Function):
    """h = silu(g) * u (crates/core/src/ops/swiglu.rs)."""

    @staticmethod
    def forward(ctx, g, u):
        g, u = g.contiguous(), u.contiguous()
        h = torch.empty_like(g)
        P.silu_mul_forward(g, u, h)
        ctx.save_for_backward(g, u)
        return h

    @staticmethod
    def backward(ctx, dh):
        g, u = ctx.saved_tensors
        dg, du = _zeros(g, u)
        P.silu_mul_backward(dh.contiguous(), g, u, dg, du)
        return dg, du


class LinearFn(torch.autograd.Function):
    """y = x W^T (+ scale (x A^T) B^T) (crates/model/src/linear.rs:56-91)."""

    @staticmethod
    def forward(ctx, x, w, a, b, scale: float):
        inn, out = w.shape[1], w.shape[0]
        x2 = _flat(x, inn)
        t = x2.shape[0]
        y = torch.empty(t, out, device=x.device, dtype=torch.float32)
        xs = torch.empty(t, a.shape[0], device=x.device, dtype=torch.float32) if a is not None else None
        P.linear_forward(x2, w, t, inn, out, y, a, b, scale, xs)
        ctx.save_for_backward(x2, xs, w, a, b)
        ctx.scale = scale
        return y.view(*x.shape[:-1], out)

    @staticmethod
    def backward(ctx, dy):
        x2, xs, w, a, b = ctx.saved_tensors
        t, inn = x2.shape
        out = w.shape[0]
        need = ctx.needs_input_grad
        dx, gw, ga, gb = _zeros(x2, w if need[1] else None, a if a is not None and need[2] else None,
                                b if b is not None and need[3] else None)
        P.linear_backward(x2, xs, _flat(dy, out), w, t, inn, out, dx, gw, ga, gb, a, b, ctx.scale)
        return dx.view(*dy.shape[:-1], inn), gw, ga, gb, None


class SharedInputLinearsFn(torch.autograd.Function):
    """Several linears of one input (the q/k/v projections of a layer, or its
    gate and up projections): each forward as LinearFn, and one backward that
    accumulates every linear's dx into one zeroed buffer in order, as the
    reference's Layer::backward does for dn2 (crates/model/src/layer.rs:170-171)
    and dn1 (layer.rs:208-211).  `flat` holds (w, a, b) per linear."""

    @staticmethod
    def forward(ctx, x, scales, *flat):
        inn = flat[0].shape[1]
        x2 = _flat(x, inn)
        t = x2.shape[0]
        ys, xss = [], []
        for i, scale in enumerate(scales):
            w, a, b = flat[3 * i:3 * i + 3]
            y = torch.empty(t, w.shape[0], device=x.device, dtype=torch.float32)
            xs = torch.empty(t, a.shape[0], device=x.device, dtype=torch.float32) if a is not None else None
            P.linear_forward(x2, w, t, inn, w.shape[0], y, a, b, scale, xs)
            ys.append(y.view(*x.shape[:-1], w.shape[0]))
            xss.append(xs)
        ctx.save_for_backward(x2, *flat, *[xs if xs is not None else torch.empty(0) for xs in xss])
        ctx.scales = scales
        ctx.has_xs = [xs is not None for xs in xss]
        ctx.shape = x.shape
        return tuple(ys)

    @staticmethod
    def backward(ctx, *dys):
        saved = ctx.saved_tensors
        n = len(ctx.scales)
        x2, flat, xss = saved[0], saved[1:1 + 3 * n], saved[1 + 3 * n:]
        t, inn = x2.shape
        need = ctx.needs_input_grad[2:]
        likes = [x2]
        for i in range(3 * n):
            likes.append(flat[i] if flat[i] is not None and need[i] else None)
        bufs = _zeros(*likes)
        dx, grads = bufs[0], bufs[1:]
        for i, scale in enumerate(ctx.scales):
            w, a, b = flat[3 * i:3 * i + 3]
            if dys[i] is None:
                continue
            gw, ga, gb = grads[3 * i:3 * i + 3]
            xs = xss[i] if ctx.has_xs[i] else None
            P.linear_backward(x2, xs, _flat(dys[i], w.shape[0]), w, t, inn, w.shape[0], dx, gw, ga, gb, a, b,
                              scale)
        return (dx.view(ctx.shape), None, *grads)


class LMHeadCEFn(torch.autograd.Function):
    """Mean cross-entropy of logits = hn head^T (model.rs:436-457); the
    forward already forms dhn (and dhead), as cross_entropy_fwd_bwd does."""

    @staticmethod
    def forward(ctx, hn, head, targets):
        d = hn.shape[-1]
        h2 = _flat(hn, d)
        t, vocab = h2.shape[0], head.shape[0]
        dhn = torch.empty_like(h2)
        dhead = torch.zeros_like(head) if ctx.needs_input_grad[1] else None
        loss = P.lm_head_ce(h2, head, targets.contiguous().view(-1), t, d, vocab, dhn, dhead)
        ctx.save_for_backward(dhn, dhead if dhead is not None else torch.empty(0))
        ctx.has_dhead = dhead is not None
        ctx.shape = hn.shape
        return torch.tensor(loss, device=hn.device)

    @staticmethod
    def backward(ctx, g):
        dhn, dhead = ctx.saved_tensors
        return (dhn * g).view(ctx.shape), (dhead * g if ctx.has_dhead else None), None


class LMHeadCEDevFn(torch.autograd.Function):
    """LMHeadCEFn with no host wait (ops.lm_head_ce_dev), for a step captured
    in a HIP graph: returns the loss as a device tensor and the loss block
    (cfops_ce_result), whose target check the caller runs after the stream
    drains (ops.ce_check)."""

    @staticmethod
    def forward(ctx, hn, head, targets):
        d = hn.shape[-1]
        h2 = _flat(hn, d)
        t, vocab = h2.shape[0], head.shape[0]
        dhn = torch.empty_like(h2)
        dhead = torch.zeros_like(head) if ctx.needs_input_grad[1] else None
        result = P.ce_result_buffer(hn.device)
        P.lm_head_ce_dev(h2, head, targets.contiguous().view(-1), t, d, vocab, dhn, dhead, result)
        ctx.save_for_backward(dhn, dhead if dhead is not None else torch.empty(0))
        ctx.has_dhead = dhead is not None
        ctx.shape = hn.shape
        ctx.mark_non_differentiable(result)
        return P.ce_result_loss(result).clone(), result

    @staticmethod
    def backward(ctx, g, _g_result):
        dhn, dhead = ctx.saved_tensors
        return (dhn * g).view(ctx.shape), (dhead * g if ctx.has_dhead else None), None


def rmsnorm(x, w, eps):
    return RMSNormFn.apply(x, w, eps)


def silu_mul(g, u):
    return SiluMulFn.apply(g, u)


def linear(x, w, a=None, b=None, scale=1.0):
    return LinearFn.apply(x, w, a, b, scale)


def shared_input_linears(x, specs):
    """[(w, a, b, scale), ...] -> the linears' outputs for input x, with one
    accumulated dx in the backward."""
    flat = [t for w, a, b, _ in specs for t in (w, a, b)]
    return SharedInputLinearsFn.apply(x, tuple(float(s) for *_, s in specs), *flat)


def lm_head_ce(hn, head, targets):
    return LMHeadCEFn.apply(hn, head, targets)


def lm_head_ce_dev(hn, head, targets):
    """(loss, cfops_ce_result block): the loss with no host wait."""
    return LMHeadCEDevFn.apply(hn, head, targets)
