"""The attention part of cpuforge's `Layer` on the GPU (crates/model/src/layer.rs).

`Layer::forward` (layer.rs:90-143) turns the q/k/v projections into the
attention output in three steps:
  - optional per-head RMSNorm of q and k (Qwen3, layer.rs:104-114);
  - RoPE at positions 0..t (layer.rs:115-116);
  - attention_forward (layer.rs:118-121).

`Layer::backward` (layer.rs:180-206) reverses them:
  - attention_backward;
  - inverse RoPE;
  - the q/k norm backward, including the norm gains' gradients.

`LayerAttention` runs both directions through libcfattn's fused entry points
(cfattn_fused_fwd / cfattn_fused_bwd) as one torch autograd function. Between
them it keeps the `LayerCache` contract (layer.rs:65-86): the post-prologue
q/k, v, q_pre/k_pre, q/k rstd, attn_o and lse.

Checkpoint mode (`MemoryMode::Checkpoint`, crates/model/src/model.rs:19-25,
486-491) does not keep that cache. The backward recomputes the forward from
q_pre/k_pre/v first. The kernels use no atomics, so the recomputed O and lse
equal the first ones bit for bit.
"""
from __future__ import annotations

import torch

from . import device as D
from .rope import RopeCache


class LayerRope:
    """The model's RoPE table and q/k norm gains, resident on the device
    (model/src/model.rs:240 builds one RopeCache for max_seq positions)."""

    def __init__(self, rope: RopeCache, device="cuda", q_norm=None, k_norm=None, eps: float = 1e-6):
        self.pr = D.DeviceRope(rope, device, 0, q_norm, k_norm, eps)


class LayerAttention(torch.autograd.Function):
    """o = attention(rope(norm(q_pre)), rope(norm(k_pre)), v), causal GQA.

    - Inputs: q_pre `[B,S,Hq,D]` and k_pre `[B,S,Hkv,D]` float32; v
      `[B,S,Hkv,D]` float32 or bfloat16. v's dtype selects the attention mode.
    - Output: o, float32, `[B,S,Hq,D]`.
    - Gradients flow to q_pre, k_pre, v and the norm gains.
    """

    @staticmethod
    def forward(ctx, q_pre, k_pre, v, lr: LayerRope, checkpoint: bool, q_norm=None, k_norm=None):
        q_pre, k_pre, v = q_pre.contiguous(), k_pre.contiguous(), v.contiguous()
        o, lse, q, k, q_rstd, k_rstd = D.fused_fwd(q_pre, k_pre, v, lr.pr)
        ctx.lr = lr
        ctx.checkpoint = checkpoint
        ctx.has_norm = lr.pr.q_norm is not None
        if checkpoint:
            ctx.save_for_backward(q_pre, k_pre, v)
        else:
            saved = [q_pre, k_pre, v, q, k, o, lse]
            if ctx.has_norm:
                saved += [q_rstd, k_rstd]
            ctx.save_for_backward(*saved)
        return o

    @staticmethod
    def backward(ctx, g):
        if ctx.checkpoint:
            q_pre, k_pre, v = ctx.saved_tensors
            o, lse, q, k, q_rstd, k_rstd = D.fused_fwd(q_pre, k_pre, v, ctx.lr.pr)
        else:
            saved = ctx.saved_tensors
            q_pre, k_pre, v, q, k, o, lse = saved[:7]
            q_rstd, k_rstd = saved[7:] if ctx.has_norm else (None, None)
        d_o = g.contiguous().to(v.dtype)
        dq_pre, dk_pre, dv, dqn, dkn = D.fused_bwd(d_o, q_pre, k_pre, q, k, v, o, lse, q_rstd, k_rstd, ctx.lr.pr)
        return dq_pre, dk_pre, dv.to(v.dtype), None, None, dqn, dkn


def layer_attention(q_pre, k_pre, v, lr: LayerRope, checkpoint: bool = False):
    """Layer::forward's q_pre/k_pre/v -> attn_o, differentiable.  The norm
    gains of `lr` (if any) receive gradients through `LayerAttention`."""
    return LayerAttention.apply(q_pre, k_pre, v, lr, checkpoint, lr.pr.q_norm, lr.pr.k_norm)
