"""cpuforge_amd: MI355X (gfx950) causal grouped-query attention for cpuforge.

The reference-shaped API (crates/core/src/ops/attention.rs, ops/rope.rs):

    from cpuforge_amd import AttnShape, attention_forward, attention_backward
    attention_forward(q, k, v, o, lse, AttnShape(seq, n_heads, n_kv, head_dim))

runs the hand-written HIP kernels in libcfattn.so.  `cpuforge_amd.device`
holds the batched device-tensor entry points and the fused RoPE / q-k-norm
prologue.  Build the library with `python -m cpuforge_amd.build`.
"""
from ._lib import CfattnError, ShapeError  # noqa: F401
from .attention import (  # noqa: F401
    DEFAULT_Q_BLOCK,
    AttnShape,
    Context,
    attention_backward,
    attention_backward_blocked,
    attention_forward,
    attention_forward_blocked,
    default_context,
    flops_fwd_bwd,
    set_mode,
)
from .rope import Llama3Scaling, RopeCache  # noqa: F401

__version__ = "0.1.0"
