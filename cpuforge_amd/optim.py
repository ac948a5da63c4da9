"""AdamW over a model's device-resident parameters (crates/train/src/optim.rs).

`AdamW` keeps the reference struct's fields (beta1, beta2, eps,
weight_decay, `step` = optimizer steps taken, `state` = first and second
moments keyed by parameter name, optim.rs:32-41).  Its `update` is the
reference's `AdamW::step` (optim.rs:48-61): the count goes up by one, and every
parameter that has a gradient gets `adamw_update` (cfops_adamw_update, bitwise
the reference's f32 arithmetic) with no weight decay for the norm gains.  (The
method is not called `step` because Python cannot hold a field and a method of
one name.)

A model here is any object whose `named_params()` yields (name, tensor) in
`visit_params` order (crates/model/src/model.rs:179-208); a parameter has a
gradient when it requires one, as a non-empty `Grads` entry does in the
reference (TrainSpec decides both).
"""
from __future__ import annotations

import torch

from . import ops as P


class AdamW:
    def __init__(self, beta1: float, beta2: float, eps: float, weight_decay: float):
        self.beta1, self.beta2, self.eps, self.weight_decay = beta1, beta2, eps, weight_decay
        self.step = 0
        self.state: dict = {}

    @torch.no_grad()
    def update(self, model, lr: float) -> None:
        self.step += 1
        for name, p in model.named_params():
            if not p.requires_grad:
                continue
            g = p.grad if p.grad is not None else torch.zeros_like(p)
            if name not in self.state:
                self.state[name] = (torch.zeros_like(p), torch.zeros_like(p))
            m, v = self.state[name]
            decay = 0.0 if "norm" in name else self.weight_decay
            P.adamw_update(p, g.contiguous(), m, v, self.step, lr, self.beta1, self.beta2, self.eps, decay)
