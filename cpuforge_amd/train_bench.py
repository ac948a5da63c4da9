"""SmolLM-135M-shaped LoRA training step with cpuforge's attention on the GPU.

This is the measurement behind "SmolLM-135M train tok/s", the second half of
the tier's metric. It follows the reference's `cpuforge bench-train`
(crates/cli/src/cmd_bench.rs:43-99):

- **Model.** A random-init SmolLM-135M shape (`smollm_135m_config`,
  cmd_bench.rs:43-50):
  - 30 layers, hidden 576, FFN 1536, 9 query / 3 KV heads of 64, vocab 49152;
  - tied embeddings, RMSNorm eps 1e-5, RoPE theta 1e4.
- **Init** (`Model::random`, crates/model/src/model.rs:282-305): weights
  N(0, 0.02), norm gains 1.
- **LoRA** (`Linear::add_lora`, crates/model/src/linear.rs:44-53):
  - rank 16, alpha 32, on q, k, v, o, gate, up, down;
  - A uniform in ±1/sqrt(in), B zero;
  - only the adapters train (`TrainSpec::LORA_ONLY`).
- **Timed step.** `grads.zero()` plus one `forward_backward` (cmd_bench.rs:78-87):
  embeddings → 30 × Layer → final norm → tied LM head → mean cross-entropy,
  then the backward. There is no optimizer step, as in the reference.
- **Batch.** The reference runs one sequence per call; this harness runs
  `batch` sequences in one device pass. tok/s = batch·seq / step time.

The attention of every layer is `cpuforge_amd.layer.layer_attention`, the
fused RoPE + attention kernels.  With `backend="cfops"` (the default) every
other op of the step also runs through libcfattn.so (include/cfops.h, via
`cpuforge_amd.autograd`): RMSNorm, the LoRA linears (hipBLASLt GEMMs), the
SwiGLU gate and the LM head with its cross-entropy, whose [t, vocab] logits
are formed a chunk of rows at a time.  Only the embedding gather and the
residual adds stay torch ops.  `backend="torch"` runs those ops as plain torch
ops instead, for comparison.
"""
from __future__ import annotations

import time
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import autograd as A
from .layer import LayerRope, layer_attention
from .rope import RopeCache
from .st import FormatError

SMOLLM_135M = dict(vocab=49152, d=576, ffn=1536, heads=9, kv_heads=3, head_dim=64, eps=1e-5, theta=1e4)


class LoRALinear:
    """y = x Wᵀ (+ (alpha/r) (x Aᵀ) Bᵀ with an adapter) (linear.rs:1-3, 56-69)."""

    def __init__(self, out: int, inn: int, std: float, gen, dtype, device):
        self.w = (torch.randn(out, inn, generator=gen, device=device) * std).to(dtype)
        self.a = self.b = None
        self.scale = 1.0

    def add_lora(self, rank: int, alpha: float, gen) -> None:
        """Linear::add_lora (linear.rs:44-52): A uniform in ±1/sqrt(in), B zero,
        scale alpha / rank."""
        out, inn = self.w.shape
        bound = 1.0 / inn ** 0.5
        dev, dt = self.w.device, self.w.dtype
        self.a = ((torch.rand(rank, inn, generator=gen, device=dev) * 2 - 1) * bound).to(dt).requires_grad_()
        self.b = torch.zeros(out, rank, device=dev, dtype=dt, requires_grad=True)
        self.scale = alpha / rank

    def __call__(self, x, backend="torch"):
        if backend == "cfops":
            return A.linear(x, self.w, self.a, self.b, self.scale)
        y = x @ self.w.t()
        if self.a is None:
            return y
        return y + (self.scale * (x @ self.a.t())) @ self.b.t()

    def spec(self):
        """(w, a, b, scale) for the shared-input linears."""
        return self.w, self.a, self.b, self.scale

    def named(self, prefix: str):
        """visit_linear (crates/model/src/model.rs:164-173)."""
        yield f"{prefix}.weight", self.w
        if self.a is not None:
            yield f"{prefix}.lora_A", self.a
            yield f"{prefix}.lora_B", self.b

    def params(self):
        return [self.a, self.b] if self.a is not None else []


def rmsnorm(x, w, eps):
    return x * torch.rsqrt((x * x).mean(-1, keepdim=True) + eps) * w


@dataclass
class LoraConfig:
    """crates/model/src/model.rs:45-49."""
    rank: int
    alpha: float
    targets: list


LORA_TARGETS = ("q", "k", "v", "o", "gate", "up", "down")
_LINEARS = (("q", "wq"), ("k", "wk"), ("v", "wv"), ("o", "wo"), ("gate", "gate"), ("up", "up"), ("down", "down"))


class SmolLM:
    """`rank` > 0 attaches adapters (alpha 2·rank) to every projection, as
    `cpuforge bench-train` does; `train` is the TrainSpec: "lora" trains the
    adapters only (LORA_ONLY), "full" every parameter (FULL).  `config`
    overrides entries of SMOLLM_135M (a smaller model for tests)."""

    def __init__(self, layers: int = 30, seq: int = 512, rank: int = 16, dtype=torch.float32, device="cuda",
                 seed: int = 1, attn_dtype=None, backend: str = "cfops", config: dict | None = None,
                 train: str = "lora"):
        if backend not in ("cfops", "torch"):
            raise ValueError(f"unknown backend {backend!r}")
        if backend == "cfops" and dtype != torch.float32:
            raise ValueError("the cfops backend runs the reference's f32 arithmetic")
        if train not in ("lora", "full"):
            raise ValueError(f"unknown train spec {train!r}")
        c = dict(SMOLLM_135M, **(config or {}))
        self.c, self.dtype, self.layers_n, self.backend, self.train = c, dtype, layers, backend, train
        self.attn_dtype = attn_dtype or dtype
        self.device = device
        gen = torch.Generator(device=device)
        gen.manual_seed(seed)
        d, f, hd = c["d"], c["ffn"], c["head_dim"]
        qd, kvd = c["heads"] * hd, c["kv_heads"] * hd
        lin = lambda o, i: LoRALinear(o, i, 0.02, gen, dtype, device)  # noqa: E731
        self.layers = [dict(attn_norm=torch.ones(d, device=device, dtype=dtype), wq=lin(qd, d), wk=lin(kvd, d),
                            wv=lin(kvd, d), wo=lin(d, qd), mlp_norm=torch.ones(d, device=device, dtype=dtype),
                            gate=lin(f, d), up=lin(f, d), down=lin(d, f)) for _ in range(layers)]
        self.embed = (torch.randn(c["vocab"], d, generator=gen, device=device) * 0.02).to(dtype)
        self.final_norm = torch.ones(d, device=device, dtype=dtype)
        self.rope = LayerRope(RopeCache(hd, seq, c["theta"]), device)
        self.attention = layer_attention  # (q_pre, k_pre, v, LayerRope) -> o
        # With ce_on_device the cfops loss leaves its value on the device
        # (no host wait: a step that can be captured in a HIP graph) and the
        # target check waits for check_targets().
        self.ce_on_device = False
        self._ce = None
        self.lora_cfg = None
        if train == "full":
            for _, p in self.named_params():
                p.requires_grad_()
        if rank:
            self.add_lora(rank, 2.0 * rank, list(LORA_TARGETS), seed)

    def add_lora(self, rank: int, alpha: float, targets, seed: int) -> None:
        """Model::add_lora (crates/model/src/model.rs:309-335): adapters on the
        named projections of every layer, initialised from `seed`."""
        for t in targets:
            if t not in LORA_TARGETS:
                raise FormatError(f"unknown LoRA target '{t}'")
        if self.lora_cfg is not None:
            raise FormatError("model already has LoRA adapters")
        gen = torch.Generator(device=self.device)
        gen.manual_seed(seed)
        for layer in self.layers:
            for short, attr in _LINEARS:
                if short in targets:
                    layer[attr].add_lora(rank, alpha, gen)
        self.lora_cfg = LoraConfig(rank, alpha, [str(t) for t in targets])

    def named_params(self):
        """visit_params order and names (crates/model/src/model.rs:179-208)."""
        yield "model.embed_tokens.weight", self.embed
        for i, layer in enumerate(self.layers):
            p = f"model.layers.{i}"
            yield f"{p}.input_layernorm.weight", layer["attn_norm"]
            yield from layer["wq"].named(f"{p}.self_attn.q_proj")
            yield from layer["wk"].named(f"{p}.self_attn.k_proj")
            yield from layer["wv"].named(f"{p}.self_attn.v_proj")
            yield from layer["wo"].named(f"{p}.self_attn.o_proj")
            yield f"{p}.post_attention_layernorm.weight", layer["mlp_norm"]
            yield from layer["gate"].named(f"{p}.mlp.gate_proj")
            yield from layer["up"].named(f"{p}.mlp.up_proj")
            yield from layer["down"].named(f"{p}.mlp.down_proj")
        yield "model.norm.weight", self.final_norm

    def params(self):
        """The parameters that train (TrainSpec)."""
        return [p for _, p in self.named_params() if p.requires_grad]

    def loss(self, tokens, targets):
        if self.backend == "cfops":
            return self._loss_cfops(tokens, targets)
        c = self.c
        B, S = tokens.shape
        x = self.embed[tokens]
        for layer in self.layers:
            n1 = rmsnorm(x, layer["attn_norm"], c["eps"])
            q = layer["wq"](n1).view(B, S, c["heads"], c["head_dim"])
            k = layer["wk"](n1).view(B, S, c["kv_heads"], c["head_dim"])
            v = layer["wv"](n1).view(B, S, c["kv_heads"], c["head_dim"])
            o = self.attention(q.float(), k.float(), v.to(self.attn_dtype), self.rope)
            x = x + layer["wo"](o.view(B, S, -1).to(self.dtype))
            n2 = rmsnorm(x, layer["mlp_norm"], c["eps"])
            x = x + layer["down"](F.silu(layer["gate"](n2)) * layer["up"](n2))
        hn = rmsnorm(x, self.final_norm, c["eps"])
        logits = hn @ self.embed.t()
        return F.cross_entropy(logits.view(-1, c["vocab"]).float(), targets.view(-1))

    def _loss_cfops(self, tokens, targets):
        """Layer::forward (crates/model/src/layer.rs:90-143) per layer, then the
        final norm and the tied LM head with its loss (model.rs:436-442), every
        op but the gather and the residual adds in libcfattn.so."""
        c, cf = self.c, "cfops"
        B, S = tokens.shape
        x = self.embed[tokens]
        for layer in self.layers:
            n1 = A.rmsnorm(x, layer["attn_norm"], c["eps"])
            q, k, v = A.shared_input_linears(n1, [layer[n].spec() for n in ("wq", "wk", "wv")])
            q = q.view(B, S, c["heads"], c["head_dim"])
            k = k.view(B, S, c["kv_heads"], c["head_dim"])
            v = v.view(B, S, c["kv_heads"], c["head_dim"])
            o = self.attention(q, k, v.to(self.attn_dtype), self.rope)
            x = x + layer["wo"](o.view(B, S, -1), cf)
            n2 = A.rmsnorm(x, layer["mlp_norm"], c["eps"])
            g, u = A.shared_input_linears(n2, [layer[n].spec() for n in ("gate", "up")])
            x = x + layer["down"](A.silu_mul(g, u), cf)
        hn = A.rmsnorm(x, self.final_norm, c["eps"])
        if self.ce_on_device:
            loss, res = A.lm_head_ce_dev(hn, self.embed, targets)
            self._ce = (res, targets)
            return loss
        return A.lm_head_ce(hn, self.embed, targets)

    def check_targets(self) -> None:
        """Raises, as the loss would have, if the last device-side loss met
        a target out of range (waits for it)."""
        if self._ce is not None:
            from .ops import ce_check
            res, targets = self._ce
            ce_check(res, targets, self.c["vocab"])


def capture_step(model: SmolLM, tokens, targets, warmup: int = 2):
    """The training step (every trained parameter's .grad reset, forward,
    loss, backward) captured in a HIP graph: `warmup` eager steps on a side
    stream (the capture recipe: the library's scratch, the GEMM plans and
    torch's allocations are made there), then the capture.  Returns the graph
    and the loss tensor its replays write; each replay leaves the step's
    gradients in the parameters' .grad.  Needs the cfops backend with
    model.ce_on_device, so that no op waits for the host."""
    if model.backend != "cfops" or not model.ce_on_device:
        raise ValueError("graph capture needs the cfops backend with ce_on_device")
    params = model.params()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(warmup):
            for p_ in params:
                p_.grad = None
            loss = model.loss(tokens, targets)
            loss.backward()
            del loss
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    model.check_targets()
    for p_ in params:
        p_.grad = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_loss = model.loss(tokens, targets)
        static_loss.backward()
    return graph, static_loss


def train_tok_s(batch: int = 8, seq: int = 512, layers: int = 30, rank: int = 16, steps: int = 3,
                dtype=torch.float32, attn_dtype=None, device="cuda", backend: str = "cfops",
                warmup: int = 3, graph: bool = False) -> dict:
    """Build the model, run `warmup` untimed steps (the first allocates the
    library's scratch and plans; the clock settles over the next ones),
    then time `steps` forward+backward passes; returns tok/s and the step
    time.  With `graph` (cfops backend) the step is captured in a HIP graph
    after the warm-up steps and the timed steps are its replays: the same
    kernels in the same order, without the host's launch work between
    them."""
    model = SmolLM(layers, seq, rank, dtype, device, attn_dtype=attn_dtype, backend=backend)
    gen = torch.Generator(device=device)
    gen.manual_seed(7)
    tokens = torch.randint(0, model.c["vocab"], (batch, seq), generator=gen, device=device)
    targets = torch.randint(0, model.c["vocab"], (batch, seq), generator=gen, device=device)
    params = model.params()

    def step():
        for p_ in params:
            p_.grad = None
        loss = model.loss(tokens, targets)
        loss.backward()
        return loss

    loss0 = step().item()
    out = {}
    if graph:
        model.ce_on_device = True
        g, static_loss = capture_step(model, tokens, targets, max(warmup - 1, 1))
        g.replay()
        torch.cuda.synchronize()
        model.check_targets()
        out["graph_first_loss"] = static_loss.item()
        run = g.replay
    else:
        for _ in range(warmup - 1):
            step()
        run = step
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        run()
    torch.cuda.synchronize()
    per = (time.perf_counter() - t0) / steps
    if graph:
        model.check_targets()
    return {"value": batch * seq / per, "unit": "tok/s", "ms_per_step": per * 1e3, "batch": batch, "seq": seq,
            "layers": layers, "lora_rank": rank, "dtype": str(dtype).replace("torch.", ""),
            "attn_dtype": str(attn_dtype or dtype).replace("torch.", ""), "steps": steps, "warmup": warmup,
            "first_loss": loss0, "backend": backend, "graph": graph, **out}
