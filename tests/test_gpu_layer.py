"""GPU tests of the Layer attention contract (cpuforge_amd.layer, restating
crates/model/src/layer.rs:90-218) and of the SmolLM-135M train harness
(cpuforge_amd.train_bench, restating crates/cli/src/cmd_bench.rs:52-99).

The references are independent float64 CPU implementations written here
with torch autograd:
  - RMSNorm, rotate-half RoPE and causal GQA attention by explicit matmul and
    softmax;
  - the whole SmolLM forward on top of them.
The checkpoint-mode test restates crates/model/src/tests.rs:147-163: the
recomputed forward gives the identical result.

Tolerances (fp32 mode): attention outputs and gradients max abs 1e-4
against the float64 reference; the model loss relative 1e-5; the LoRA
gradients use the reference's gradcheck metric |a-r|/(1+|r|) <= 1e-4.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _ref_prologue(x, w, cos, sin, eps):
    """[B,S,H,D] float64: optional RMSNorm per (token, head), then RoPE."""
    import torch
    if w is not None:
        x = x * torch.rsqrt((x * x).mean(-1, keepdim=True) + eps) * w
    half = x.shape[-1] // 2
    c, s = cos[None, :, None, :], sin[None, :, None, :]
    x1, x2 = x[..., :half], x[..., half:]
    return torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], -1)


def _ref_attention(q, k, v):
    """Causal GQA, [B,S,Hq,D] x [B,S,Hkv,D], float64."""
    import torch
    B, S, Hq, D = q.shape
    grp = Hq // k.shape[2]
    k = k.repeat_interleave(grp, dim=2)
    v = v.repeat_interleave(grp, dim=2)
    s = torch.einsum("bthd,bshd->bhts", q, k) / D ** 0.5
    mask = torch.ones(S, S, dtype=torch.bool).triu(1)
    s = s.masked_fill(mask, float("-inf"))
    return torch.einsum("bhts,bshd->bthd", torch.softmax(s, -1), v)


@pytest.mark.parametrize("qk_norm", [False, True])
def test_layer_attention_matches_float64_autograd(qk_norm):
    import torch

    from cpuforge_amd import RopeCache
    from cpuforge_amd.layer import LayerRope, layer_attention
    B, S, Hq, Hk, D, eps = 2, 45, 4, 2, 64, 1e-6
    torch.manual_seed(3)
    qp, kp, vv, g = (torch.randn(B, S, h, D) for h in (Hq, Hk, Hk, Hq))
    rope = RopeCache(D, S, 1e4)
    qw = kw = None
    if qk_norm:
        qw, kw = 1 + 0.02 * torch.randn(D), 1 + 0.02 * torch.randn(D)
    lr = LayerRope(rope, "cuda", qw.cuda().requires_grad_() if qk_norm else None,
                   kw.cuda().requires_grad_() if qk_norm else None, eps)
    dq, dk, dv = (x.cuda().requires_grad_() for x in (qp, kp, vv))
    o = layer_attention(dq, dk, dv, lr)
    (o * g.cuda()).sum().backward()
    torch.cuda.synchronize()

    cos = torch.tensor(rope.cos, dtype=torch.float64)
    sin = torch.tensor(rope.sin, dtype=torch.float64)
    rq, rk, rv = (x.double().requires_grad_() for x in (qp, kp, vv))
    rqw = qw.double().requires_grad_() if qk_norm else None
    rkw = kw.double().requires_grad_() if qk_norm else None
    ro = _ref_attention(_ref_prologue(rq, rqw, cos, sin, eps), _ref_prologue(rk, rkw, cos, sin, eps), rv)
    (ro * g.double()).sum().backward()
    pairs = [("o", o, ro), ("dq_pre", dq.grad, rq.grad), ("dk_pre", dk.grad, rk.grad), ("dv", dv.grad, rv.grad)]
    if qk_norm:
        pairs += [("dq_norm", lr.pr.q_norm.grad, rqw.grad), ("dk_norm", lr.pr.k_norm.grad, rkw.grad)]
    for name, a, r in pairs:
        a = a.detach().cpu().double().numpy()
        r = r.detach().numpy()
        tol = 1e-4 * (1 + np.abs(r).max()) if name.endswith("norm") else 1e-4
        e = np.abs(a - r).max()
        print(f"{name}: {e:.3e}", flush=True)
        assert e <= tol, f"{name}: {e}"


def test_checkpoint_mode_recompute_is_bitwise_identical():
    """MemoryMode::Checkpoint recomputes the forward before the backward
    (model/src/model.rs:486-491); gradients must equal Full mode's exactly."""
    import torch

    from cpuforge_amd import RopeCache
    from cpuforge_amd.layer import LayerRope, layer_attention
    torch.manual_seed(4)
    B, S, Hq, Hk, D = 2, 200, 8, 2, 128
    lr = LayerRope(RopeCache(D, S, 5e5), "cuda")
    base = [torch.randn(B, S, h, D, device="cuda") for h in (Hq, Hk)]
    v0 = torch.randn(B, S, Hk, D, device="cuda").bfloat16()
    g = torch.randn(B, S, Hq, D, device="cuda")
    res = []
    for ckpt in (False, True):
        qp, kp = (x.clone().requires_grad_() for x in base)
        v = v0.clone().requires_grad_()
        o = layer_attention(qp, kp, v, lr, checkpoint=ckpt)
        (o * g).sum().backward()
        torch.cuda.synchronize()
        res.append([x.detach().float().cpu().numpy() for x in (o, qp.grad, kp.grad, v.grad)])
    for a, b in zip(*res):
        assert np.array_equal(a, b)


def _reference_loss(model, tokens, targets):
    """The SmolLM forward in float64 on the CPU with the reference attention,
    from the same weights (LoRA parameters as leaves)."""
    import torch
    import torch.nn.functional as F
    c = model.c
    cos = torch.tensor(model.rope.pr.rope.cos, dtype=torch.float64)
    sin = torch.tensor(model.rope.pr.rope.sin, dtype=torch.float64)
    d64 = lambda t: t.detach().cpu().double()  # noqa: E731
    leaves = []

    def lin(m, x):
        a, b = d64(m.a).requires_grad_(), d64(m.b).requires_grad_()
        leaves.extend([a, b])
        return x @ d64(m.w).t() + (m.scale * (x @ a.t())) @ b.t()

    def rms(x, w):
        return x * torch.rsqrt((x * x).mean(-1, keepdim=True) + c["eps"]) * d64(w)

    B, S = tokens.shape
    emb = d64(model.embed)
    x = emb[tokens.cpu()]
    for layer in model.layers:
        n1 = rms(x, layer["attn_norm"])
        q = lin(layer["wq"], n1).view(B, S, c["heads"], c["head_dim"])
        k = lin(layer["wk"], n1).view(B, S, c["kv_heads"], c["head_dim"])
        v = lin(layer["wv"], n1).view(B, S, c["kv_heads"], c["head_dim"])
        o = _ref_attention(_ref_prologue(q, None, cos, sin, 0), _ref_prologue(k, None, cos, sin, 0), v)
        x = x + lin(layer["wo"], o.reshape(B, S, -1))
        n2 = rms(x, layer["mlp_norm"])
        x = x + lin(layer["down"], F.silu(lin(layer["gate"], n2)) * lin(layer["up"], n2))
    logits = rms(x, model.final_norm) @ emb.t()
    return F.cross_entropy(logits.view(-1, c["vocab"]), targets.cpu().view(-1)), leaves


@pytest.mark.parametrize("backend", ["cfops", "torch"])
def test_smollm_lora_train_step_matches_float64_reference(backend):
    """Two layers of the SmolLM-135M shape, batch 2, seq 48: loss and every
    LoRA gradient against the float64 CPU model with the reference attention,
    with the layer ops in libcfattn.so (cfops) or as torch ops."""
    import torch

    from cpuforge_amd.train_bench import SmolLM
    print(f"smollm backend={backend}", flush=True)
    model = SmolLM(layers=2, seq=48, rank=16, backend=backend)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(11)
    tokens = torch.randint(0, model.c["vocab"], (2, 48), generator=gen, device="cuda")
    targets = torch.randint(0, model.c["vocab"], (2, 48), generator=gen, device="cuda")
    # B starts at zero (linear.rs:44-53); give it values so every path carries gradient.
    with torch.no_grad():
        for p_ in model.params():
            if p_.shape[1] == 16:
                p_.copy_(0.05 * torch.randn(p_.shape, generator=gen, device="cuda"))
    loss = model.loss(tokens, targets)
    loss.backward()
    torch.cuda.synchronize()
    ref, leaves = _reference_loss(model, tokens, targets)
    ref.backward()
    assert abs(float(loss) - float(ref)) <= 1e-5 * abs(float(ref)), (float(loss), float(ref))
    worst = 0.0
    for p_, r in zip(model.params(), leaves):
        a = p_.grad.detach().cpu().double().numpy()
        rr = r.grad.numpy()
        worst = max(worst, float((np.abs(a - rr) / (1 + np.abs(rr))).max()))
    print(f"loss {float(loss):.6f} ref {float(ref):.6f}; worst LoRA grad metric {worst:.3e}", flush=True)
    assert worst <= 1e-4
