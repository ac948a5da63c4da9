"""GPU parity of the fused attention prologue (Layer::forward's q/k RMSNorm +
RoPE, crates/model/src/layer.rs:104-116) and its backward chain
(layer.rs:191-206), alone and fused with the attention op, against the
oracle's restatement of rmsnorm_forward/backward (core/src/ops/rmsnorm.rs)
and RopeCache::apply (core/src/ops/rope.rs:71-89).

Tolerances: the prologue forward is elementwise per row in the reference's
f32 order, so it is compared bit for bit; its backward and the fused
attention follow the attention bars (fp32 mode max abs 1e-4, bf16 mode
max|a-r|/max|r| 2e-2), and the norm-gain gradients, which sum over every
(token, head) row, use the reference's gradcheck metric |a-r|/(1+|r|) <= 1e-4.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests.cases import CONFIGS, grad_metric, max_abs, rel_err, seq_inputs, norm_gains

pytestmark = pytest.mark.gpu

F32_TOL = 1e-4
BF16_TOL = 2e-2
L3 = (32.0, 1.0, 4.0, 8192.0)

# name: (batch, seq, n_heads, n_kv, head_dim, theta, scaling, qk_norm, pos0)
PROLOGUES = {
    "plain": (2, 37, 6, 2, 64, 1e4, None, False, 0),
    "llama3": (1, 50, 4, 1, 64, 5e5, L3, False, 3),
    "qknorm": (2, 29, 4, 2, 128, 1e6, None, True, 0),
    "qknorm_pos": (1, 17, 2, 2, 32, 1e6, None, True, 7),
}


@pytest.fixture(scope="module")
def env():
    import torch

    import cpuforge_amd as cf
    from cpuforge_amd import device as D
    ctx = cf.Context(0)
    yield torch, cf, D, ctx
    ctx.close()


def _setup(env, name, seed=900):
    torch, cf, D, ctx = env
    B, S, Hq, Hk, Dh, theta, sc, qkn, pos0 = PROLOGUES[name]
    max_pos = S + pos0
    rope = cf.RopeCache(Dh, max_pos, theta, cf.Llama3Scaling(*sc) if sc else None)
    cos, sin = O.rope_table(Dh, max_pos, theta, sc)
    qw = kw = None
    if qkn:
        qw = (1.0 + O.rand(Dh, seed + 50, 0.02)).astype(np.float32)
        kw = (1.0 + O.rand(Dh, seed + 51, 0.02)).astype(np.float32)
    pr = D.DeviceRope(rope, "cuda", pos0, torch.from_numpy(qw).cuda() if qkn else None,
                      torch.from_numpy(kw).cuda() if qkn else None, 1e-6)
    qp = [O.rand(S * Hq * Dh, seed + 16 * b, 1.0) for b in range(B)]
    kp = [O.rand(S * Hk * Dh, seed + 16 * b + 1, 1.0) for b in range(B)]
    ref = [O.layer_prologue_forward(qp[b], kp[b], S, Hq, Hk, Dh, cos, sin, max_pos, pos0, qw, kw, 1e-6)
           for b in range(B)]
    return (B, S, Hq, Hk, Dh, pos0, max_pos, cos, sin, qw, kw), pr, qp, kp, ref


def _dev(torch, arrs, B, S, H, Dh, dtype=None):
    import torch as T
    t = T.from_numpy(np.stack(arrs)).view(B, S, H, Dh).cuda()
    return t if dtype is None else t.to(dtype)


@pytest.mark.parametrize("name", sorted(PROLOGUES))
def test_prologue_forward_is_bitwise_the_reference(env, name):
    torch, cf, D, ctx = env
    (B, S, Hq, Hk, Dh, *_), pr, qp, kp, ref = _setup(env, name)
    q_pre, k_pre = _dev(torch, qp, B, S, Hq, Dh), _dev(torch, kp, B, S, Hk, Dh)
    for dt in (torch.float32, torch.bfloat16):
        q, k, qr, kr = D.prologue_fwd(q_pre, k_pre, pr, dtype=dt, ctx=ctx)
        torch.cuda.synchronize()
        for b in range(B):
            rq, rk, rqr, rkr = ref[b]
            if dt == torch.float32:
                assert np.array_equal(q[b].cpu().numpy().reshape(-1), rq), f"{name} q seq {b}"
                assert np.array_equal(k[b].cpu().numpy().reshape(-1), rk), f"{name} k seq {b}"
            else:
                got_q = q[b].view(torch.int16).cpu().numpy().reshape(-1).view(np.uint16)
                got_k = k[b].view(torch.int16).cpu().numpy().reshape(-1).view(np.uint16)
                assert np.array_equal(got_q, O.f32_to_bf16_bits(rq)), f"{name} bf16 q seq {b}"
                assert np.array_equal(got_k, O.f32_to_bf16_bits(rk)), f"{name} bf16 k seq {b}"
            if qr is not None:
                n_q, n_k = S * Hq, S * Hk
                assert np.array_equal(qr.cpu().numpy()[b * n_q:(b + 1) * n_q], rqr)
                assert np.array_equal(kr.cpu().numpy()[b * n_k:(b + 1) * n_k], rkr)


@pytest.mark.parametrize("name", sorted(PROLOGUES))
def test_prologue_backward_matches_reference_chain(env, name):
    torch, cf, D, ctx = env
    (B, S, Hq, Hk, Dh, pos0, max_pos, cos, sin, qw, kw), pr, qp, kp, ref = _setup(env, name)
    gq = [O.rand(S * Hq * Dh, 40 + b, 1.0) for b in range(B)]
    gk = [O.rand(S * Hk * Dh, 60 + b, 1.0) for b in range(B)]
    q_pre, k_pre = _dev(torch, qp, B, S, Hq, Dh), _dev(torch, kp, B, S, Hk, Dh)
    _, _, qr, kr = D.prologue_fwd(q_pre, k_pre, pr, dtype=torch.float32, ctx=ctx)
    dq_pre, dk_pre, dqw, dkw = D.prologue_bwd(_dev(torch, gq, B, S, Hq, Dh), _dev(torch, gk, B, S, Hk, Dh), q_pre,
                                              k_pre, qr, kr, pr, ctx=ctx)
    torch.cuda.synchronize()
    want_qw = np.zeros(Dh) if qw is not None else None
    want_kw = np.zeros(Dh) if kw is not None else None
    for b in range(B):
        _, _, rqr, rkr = ref[b]
        rdq, rdk, rqw, rkw = O.layer_prologue_backward(gq[b], gk[b], qp[b], kp[b], S, Hq, Hk, Dh, cos, sin, max_pos,
                                                       pos0, qw, kw, rqr, rkr)
        eq = max_abs(dq_pre[b].cpu().numpy().reshape(-1), rdq)
        ek = max_abs(dk_pre[b].cpu().numpy().reshape(-1), rdk)
        print(f"{name} seq {b}: dq_pre {eq:.3e} dk_pre {ek:.3e}", flush=True)
        assert eq <= 1e-5 and ek <= 1e-5, f"{name} seq {b}: dq_pre {eq}, dk_pre {ek}"
        if qw is not None:
            want_qw += rqw
            want_kw += rkw
    if qw is not None:
        eqw = O.grad_close_metric(dqw.cpu().numpy(), want_qw)[0]
        ekw = O.grad_close_metric(dkw.cpu().numpy(), want_kw)[0]
        print(f"{name}: dq_norm {eqw:.3e} dk_norm {ekw:.3e}", flush=True)
        assert eqw <= 1e-4 and ekw <= 1e-4, f"{name}: dq_norm {eqw}, dk_norm {ekw}"


def _oracle_layer(qp, kp, v, g, S, Hq, Hk, Dh, cos, sin, max_pos, pos0, qw, kw, bf16, heads=None):
    """Oracle chain for one sequence: prologue -> attention fwd -> attention
    bwd -> prologue bwd (layer.rs:104-121, 183-206).  With bf16 the attention
    inputs are rounded as the device rounds them."""
    q, k, qr, kr = O.layer_prologue_forward(qp, kp, S, Hq, Hk, Dh, cos, sin, max_pos, pos0, qw, kw, 1e-6)
    if bf16:
        q, k, v, g = (O.round_bf16(x) for x in (q, k, v, g))
    o = np.zeros(S * Hq * Dh, np.float32)
    lse = np.zeros(Hq * S, np.float32)
    O.attention_forward_blocked(q, k, v, o, lse, S, Hq, Hk, Dh, 128, heads=heads)
    dq, dk, dv = np.zeros_like(o), np.zeros(S * Hk * Dh, np.float32), np.zeros(S * Hk * Dh, np.float32)
    O.attention_backward_blocked(g, q, k, v, o, lse, dq, dk, dv, S, Hq, Hk, Dh, 128, heads=heads)
    dqp, dkp, dqw, dkw = O.layer_prologue_backward(dq, dk, qp, kp, S, Hq, Hk, Dh, cos, sin, max_pos, pos0, qw, kw,
                                                   qr, kr)
    return o, lse, dqp, dkp, dv, dqw, dkw


@pytest.mark.parametrize("name", sorted(PROLOGUES))
def test_fused_layer_attention_f32(env, name):
    """cfattn_fused_fwd / cfattn_fused_bwd (q_pre, k_pre -> O, lse ->
    dq_pre, dk_pre, dv and the norm-gain gradients) in fp32 mode."""
    torch, cf, D, ctx = env
    (B, S, Hq, Hk, Dh, pos0, max_pos, cos, sin, qw, kw), pr, qp, kp, _ = _setup(env, name)
    v = [O.rand(S * Hk * Dh, 300 + b, 1.0) for b in range(B)]
    g = [O.rand(S * Hq * Dh, 400 + b, 1.0) for b in range(B)]
    q_pre, k_pre = _dev(torch, qp, B, S, Hq, Dh), _dev(torch, kp, B, S, Hk, Dh)
    vd, gd = _dev(torch, v, B, S, Hk, Dh), _dev(torch, g, B, S, Hq, Dh)
    o, lse, q, k, qr, kr = D.fused_fwd(q_pre, k_pre, vd, pr, ctx=ctx)
    dqp, dkp, dv, dqw, dkw = D.fused_bwd(gd, q_pre, k_pre, q, k, vd, o, lse, qr, kr, pr, ctx=ctx)
    torch.cuda.synchronize()
    sum_qw = np.zeros(Dh) if qw is not None else None
    sum_kw = np.zeros(Dh) if qw is not None else None
    for b in range(B):
        ro, rl, rdqp, rdkp, rdv, rqw, rkw = _oracle_layer(qp[b], kp[b], v[b], g[b], S, Hq, Hk, Dh, cos, sin, max_pos,
                                                          pos0, qw, kw, False)
        for nm, a, r in (("o", o, ro), ("lse", lse, rl), ("dq_pre", dqp, rdqp), ("dk_pre", dkp, rdkp),
                         ("dv", dv, rdv)):
            e = max_abs(a[b].cpu().numpy().reshape(-1), r)
            assert e <= F32_TOL, f"{name} {nm} seq {b}: {e}"
        if qw is not None:
            sum_qw += rqw
            sum_kw += rkw
    if qw is not None:
        assert O.grad_close_metric(dqw.cpu().numpy(), sum_qw)[0] <= 1e-4
        assert O.grad_close_metric(dkw.cpu().numpy(), sum_kw)[0] <= 1e-4


@pytest.mark.parametrize("cfg_name", ["C3", "C4"])
def test_fused_config_bf16(env, cfg_name):
    """C3 (Llama-3 RoPE scaling) and C4 (Qwen3 q/k norm) at full size in bf16
    mode through the fused entry points; sequences 0 and B-1 and the first
    and last KV groups are checked against the oracle chain."""
    torch, cf, D, ctx = env
    cfg = CONFIGS[cfg_name]
    B, S, Hq, Hk, Dh, grp = cfg.batch, cfg.seq, cfg.n_heads, cfg.n_kv, cfg.head_dim, cfg.group
    print(f"{cfg_name}: B={B} S={S} {Hq}/{Hk} D={Dh}", flush=True)
    cos, sin = O.rope_table(Dh, S, cfg.theta, cfg.scaling)
    rope = cf.RopeCache(Dh, S, cfg.theta, cf.Llama3Scaling(*cfg.scaling) if cfg.scaling else None)
    qw = kw = None
    if cfg.qk_norm:
        qw, kw = norm_gains(cfg)
    pr = D.DeviceRope(rope, "cuda", 0, torch.from_numpy(qw).cuda() if qw is not None else None,
                      torch.from_numpy(kw).cuda() if kw is not None else None, cfg.eps)
    host = [seq_inputs(cfg, b) for b in range(B)]
    q_pre = _dev(torch, [h[0] for h in host], B, S, Hq, Dh)
    k_pre = _dev(torch, [h[1] for h in host], B, S, Hk, Dh)
    vd = _dev(torch, [O.round_bf16(h[2]) for h in host], B, S, Hk, Dh, torch.bfloat16)
    gd = _dev(torch, [O.round_bf16(h[3]) for h in host], B, S, Hq, Dh, torch.bfloat16)
    o, lse, q, k, qr, kr = D.fused_fwd(q_pre, k_pre, vd, pr, ctx=ctx)
    dqp, dkp, dv, dqw, dkw = D.fused_bwd(gd, q_pre, k_pre, q, k, vd, o, lse, qr, kr, pr, ctx=ctx)
    torch.cuda.synchronize()
    worst, gworst = {}, {}
    for b in (0, B - 1):
        qp, kp, v, g = host[b]
        for gi in (0, Hk - 1):
            h0, h1 = gi * grp, (gi + 1) * grp
            ro, rl, rdqp, rdkp, rdv, _, _ = _oracle_layer(qp, kp, v, g, S, Hq, Hk, Dh, cos, sin, S, 0, qw, kw, True,
                                                          heads=(h0, h1))
            selq = lambda x: x.reshape(S, Hq, Dh)[:, h0:h1]  # noqa: E731
            selk = lambda x: x.reshape(S, Hk, Dh)[:, gi]  # noqa: E731
            pairs = {"o": (selq(o[b].cpu().numpy()), selq(ro)),
                     "lse": (lse[b].cpu().numpy()[h0:h1], rl.reshape(Hq, S)[h0:h1]),
                     "dq_pre": (selq(dqp[b].cpu().numpy()), selq(rdqp)),
                     "dk_pre": (selk(dkp[b].cpu().numpy()), selk(rdkp)),
                     "dv": (selk(dv[b].cpu().numpy()), selk(rdv))}
            for nm, (a, r) in pairs.items():
                worst[nm] = max(worst.get(nm, 0.0), rel_err(a, r))
                gworst[nm] = max(gworst.get(nm, 0.0), grad_metric(a, r))
    print(f"{cfg_name} bf16 fused: " + ", ".join(f"{n} {e:.3e}" for n, e in worst.items()), flush=True)
    print(f"{cfg_name} bf16 fused gradcheck |a-r|/(1+|r|): " + ", ".join(f"{n} {e:.3e}" for n, e in gworst.items()),
          flush=True)
    for nm, e in worst.items():
        assert e <= BF16_TOL, f"{cfg_name} {nm}: {e}"
    for nm, e in gworst.items():
        assert e <= BF16_TOL, f"{cfg_name} {nm} gradcheck metric: {e}"


# Shapes of the fast bf16 kernels (head_dim 64 and 128; stored-dS dQ at 128),
# with and without the Qwen3 norm, and a ragged tail.
EPILOGUE_SHAPES = {
    "plain": PROLOGUES["plain"],
    "llama3": PROLOGUES["llama3"],
    "qknorm": PROLOGUES["qknorm"],
    "rope128": (2, 97, 8, 2, 128, 5e5, None, False, 5),
    "qknorm64": (1, 70, 4, 4, 64, 1e6, None, True, 2),
}


class _DsLimit:
    def __init__(self, ctx, nbytes):
        self.ctx, self.nbytes = ctx, nbytes

    def __enter__(self):
        self.old = self.ctx.ds_limit
        self.ctx.ds_limit = self.nbytes

    def __exit__(self, *a):
        self.ctx.ds_limit = self.old


# The Qwen3 shapes again through each variant of the fused backward: the norm
# backward in the epilogues (default) with the stored-dS dQ kernel, with the
# recompute dQ kernel (no dS scratch), with the two-waves-per-SIMD dK/dV
# kernel; and the unrotated rows stored for a separate norm pass
# (CFATTN_NORM_EPILOGUE=0).
NORM_VARIANTS = ["qknorm-nods", "qknorm-ws", "qknorm-sep", "qknorm64-sep", "qknorm-ragged", "qknorm-offset-x"]
EPILOGUE_SHAPES["qknorm-ragged"] = (3, 161, 8, 2, 128, 1e6, None, True, 4)


@pytest.mark.parametrize("name", sorted(EPILOGUE_SHAPES) + ["rope128-offset-tables", "qknorm64-offset-tables"] +
                         NORM_VARIANTS)
def test_fused_bwd_epilogue_matches_separate_passes(env, name, monkeypatch):
    """In bf16 mode cfattn_fused_bwd folds the inverse RoPE into the dQ and
    dK kernels' epilogues (adding into dq_pre/dk_pre) and, with the Qwen3
    norm, the norm backward too (or, with CFATTN_NORM_EPILOGUE=0, stores the
    unrotated rows for a norm-only pass).  dq_pre, dk_pre and dv must be the
    same bits as the attention backward into zeroed dq/dk followed by the
    separate prologue backward, also on top of nonzero dq_pre/dk_pre.  The
    norm gains' gradients are the same sums over every (token, head) row in
    another fixed order when the epilogues form them (their own partial sums
    per wave): within |a-r|/(1+|r|) <= 1e-5 of the separate pass's, and the
    same bits with the norm-only pass.  With cos/sin tables 4 bytes off a
    16-byte boundary (the epilogue reads them 16 bytes at a time) the fused
    call takes the separate passes itself; so it does with q_pre/k_pre rows
    off a 16-byte boundary."""
    offset_tables = name.endswith("-offset-tables")
    offset_x = name.endswith("-offset-x")
    name = name.replace("-offset-tables", "").replace("-offset-x", "")
    variant = None
    for suffix in ("-nods", "-ws", "-sep"):
        if name.endswith(suffix):
            variant, name = suffix[1:], name[: -len(suffix)]
    if variant == "ws":
        monkeypatch.setenv("CFATTN_DKDV_KERNEL", "ws")
    if variant == "sep":
        monkeypatch.setenv("CFATTN_NORM_EPILOGUE", "0")
    torch, cf, D, ctx = env
    with _DsLimit(ctx, 0 if variant == "nods" else ctx.ds_limit):
        _epilogue_case(torch, cf, D, ctx, name, offset_tables, offset_x, norm_in_epilogue=variant != "sep")


def _epilogue_case(torch, cf, D, ctx, name, offset_tables, offset_x, norm_in_epilogue):
    B, S, Hq, Hk, Dh, theta, sc, qkn, pos0 = EPILOGUE_SHAPES[name]
    max_pos = S + pos0
    rope = cf.RopeCache(Dh, max_pos, theta, cf.Llama3Scaling(*sc) if sc else None)
    qw = kw = None
    if qkn:
        qw = torch.from_numpy((1.0 + O.rand(Dh, 950, 0.02)).astype(np.float32)).cuda()
        kw = torch.from_numpy((1.0 + O.rand(Dh, 951, 0.02)).astype(np.float32)).cuda()
    pr = D.DeviceRope(rope, "cuda", pos0, qw, kw, 1e-6)
    if offset_tables:
        for nm in ("cos", "sin"):
            t = getattr(pr, nm)
            buf = torch.zeros(t.numel() + 1, dtype=t.dtype, device="cuda")
            buf[1:] = t.reshape(-1)
            setattr(pr, nm, buf[1:].view(t.shape))
            assert getattr(pr, nm).data_ptr() % 16 == 4
    torch.manual_seed(31)
    q_pre = torch.randn(B, S, Hq, Dh, device="cuda")
    k_pre = torch.randn(B, S, Hk, Dh, device="cuda")
    if offset_x:
        # Rows one float off a 16-byte boundary: the forward and the separate
        # passes take any alignment, the norm epilogue does not.
        bq = torch.zeros(q_pre.numel() + 1, device="cuda")
        bq[1:] = q_pre.reshape(-1)
        q_pre = bq[1:].view(B, S, Hq, Dh)
        assert q_pre.data_ptr() % 16 == 4
    vd = torch.randn(B, S, Hk, Dh, device="cuda").to(torch.bfloat16)
    gd = torch.randn(B, S, Hq, Dh, device="cuda").to(torch.bfloat16)
    init_q = torch.randn(B, S, Hq, Dh, device="cuda")
    init_k = torch.randn(B, S, Hk, Dh, device="cuda")
    o, lse, q, k, qr, kr = D.fused_fwd(q_pre, k_pre, vd, pr, ctx=ctx)
    fz = D.fused_bwd(gd, q_pre, k_pre, q, k, vd, o, lse, qr, kr, pr, dq_pre=init_q.clone(), dk_pre=init_k.clone(),
                     ctx=ctx)
    dq, dk, dv = D.bwd(gd, q, k, vd, o, lse, ctx=ctx)
    sp = D.prologue_bwd(dq, dk, q_pre, k_pre, qr, kr, pr, dq_pre=init_q.clone(), dk_pre=init_k.clone(), ctx=ctx)
    torch.cuda.synchronize()
    got = {"dq_pre": fz[0], "dk_pre": fz[1], "dv": fz[2]}
    want = {"dq_pre": sp[0], "dk_pre": sp[1], "dv": dv}
    for nm in got:
        a, r = got[nm].cpu().numpy(), want[nm].cpu().numpy()
        assert np.array_equal(a, r), f"{name} {nm}: max diff {np.abs(a - r).max():.3e}"
    if qkn:
        for i, j, nm in ((3, 2, "dq_norm"), (4, 3, "dk_norm")):
            a, r = fz[i].cpu().numpy(), sp[j].cpu().numpy()
            if norm_in_epilogue and not (offset_tables or offset_x):
                e = float(np.max(np.abs(a - r) / (1.0 + np.abs(r))))
                print(f"{name} {nm}: |a-r|/(1+|r|) {e:.2e} against the separate pass", flush=True)
                assert e <= 1e-5, f"{name} {nm}: {e:.3e}"
                assert not np.array_equal(a, np.zeros_like(a))
            else:
                assert np.array_equal(a, r), f"{name} {nm}: max diff {np.abs(a - r).max():.3e}"


def test_forward_and_backward_are_bitwise_repeatable(env):
    """Checkpoint mode recomputes the forward and expects the identical loss
    (crates/model/src/tests.rs:147-163): the kernels use no atomics, so two
    runs agree bit for bit, forward and backward, in both modes."""
    torch, cf, D, ctx = env
    torch.manual_seed(7)
    for dt in (torch.bfloat16, torch.float32):
        q = torch.randn(2, 300, 8, 128, device="cuda").to(dt)
        k = torch.randn(2, 300, 2, 128, device="cuda").to(dt)
        v = torch.randn(2, 300, 2, 128, device="cuda").to(dt)
        g = torch.randn(2, 300, 8, 128, device="cuda").to(dt)
        runs = []
        for _ in range(2):
            o, lse = D.fwd(q, k, v, ctx=ctx)
            dq, dk, dv = D.bwd(g, q, k, v, o, lse, ctx=ctx)
            torch.cuda.synchronize()
            runs.append([x.cpu().numpy() for x in (o, lse, dq, dk, dv)])
        for a, b in zip(*runs):
            assert np.array_equal(a, b)
