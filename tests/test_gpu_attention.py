"""GPU parity of the HIP attention kernels against the oracle.

The first four tests restate the reference's own attention tests
(crates/core/src/ops/attention.rs:324-393) with the GPU op in place of the
Rust one; the rest run the benchmark configurations through the batched
device entry points and compare with the oracle's f32 restatement of the
reference algorithm (fp32 mode: max abs error <= 1e-4 on O, lse, dQ, dK, dV;
bf16 mode: max|a-r|/max|r| <= 2e-2, oracle fed the same bf16-rounded inputs).
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests.cases import CASES, CONFIGS, case, grad_metric, max_abs, rel_err, rope_tables, seq_inputs

pytestmark = pytest.mark.gpu

F32_TOL = 1e-4  # fp32 parity bar (max abs)
BF16_TOL = 2e-2  # bf16 parity bar (max relative)


@pytest.fixture(scope="module")
def cf():
    import cpuforge_amd
    ctx = cpuforge_amd.Context(0)
    yield cpuforge_amd, ctx
    ctx.close()


def _fwd(cf, q, k, v, s, qb=128):
    mod, ctx = cf
    o = np.zeros(s.seq * s.n_heads * s.head_dim, np.float32)
    lse = np.zeros(s.n_heads * s.seq, np.float32)
    mod.attention_forward_blocked(q, k, v, o, lse, s, qb, ctx)
    return o, lse


def test_forward_matches_f64_reference(cf):
    mod, _ = cf
    for i, (seq, h, kv, hd, qb) in enumerate(CASES):
        print(f"case {i}: seq={seq} h={h} kv={kv} hd={hd} qb={qb}", flush=True)
        q, k, v = case(seq, h, kv, hd, 10 + i)
        s = mod.AttnShape(seq, h, kv, hd)
        o, lse = _fwd(cf, q, k, v, s, qb)
        want, want_lse = O.attn_ref_f64(q, k, v, seq, h, kv, hd)
        err, _ = O.grad_close_metric(o, want)
        assert err <= 1e-4, f"attn fwd case {i}: {err}"
        assert O.grad_close_metric(lse, want_lse)[0] <= 1e-4
        # and against the f32 restatement of attention_forward_blocked
        o_ref = np.zeros_like(o)
        l_ref = np.zeros_like(lse)
        O.attention_forward_blocked(q, k, v, o_ref, l_ref, seq, h, kv, hd, qb)
        assert max_abs(o, o_ref) <= F32_TOL and max_abs(lse, l_ref) <= F32_TOL


def test_block_size_does_not_change_result(cf):
    mod, _ = cf
    q, k, v = case(37, 4, 2, 8, 30)
    s = mod.AttnShape(37, 4, 2, 8)
    runs = [_fwd(cf, q, k, v, s, qb) for qb in (1, 16, 1000)]
    for o, lse in runs[1:]:
        assert np.abs(o - runs[0][0]).max() < 1e-5
        assert np.abs(lse - runs[0][1]).max() < 1e-5


def test_first_token_attends_only_to_itself(cf):
    mod, _ = cf
    q, k, v = case(5, 2, 1, 4, 40)
    o, _ = _fwd(cf, q, k, v, mod.AttnShape(5, 2, 1, 4))
    for h in range(2):
        assert np.abs(o[h * 4:(h + 1) * 4] - v[0:4]).max() < 1e-6


def test_backward_matches_f64_gradients_and_finite_differences(cf):
    mod, ctx = cf
    for i, (seq, h, kv, hd, qb) in enumerate(CASES):
        print(f"case {i}", flush=True)
        q, k, v = case(seq, h, kv, hd, 50 + i)
        g = O.rand(seq * h * hd, 70 + i, 1.0)
        s = mod.AttnShape(seq, h, kv, hd)
        o, lse = _fwd(cf, q, k, v, s, qb)
        dq = np.zeros_like(q)
        dk = np.zeros_like(k)
        dv = np.zeros_like(v)
        mod.attention_backward_blocked(g, q, k, v, o, lse, dq, dk, dv, s, qb, ctx)
        wq, wk, wv = O.attn_bwd_ref_f64(g, q, k, v, seq, h, kv, hd)
        for name, a, w in (("dq", dq, wq), ("dk", dk, wk), ("dv", dv, wv)):
            assert max_abs(a, w) <= F32_TOL, f"{name} case {i}: {max_abs(a, w)}"
        # finite differences of the f64 reference forward (attention.rs:378-392)
        q64, k64, v64, g64 = (x.astype(np.float64) for x in (q, k, v, g))

        def loss(qq, kk, vv):
            return float(np.dot(O.attn_ref_f64(qq, kk, vv, seq, h, kv, hd)[0], g64))

        for name, a, x, which in (("dq", dq, q64, 0), ("dk", dk, k64, 1), ("dv", dv, v64, 2)):
            num = np.zeros_like(x)
            for j in range(x.size):
                xp = x.copy()
                xm = x.copy()
                xp[j] += 1e-6
                xm[j] -= 1e-6
                args_p = [q64, k64, v64]
                args_m = [q64, k64, v64]
                args_p[which] = xp
                args_m[which] = xm
                num[j] = (loss(*args_p) - loss(*args_m)) / 2e-6
            assert O.grad_close_metric(a, num)[0] <= 1e-3, f"attn {name} case {i} vs finite differences"


def test_backward_accumulates(cf):
    mod, ctx = cf
    q, k, v = case(40, 6, 2, 16, 5)
    g = O.rand(q.size, 6, 1.0)
    s = mod.AttnShape(40, 6, 2, 16)
    o, lse = _fwd(cf, q, k, v, s)
    grads = [np.zeros_like(x) for x in (q, k, v)]
    mod.attention_backward(g, q, k, v, o, lse, *grads, s, ctx)
    once = [x.copy() for x in grads]
    mod.attention_backward(g, q, k, v, o, lse, *grads, s, ctx)
    for a, b in zip(grads, once):
        assert np.abs(a - 2 * b).max() <= 1e-6 * (1 + np.abs(b).max())


def _prologue_cpu(cfg, qp, kp):
    cos, sin = rope_tables(cfg)
    q, k, _, _ = O.layer_prologue_forward(qp, kp, cfg.seq, cfg.n_heads, cfg.n_kv, cfg.head_dim, cos, sin, cfg.seq)
    return q, k


def test_c1_f32_parity(cf):
    """C1: SmolLM-135M layer, f32, RoPE theta 1e4; the host-slice drop-in."""
    mod, ctx = cf
    cfg = CONFIGS["C1"]
    qp, kp, v, g = seq_inputs(cfg, 0)
    q, k = _prologue_cpu(cfg, qp, kp)
    s = mod.AttnShape(cfg.seq, cfg.n_heads, cfg.n_kv, cfg.head_dim)
    o, lse = _fwd(cf, q, k, v, s)
    dq, dk, dv = (np.zeros_like(x) for x in (q, k, v))
    mod.attention_backward(g, q, k, v, o, lse, dq, dk, dv, s, ctx)
    ro, rl = np.zeros_like(o), np.zeros_like(lse)
    O.attention_forward_blocked(q, k, v, ro, rl, *s.__dict__.values(), 128)
    rq, rk, rv = (np.zeros_like(x) for x in (q, k, v))
    O.attention_backward_blocked(g, q, k, v, ro, rl, rq, rk, rv, *s.__dict__.values(), 128)
    for name, a, r in (("o", o, ro), ("lse", lse, rl), ("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        e = max_abs(a, r)
        print(f"C1 f32 {name}: max abs {e:.3e}", flush=True)
        assert e <= F32_TOL, name


def _device_check(cf, cfg, mode, seqs, head_groups):
    """Run the whole batch on the GPU; check the listed sequences and KV
    groups against the oracle's f32 restatement."""
    import torch
    from cpuforge_amd import device as D
    mod, ctx = cf
    B, S, Hq, Hk, Dh = cfg.batch, cfg.seq, cfg.n_heads, cfg.n_kv, cfg.head_dim
    grp = cfg.group
    cos, sin = rope_tables(cfg)
    host = []
    for b in range(B):
        qp, kp, v, g = seq_inputs(cfg, b)
        q, k, _, _ = O.layer_prologue_forward(qp, kp, S, Hq, Hk, Dh, cos, sin, S)
        if mode == "bf16":
            q, k, v, g = (O.round_bf16(x) for x in (q, k, v, g))
        host.append((q, k, v, g))
    tdt = torch.bfloat16 if mode == "bf16" else torch.float32

    def dev(i, heads):
        return torch.from_numpy(np.stack([h[i] for h in host])).view(B, S, heads, Dh).to("cuda").to(tdt)

    q, k, v, g = dev(0, Hq), dev(1, Hk), dev(2, Hk), dev(3, Hq)
    o, lse = D.fwd(q, k, v, ctx=ctx)
    dq, dk, dv = D.bwd(g, q, k, v, o, lse, ctx=ctx)
    torch.cuda.synchronize()
    o, lse, dq, dk, dv = (x.cpu().numpy() for x in (o, lse, dq, dk, dv))
    worst, gworst = {}, {}
    for b in seqs:
        hq, hk, hv, hg = host[b]
        for grp_i in head_groups:
            h0, h1 = grp_i * grp, (grp_i + 1) * grp
            ro = np.zeros(S * Hq * Dh, np.float32)
            rl = np.zeros(Hq * S, np.float32)
            O.attention_forward_blocked(hq, hk, hv, ro, rl, S, Hq, Hk, Dh, 128, heads=(h0, h1))
            rq = np.zeros_like(ro)
            rk = np.zeros(S * Hk * Dh, np.float32)
            rv = np.zeros_like(rk)
            O.attention_backward_blocked(hg, hq, hk, hv, ro, rl, rq, rk, rv, S, Hq, Hk, Dh, 128, heads=(h0, h1))
            sel_q = lambda x: x.reshape(S, Hq, Dh)[:, h0:h1]  # noqa: E731
            sel_k = lambda x: x.reshape(S, Hk, Dh)[:, grp_i]  # noqa: E731
            pairs = {
                "o": (sel_q(o[b]), sel_q(ro)),
                "lse": (lse[b][h0:h1], rl.reshape(Hq, S)[h0:h1]),
                "dq": (sel_q(dq[b]), sel_q(rq)),
                "dk": (sel_k(dk[b]), sel_k(rk)),
                "dv": (sel_k(dv[b]), sel_k(rv)),
            }
            for name, (a, r) in pairs.items():
                e = max_abs(a, r) if mode == "f32" else rel_err(a, r)
                worst[name] = max(worst.get(name, 0.0), e)
                if mode == "bf16":
                    gworst[name] = max(gworst.get(name, 0.0), grad_metric(a, r))
    print(f"{cfg.name} {mode}: " + ", ".join(f"{n} {e:.3e}" for n, e in worst.items()), flush=True)
    if mode == "bf16":
        print(f"{cfg.name} {mode} gradcheck |a-r|/(1+|r|): " + ", ".join(f"{n} {e:.3e}" for n, e in gworst.items()),
              flush=True)
    tol = F32_TOL if mode == "f32" else BF16_TOL
    for name, e in worst.items():
        assert e <= tol, f"{cfg.name} {mode} {name}: {e}"
    for name, e in gworst.items():
        assert e <= BF16_TOL, f"{cfg.name} {mode} {name} gradcheck metric: {e}"


@pytest.mark.parametrize("mode", ["f32", "bf16"])
def test_c2_parity(cf, mode):
    _device_check(cf, CONFIGS["C2"], mode, seqs=(0, 7), head_groups=(0, 2))


def test_c5_bf16_parity(cf):
    _device_check(cf, CONFIGS["C5"], "bf16", seqs=(0,), head_groups=(0, 7))


# Shapes that exercise the bf16 fast paths (head_dim 64/128, 16-byte rows):
# ragged last tiles, seq 1, GQA with 4/2/1 heads per workgroup, MHA and MQA,
# several sequences per call.  (batch, seq, n_heads, n_kv, head_dim)
FAST_SHAPES = [(1, 1, 4, 1, 128), (2, 33, 4, 2, 64), (1, 100, 8, 2, 128), (1, 257, 6, 3, 64),
               (2, 130, 3, 3, 128), (1, 200, 4, 1, 64), (1, 511, 2, 2, 128)]


def _fast_inputs(shape, seed=500, mode="bf16"):
    import torch
    B, S, Hq, Hk, Dh = shape
    rnd = O.round_bf16 if mode == "bf16" else (lambda x: x)
    tdt = torch.bfloat16 if mode == "bf16" else torch.float32
    host = []
    for b in range(B):
        sd = seed + 16 * b
        host.append(tuple(rnd(O.rand(S * h * Dh, sd + i, 1.0)) for i, h in enumerate((Hq, Hk, Hk, Hq))))

    def dev(i, heads):
        return torch.from_numpy(np.stack([h[i] for h in host])).view(B, S, heads, Dh).to("cuda").to(tdt)

    return host, (dev(0, Hq), dev(1, Hk), dev(2, Hk), dev(3, Hq))


class _DsLimit:
    """Sets the context's stored-dS scratch limit for a block (0: dQ
    recomputes the softmax) and restores it afterwards."""

    def __init__(self, ctx, nbytes):
        self.ctx, self.nbytes = ctx, nbytes

    def __enter__(self):
        self.old = self.ctx.ds_limit
        self.ctx.ds_limit = self.nbytes

    def __exit__(self, *exc):
        self.ctx.ds_limit = self.old


@pytest.mark.parametrize("ds", ["stored", "recompute"])
@pytest.mark.parametrize("shape", FAST_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_bf16_fast_path_shapes(cf, shape, ds):
    import torch
    from cpuforge_amd import device as D
    mod, ctx = cf
    B, S, Hq, Hk, Dh = shape
    print(f"fast-path shape {shape}, dQ from {ds} dS", flush=True)
    host, (q, k, v, g) = _fast_inputs(shape)
    with _DsLimit(ctx, ctx.ds_limit if ds == "stored" else 0):
        o, lse = D.fwd(q, k, v, ctx=ctx)
        dq, dk, dv = D.bwd(g, q, k, v, o, lse, ctx=ctx)
        torch.cuda.synchronize()
    o, lse, dq, dk, dv = (x.cpu().numpy() for x in (o, lse, dq, dk, dv))
    for b in range(B):
        hq, hk, hv, hg = host[b]
        ro = np.zeros(S * Hq * Dh, np.float32)
        rl = np.zeros(Hq * S, np.float32)
        O.attention_forward_blocked(hq, hk, hv, ro, rl, S, Hq, Hk, Dh, 128)
        rq, rk, rv = np.zeros_like(ro), np.zeros(S * Hk * Dh, np.float32), np.zeros(S * Hk * Dh, np.float32)
        O.attention_backward_blocked(hg, hq, hk, hv, ro, rl, rq, rk, rv, S, Hq, Hk, Dh, 128)
        for name, a, r in (("o", o[b], ro), ("lse", lse[b], rl), ("dq", dq[b], rq), ("dk", dk[b], rk),
                           ("dv", dv[b], rv)):
            e = rel_err(a.reshape(-1), r)
            assert e <= BF16_TOL, f"{shape} seq {b} {name}: {e}"


@pytest.mark.parametrize("shape", [(1, 1024, 8, 2, 128), (2, 300, 4, 4, 128), (1, 700, 4, 1, 128)],
                         ids=lambda s: "x".join(map(str, s)))
def test_bf16_running_max_moves(cf, shape):
    """Keys whose scale grows along the sequence (x1 at token 0 to x12 at the
    end): every query row's running max moves several times, and tiles whose
    max stays within the lazy bound still carry large P sums.  The forward
    forms P against the running max first and settles a tile (exact max,
    rescale, P again) only when its sums show that the max may have moved,
    so this is the case where that matters; O, lse and the gradients must
    still match the oracle."""
    import torch
    from cpuforge_amd import device as D
    mod, ctx = cf
    B, S, Hq, Hk, Dh = shape
    print(f"running-max shape {shape}", flush=True)
    grow = (1.0 + 11.0 * np.arange(S, dtype=np.float32) / S).repeat(Hk * Dh)
    host = []
    for b in range(B):
        sd = 900 + 16 * b
        q = O.round_bf16(O.rand(S * Hq * Dh, sd, 1.0))
        k = O.round_bf16(O.rand(S * Hk * Dh, sd + 1, 1.0) * grow)
        v = O.round_bf16(O.rand(S * Hk * Dh, sd + 2, 1.0))
        g = O.round_bf16(O.rand(S * Hq * Dh, sd + 3, 1.0))
        host.append((q, k, v, g))

    def dev(i, heads):
        return torch.from_numpy(np.stack([h[i] for h in host])).view(B, S, heads, Dh).to("cuda").to(torch.bfloat16)

    q, k, v, g = dev(0, Hq), dev(1, Hk), dev(2, Hk), dev(3, Hq)
    o, lse = D.fwd(q, k, v, ctx=ctx)
    dq, dk, dv = D.bwd(g, q, k, v, o, lse, ctx=ctx)
    torch.cuda.synchronize()
    o, lse, dq, dk, dv = (x.cpu().numpy() for x in (o, lse, dq, dk, dv))
    for b in range(B):
        hq, hk, hv, hg = host[b]
        ro = np.zeros(S * Hq * Dh, np.float32)
        rl = np.zeros(Hq * S, np.float32)
        O.attention_forward_blocked(hq, hk, hv, ro, rl, S, Hq, Hk, Dh, 128)
        rq, rk, rv = np.zeros_like(ro), np.zeros(S * Hk * Dh, np.float32), np.zeros(S * Hk * Dh, np.float32)
        O.attention_backward_blocked(hg, hq, hk, hv, ro, rl, rq, rk, rv, S, Hq, Hk, Dh, 128)
        # The scores reach ~25 standard units: the softmax is far from flat.
        assert float(np.max(rl)) > 20.0
        for name, a, r in (("o", o[b], ro), ("lse", lse[b], rl), ("dq", dq[b], rq), ("dk", dk[b], rk),
                           ("dv", dv[b], rv)):
            e = rel_err(a.reshape(-1), r)
            assert e <= BF16_TOL, f"{shape} seq {b} {name}: {e}"


def _guard_case(Dh=128, S=320, Hq=4, Hk=1):
    """Every query row is one vector u and key j is a multiple of u, so that
    all rows see the same scores, tile by tile (log2 units against the first
    tile's max): 0, then 60 (P = 2^60 per key: a lane's share of the tile's
    P sum, 32 such keys, exceeds the forward's guard, 2^64, but the max stays
    within the lazy bound of 64, so m must not move), then 70 (m moves),
    then 130 (60 above the new max: trips again without a move), then a ramp
    to 200 (m moves).  Returns host q, k, v."""
    rng = np.random.default_rng(77)
    u = O.round_bf16(rng.standard_normal(Dh).astype(np.float32))
    target = np.concatenate([np.zeros(64), np.full(64, 60.0), np.full(64, 70.0), np.full(64, 130.0),
                             np.linspace(130.0, 200.0, 64)]).astype(np.float64)[:S]
    dots = target * np.sqrt(Dh) / np.log2(np.e)
    k = (dots[:, None] / float(np.dot(u, u))) * u[None, :]
    q = np.tile(u, (S, Hq, 1)).astype(np.float32).reshape(-1)
    k = O.round_bf16(k.astype(np.float32).reshape(-1))
    v = O.round_bf16(rng.standard_normal(S * Hk * Dh).astype(np.float32))
    return q, k, v


def test_bf16_guard_trips_with_and_without_a_max_move(cf):
    """The forward on _guard_case's scores: its guard trips on every tile,
    with and without a move of the running max.  O and lse must match the
    oracle."""
    import torch
    from cpuforge_amd import device as D
    mod, ctx = cf
    S, Hq, Hk, Dh = 320, 4, 1, 128
    q, k, v = _guard_case(Dh, S, Hq, Hk)
    qd, kd, vd = (torch.from_numpy(x).view(1, S, h, Dh).to("cuda").to(torch.bfloat16)
                  for x, h in ((q, Hq), (k, Hk), (v, Hk)))
    o, lse = D.fwd(qd, kd, vd, ctx=ctx)
    torch.cuda.synchronize()
    ro = np.zeros(S * Hq * Dh, np.float32)
    rl = np.zeros(Hq * S, np.float32)
    O.attention_forward_blocked(q, k, v, ro, rl, S, Hq, Hk, Dh, 128)
    assert float(np.max(rl)) > 130.0  # the scores reach ~139 natural units
    assert rel_err(o.cpu().numpy().reshape(-1), ro) <= BF16_TOL
    assert rel_err(lse.cpu().numpy().reshape(-1), rl) <= BF16_TOL


def test_bf16_forward_settles_exactly_where_the_guard_says(cf):
    """cfattn_fwd_stats counts the wave-tiles on which the head_dim-128
    forward takes its guard's slow path.  A wave of 64 queries walks the key
    tiles up to its diagonal, so a sequence of nqt = ceil(S/64) query tiles
    has Hq * nqt(nqt+1)/2 wave-tiles.  On _guard_case every one of them
    trips (the first tile of every wave against m = -inf, every later one
    above the guard); on N(0,1) scores only each wave's first tile does (no
    later tile comes near 2^64 times the first one's P)."""
    import torch
    from cpuforge_amd import device as D
    mod, ctx = cf
    S, Hq, Hk, Dh = 320, 4, 1, 128
    q, k, v = _guard_case(Dh, S, Hq, Hk)
    qd, kd, vd = (torch.from_numpy(x).view(1, S, h, Dh).to("cuda").to(torch.bfloat16)
                  for x, h in ((q, Hq), (k, Hk), (v, Hk)))
    nqt = (S + 63) // 64
    ctx.fwd_stats_enable(True)
    try:
        D.fwd(qd, kd, vd, ctx=ctx)
        assert ctx.fwd_stats_read() == Hq * nqt * (nqt + 1) // 2
        B, S, Hq, Hk = 2, 1000, 8, 2
        _, (q2, k2, v2, _g) = _fast_inputs((B, S, Hq, Hk, Dh), seed=2400)
        ctx.fwd_stats_enable(True)  # restarts the count
        D.fwd(q2, k2, v2, ctx=ctx)
        assert ctx.fwd_stats_read() == B * Hq * ((S + 63) // 64)
    finally:
        ctx.fwd_stats_enable(False)


@pytest.mark.parametrize("scratch", ["slots", "generic"])
@pytest.mark.parametrize("shape", FAST_SHAPES + [(3, 64, 9, 3, 64), (1, 96, 16, 2, 64)],
                         ids=lambda s: "x".join(map(str, s)))
def test_f32_fast_path_shapes(cf, shape, scratch):
    """The fp32 fast path (head_dim 64/128) over ragged lengths, GQA, MHA and
    MQA, batches, every query-split count; with the dK/dV scratch slots, and
    with the scratch capped to zero (the generic fp32 backward)."""
    import torch
    from cpuforge_amd import device as D
    mod, ctx = cf
    B, S, Hq, Hk, Dh = shape
    print(f"f32 fast-path shape {shape}, backward with {scratch}", flush=True)
    host, (q, k, v, g) = _fast_inputs(shape, seed=700, mode="f32")
    with _DsLimit(ctx, ctx.ds_limit if scratch == "slots" else 0):
        o, lse = D.fwd(q, k, v, ctx=ctx)
        dq, dk, dv = D.bwd(g, q, k, v, o, lse, ctx=ctx)
        torch.cuda.synchronize()
    o, lse, dq, dk, dv = (x.cpu().numpy() for x in (o, lse, dq, dk, dv))
    for b in range(B):
        hq, hk, hv, hg = host[b]
        ro = np.zeros(S * Hq * Dh, np.float32)
        rl = np.zeros(Hq * S, np.float32)
        O.attention_forward_blocked(hq, hk, hv, ro, rl, S, Hq, Hk, Dh, 128)
        rq, rk, rv = np.zeros_like(ro), np.zeros(S * Hk * Dh, np.float32), np.zeros(S * Hk * Dh, np.float32)
        O.attention_backward_blocked(hg, hq, hk, hv, ro, rl, rq, rk, rv, S, Hq, Hk, Dh, 128)
        for name, a, r in (("o", o[b], ro), ("lse", lse[b], rl), ("dq", dq[b], rq), ("dk", dk[b], rk),
                           ("dv", dv[b], rv)):
            e = max_abs(a.reshape(-1), r)
            assert e <= F32_TOL, f"{shape} seq {b} {name}: {e}"


def test_f32_fast_path_is_bitwise_repeatable(cf):
    """Fixed-order slot sums and key-split merges: the same fp32 forward and
    backward twice give the same bits."""
    import torch
    from cpuforge_amd import device as D
    mod, ctx = cf
    _, (q, k, v, g) = _fast_inputs((2, 300, 9, 3, 64), seed=800, mode="f32")
    fwds = [[x.cpu().numpy() for x in D.fwd(q, k, v, ctx=ctx)] for _ in range(2)]
    for a, b in zip(*fwds):
        assert np.array_equal(a, b)
    o, lse = D.fwd(q, k, v, ctx=ctx)
    runs = [[x.cpu().numpy() for x in D.bwd(g, q, k, v, o, lse, ctx=ctx)] for _ in range(2)]
    torch.cuda.synchronize()
    for a, b in zip(*runs):
        assert np.array_equal(a, b)


@pytest.mark.parametrize("ds", ["stored", "recompute"])
@pytest.mark.parametrize("shape", [(1, 1000, 8, 2, 128), (1, 1024, 8, 2, 128), (2, 300, 4, 4, 128)],
                         ids=lambda s: "x".join(map(str, s)))
def test_bf16_backward_is_bitwise_repeatable(cf, shape, ds):
    """The bf16 backward (one-wave-per-SIMD dK/dV, stored or recomputed dQ)
    four times on the same inputs gives the same bits: every sum has a fixed
    order, and the dK/dV accumulators are never read while an MFMA is still
    writing them (small grids, where one workgroup runs alone on its CU and
    the P waves pass each barrier last, are the timing that showed such a
    read)."""
    import torch
    from cpuforge_amd import device as D
    mod, ctx = cf
    print(f"bf16 backward repeat, shape {shape}, dS {ds}", flush=True)
    _, (q, k, v, g) = _fast_inputs(shape, seed=2100)
    o, lse = D.fwd(q, k, v, ctx=ctx)
    with _DsLimit(ctx, ctx.ds_limit if ds == "stored" else 0):
        runs = [[x.cpu().numpy() for x in D.bwd(g, q, k, v, o, lse, ctx=ctx)] for _ in range(4)]
    torch.cuda.synchronize()
    for r in runs[1:]:
        for name, a, b in zip(("dq", "dk", "dv"), runs[0], r):
            assert np.array_equal(a, b), f"{shape} {ds} {name}: max diff {np.abs(a - b).max()}"


@pytest.mark.parametrize("shape", [(8, 2048, 9, 3, 64), (4, 1500, 16, 4, 64), (2, 1000, 16, 8, 128)],
                         ids=lambda s: "x".join(map(str, s)))
def test_f32_persistent_grids_match_unit_grids(cf, shape, monkeypatch):
    """The fp32 forward, dQ and dK/dV kernels run persistent grids (each
    workgroup walks a snake of work units) on shapes that fill every
    workgroup slot; CFATTN_F32_GRID=unit launches one workgroup per unit.
    Each unit computes the same sums either way: O, lse, dQ, dK, dV must be
    bitwise equal."""
    import torch
    from cpuforge_amd import device as D
    mod, ctx = cf
    print(f"f32 persistent vs unit grids, shape {shape}", flush=True)
    _, (q, k, v, g) = _fast_inputs(shape, seed=2100, mode="f32")
    out = {}
    for grid in ("unit", "persistent"):
        if grid == "unit":
            monkeypatch.setenv("CFATTN_F32_GRID", "unit")
        else:
            monkeypatch.delenv("CFATTN_F32_GRID", raising=False)
        o, lse = D.fwd(q, k, v, ctx=ctx)
        out[grid] = [x.cpu().numpy() for x in (o, lse, *D.bwd(g, q, k, v, o, lse, ctx=ctx))]
    torch.cuda.synchronize()
    for name, a, b in zip(("o", "lse", "dq", "dk", "dv"), out["persistent"], out["unit"]):
        assert np.array_equal(a, b), f"{shape} {name}: max diff {np.abs(a - b).max()}"


@pytest.mark.parametrize("grid", ["persistent", "unit"])
@pytest.mark.parametrize("shape", [(8, 2048, 9, 3, 64), (4, 1500, 16, 4, 64), (8, 1024, 8, 2, 128),
                                   (8, 777, 12, 3, 64), (8, 512, 9, 3, 64), (3, 300, 8, 2, 128)],
                         ids=lambda s: "x".join(map(str, s)))
def test_f32_stored_ds_matches_recompute(cf, shape, grid, monkeypatch):
    """fp32 backward: dK/dV stores dS (fp32 blocks) and dQ reads it instead
    of recomputing S and dP (CFATTN_F32_DS=0).  dK/dV forms dS with the same
    arithmetic as the recompute and dQ sums it in the same order, so dQ, dK
    and dV must be bitwise equal, on persistent and per-unit grids; where the
    recompute's grid splits a query tile's keys (the last two shapes: its
    partial sums are added in split order), dQ agrees to 1e-5, as the split
    does with the unsplit grid."""
    import torch
    from cpuforge_amd import device as D
    mod, ctx = cf
    print(f"f32 stored dS vs recompute, shape {shape}, {grid} grids", flush=True)
    _, (q, k, v, g) = _fast_inputs(shape, seed=2300, mode="f32")
    if grid == "unit":
        monkeypatch.setenv("CFATTN_F32_GRID", "unit")
    o, lse = D.fwd(q, k, v, ctx=ctx)
    out = {}
    for ds in ("recompute", "stored"):
        if ds == "recompute":
            monkeypatch.setenv("CFATTN_F32_DS", "0")
        else:
            monkeypatch.delenv("CFATTN_F32_DS", raising=False)
        out[ds] = [x.cpu().numpy() for x in D.bwd(g, q, k, v, o, lse, ctx=ctx)]
    torch.cuda.synchronize()
    split = shape in ((8, 512, 9, 3, 64), (3, 300, 8, 2, 128))
    for name, a, b in zip(("dq", "dk", "dv"), out["stored"], out["recompute"]):
        if split and name == "dq":
            assert max_abs(a.reshape(-1), b.reshape(-1)) <= 1e-5, f"{shape} {grid} dq"
        else:
            assert np.array_equal(a, b), f"{shape} {grid} {name}: max diff {np.abs(a - b).max()}"


@pytest.mark.parametrize("shape", [(8, 2048, 9, 3, 64), (4, 1500, 16, 4, 64), (1, 4096, 32, 8, 64),
                                   (4, 1000, 16, 8, 128)],
                         ids=lambda s: "x".join(map(str, s)))
def test_bf16_persistent_grids_match_unit_grids(cf, shape, monkeypatch):
    """The bf16 two-waves-per-SIMD forward and the recompute dQ kernel run
    persistent grids where the tiles fill every workgroup slot, up to four per
    slot (walked tile-major at 8x2048, group-major at 1x4096), and the head_dim-
    64 wave-specialised dK/dV up to two key tiles per CU (8x2048, 1x4096; its
    persistent workgroups walk each key tile the way the per-tile grid does);
    CFATTN_BF16_GRID=unit launches one workgroup per tile.  At head_dim 128
    the two-waves-per-SIMD forward is selected (CFATTN_FWD_KERNEL=two) and dQ
    recomputes the softmax.  Each tile computes the same sums either way: O,
    lse, dQ, dK, dV must be bitwise equal."""
    import torch
    from cpuforge_amd import device as D
    mod, ctx = cf
    print(f"bf16 persistent vs unit grids, shape {shape}", flush=True)
    _, (q, k, v, g) = _fast_inputs(shape, seed=2200)
    if shape[4] == 128:
        monkeypatch.setenv("CFATTN_FWD_KERNEL", "two")
    out = {}
    with _DsLimit(ctx, 0):
        for grid in ("unit", "persistent"):
            if grid == "unit":
                monkeypatch.setenv("CFATTN_BF16_GRID", "unit")
            else:
                monkeypatch.delenv("CFATTN_BF16_GRID", raising=False)
            o, lse = D.fwd(q, k, v, ctx=ctx)
            out[grid] = [x.cpu().numpy() for x in (o, lse, *D.bwd(g, q, k, v, o, lse, ctx=ctx))]
    torch.cuda.synchronize()
    for name, a, b in zip(("o", "lse", "dq", "dk", "dv"), out["persistent"], out["unit"]):
        assert np.array_equal(a, b), f"{shape} {name}: max diff {np.abs(a - b).max()}"


@pytest.mark.parametrize("shape", [(8, 512, 9, 3, 64), (1, 2048, 4, 1, 128), (1, 1000, 8, 8, 64)],
                         ids=lambda s: "x".join(map(str, s)))
def test_f32_key_split_matches_oracle_and_unsplit(cf, shape):
    """Small grids split long query tiles over key runs (four key tiles at
    the SmolLM-135M train shape, batch 8 x seq 512, 9/3 heads) and merge the
    parts in split order.  O, lse and dQ of the split path against the oracle
    on the first and last sequence, and the forward against the unsplit grid
    (scratch limit 0) on every sequence."""
    import torch
    from cpuforge_amd import device as D
    mod, ctx = cf
    B, S, Hq, Hk, Dh = shape
    print(f"f32 key split {shape}", flush=True)
    host, (q, k, v, g) = _fast_inputs(shape, seed=900, mode="f32")
    o, lse = D.fwd(q, k, v, ctx=ctx)
    dq, dk, dv = D.bwd(g, q, k, v, o, lse, ctx=ctx)
    with _DsLimit(ctx, 0):
        o1, lse1 = D.fwd(q, k, v, ctx=ctx)
    torch.cuda.synchronize()
    assert max_abs(o.cpu().numpy().reshape(-1), o1.cpu().numpy().reshape(-1)) <= 1e-5
    assert max_abs(lse.cpu().numpy().reshape(-1), lse1.cpu().numpy().reshape(-1)) <= 1e-5
    o, lse, dq, dk, dv = (x.cpu().numpy() for x in (o, lse, dq, dk, dv))
    for b in sorted({0, B - 1}):
        hq, hk, hv, hg = host[b]
        ro = np.zeros(S * Hq * Dh, np.float32)
        rl = np.zeros(Hq * S, np.float32)
        O.attention_forward_blocked(hq, hk, hv, ro, rl, S, Hq, Hk, Dh, 128)
        rq, rk, rv = np.zeros_like(ro), np.zeros(S * Hk * Dh, np.float32), np.zeros(S * Hk * Dh, np.float32)
        O.attention_backward_blocked(hg, hq, hk, hv, ro, rl, rq, rk, rv, S, Hq, Hk, Dh, 128)
        for name, a, r in (("o", o[b], ro), ("lse", lse[b], rl), ("dq", dq[b], rq), ("dk", dk[b], rk),
                           ("dv", dv[b], rv)):
            e = max_abs(a.reshape(-1), r)
            assert e <= F32_TOL, f"{shape} seq {b} {name}: {e}"


@pytest.mark.parametrize("shape", [(1, 300, 8, 2, 128), (2, 97, 4, 4, 128), (1, 1000, 4, 1, 128)],
                         ids=lambda s: "x".join(map(str, s)))
def test_stored_ds_matches_recompute(cf, shape):
    """dQ from the dS the dK/dV kernel stores against dQ with the softmax
    recomputed: the dK/dV kernel's arithmetic is the same in both, so dK and
    dV are bitwise equal; dQ sums the same bf16-rounded dS values in the
    same key order and may differ only where the two kernels' products of S
    and dP round differently."""
    import torch
    from cpuforge_amd import device as D
    mod, ctx = cf
    print(f"stored vs recomputed dS, shape {shape}", flush=True)
    _, (q, k, v, g) = _fast_inputs(shape, seed=900)
    o, lse = D.fwd(q, k, v, ctx=ctx)
    out = {}
    for ds in ("recompute", "stored"):
        with _DsLimit(ctx, ctx.ds_limit if ds == "stored" else 0):
            out[ds] = [x.cpu().numpy() for x in D.bwd(g, q, k, v, o, lse, ctx=ctx)]
    (rq, rk, rv), (sq, sk, sv) = out["recompute"], out["stored"]
    assert np.array_equal(rk, sk) and np.array_equal(rv, sv)
    e = rel_err(sq.reshape(-1), rq.reshape(-1))
    print(f"  dq rel diff {e:.3e}, bitwise equal {np.array_equal(sq, rq)}", flush=True)
    assert e <= 1e-5


@pytest.mark.parametrize("ds", ["stored", "recompute"])
@pytest.mark.parametrize("shape", [(1, 1000, 8, 2, 128), (2, 300, 4, 4, 128), (1, 2048, 32, 8, 128),
                                   (3, 129, 6, 3, 128), (1, 64, 4, 1, 128), (1, 1, 4, 1, 128)],
                         ids=lambda s: "x".join(map(str, s)))
def test_dkdv_one_wave_per_simd_matches_wave_specialised(cf, shape, ds, monkeypatch):
    """The head_dim-128 dK/dV kernel with one wave per SIMD (64 keys per
    wave) sums every element's products in the order of the two-waves-per-
    SIMD kernel (CFATTN_DKDV_KERNEL=ws): dK, dV and dQ (from the stored dS,
    or recomputed) must be bitwise equal."""
    import torch
    from cpuforge_amd import device as D
    mod, ctx = cf
    print(f"dK/dV kernels, shape {shape}, dS {ds}", flush=True)
    _, (q, k, v, g) = _fast_inputs(shape, seed=1900)
    o, lse = D.fwd(q, k, v, ctx=ctx)
    out = {}
    with _DsLimit(ctx, ctx.ds_limit if ds == "stored" else 0):
        for kern in ("ws", "k64"):
            if kern == "ws":
                monkeypatch.setenv("CFATTN_DKDV_KERNEL", "ws")
            else:
                monkeypatch.delenv("CFATTN_DKDV_KERNEL", raising=False)
            out[kern] = [x.cpu().numpy() for x in D.bwd(g, q, k, v, o, lse, ctx=ctx)]
    torch.cuda.synchronize()
    for name, a, b in zip(("dq", "dk", "dv"), out["k64"], out["ws"]):
        assert np.array_equal(a, b), f"{shape} {ds} {name}: max diff {np.abs(a - b).max()}"
