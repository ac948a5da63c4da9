"""GPU parity of the layer ops (include/cfops.h) against the oracle's
restatement of the reference (oracle/oracle_layer.c, cforge_oracle.c) on the
same seeded inputs.

Bars: bitwise where the kernel keeps the reference's order of f32 operations
(RMSNorm forward, AdamW); otherwise the reference's own test tolerance,
`|a - r| / (1 + |r|)` (core/src/gradcheck.rs:31-48): 1e-5 for RMSNorm's
backward, SwiGLU and cross-entropy, whose row sums run in a parallel order,
and matmul.rs's 1e-4 (core/src/matmul.rs:200-282) for the hipBLASLt GEMMs."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"


def ops():
    from cpuforge_amd import ops as P
    return P


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def metric(a, r):
    return O.grad_close_metric(np.asarray(a, np.float32).reshape(-1), np.asarray(r, np.float64).reshape(-1))[0]


def rnd(shape, seed, std=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * std).astype(np.float32)


# -------------------------------------------------------------- RMSNorm
@pytest.mark.parametrize("rows,dim", [(4096, 576), (33, 577), (7, 20000), (1, 1), (300, 64)])
def test_rmsnorm_forward_is_bitwise_the_reference(rows, dim):
    print(f"rmsnorm fwd rows={rows} dim={dim}", flush=True)
    x, w = rnd((rows, dim), 1), (1 + 0.1 * rnd(dim, 2)).astype(np.float32)
    y, rstd = np.zeros_like(x), np.zeros(rows, np.float32)
    O.rmsnorm_forward(x, w, y, rstd, rows, dim, 1e-5)
    gy, gr = torch.empty(rows, dim, device=DEV), torch.empty(rows, device=DEV)
    ops().rmsnorm_forward(dev(x), dev(w), gy, gr, rows, dim, 1e-5)
    assert np.array_equal(host(gy), y) and np.array_equal(host(gr), rstd)


@pytest.mark.parametrize("rows,dim", [(4096, 576), (33, 577), (7, 20000), (300, 64)])
def test_rmsnorm_backward_matches_oracle(rows, dim):
    print(f"rmsnorm bwd rows={rows} dim={dim}", flush=True)
    x, w, dy = rnd((rows, dim), 3), (1 + 0.1 * rnd(dim, 4)).astype(np.float32), rnd((rows, dim), 5)
    y, rstd = np.zeros_like(x), np.zeros(rows, np.float32)
    O.rmsnorm_forward(x, w, y, rstd, rows, dim, 1e-5)
    dx0, dw0 = rnd((rows, dim), 6, 0.1), rnd(dim, 7, 0.1)
    dx, dw = dx0.copy(), dw0.copy()
    O.rmsnorm_backward(dy, x, w, rstd, dx, dw, rows, dim)
    gdx, gdw = dev(dx0), dev(dw0)
    ops().rmsnorm_backward(dev(dy), dev(x), dev(w), dev(rstd), gdx, gdw, rows, dim)
    assert metric(host(gdx), dx) <= 1e-5
    # dw sums over every row: the oracle's sequential f32 sum drifts by up to
    # ~rows ulp, so the kernel's is held to the f64 sum of the same f32 terms,
    # at least as closely as the reference algorithm's own sum.
    x64, r64 = x.astype(np.float64), rstd.astype(np.float64)[:, None]
    dw64 = dw0.astype(np.float64) + (dy.astype(np.float64) * (x64 * r64)).sum(0)
    assert metric(host(gdw), dw64) <= max(1e-5, metric(dw, dw64))
    assert metric(host(gdw), dw) <= 1e-4
    # a frozen gain: dx alone, accumulated again
    ops().rmsnorm_backward(dev(dy), dev(x), dev(w), dev(rstd), gdx, None, rows, dim)
    assert metric(host(gdx), dx + (dx - dx0)) <= 1e-5


# --------------------------------------------------------------- SwiGLU
@pytest.mark.parametrize("n", [4096 * 1536, 1001, 4])
def test_silu_mul_matches_oracle(n):
    print(f"silu_mul n={n}", flush=True)
    g, u, dh = rnd(n, 8, 2.0), rnd(n, 9), rnd(n, 10)
    h = np.zeros(n, np.float32)
    O.silu_mul_forward(g, u, h)
    gh = torch.empty(n, device=DEV)
    ops().silu_mul_forward(dev(g), dev(u), gh)
    assert metric(host(gh), h) <= 1e-6
    dg0, du0 = rnd(n, 11, 0.1), rnd(n, 12, 0.1)
    dg, du = dg0.copy(), du0.copy()
    O.silu_mul_backward(dh, g, u, dg, du)
    gdg, gdu = dev(dg0), dev(du0)
    ops().silu_mul_backward(dev(dh), dev(g), dev(u), gdg, gdu)
    assert metric(host(gdg), dg) <= 1e-6 and metric(host(gdu), du) <= 1e-6


# -------------------------------------------------------- cross-entropy
def _targets(rows, vocab, seed, ignore_every=0):
    t = np.random.default_rng(seed).integers(0, vocab, rows).astype(np.int64)
    if ignore_every:
        t[::ignore_every] = O.IGNORE_INDEX
    return t


@pytest.mark.parametrize("rows,vocab", [(64, 49152), (37, 50), (9, 50001), (3, 300000), (2, 8)])
def test_cross_entropy_matches_oracle(rows, vocab):
    print(f"cross_entropy rows={rows} vocab={vocab}", flush=True)
    l = rnd((rows, vocab), 13, 3.0)
    t = _targets(rows, vocab, 14, ignore_every=5)
    d = np.zeros_like(l)
    want = O.cross_entropy_fwd_bwd(l, t, d, rows, vocab)
    gd = torch.full((rows, vocab), float("nan"), device=DEV)
    loss = ops().cross_entropy_fwd_bwd(dev(l), dev(t), gd, rows, vocab)
    # the loss against the f64 loss of the same logits (loss.rs:92-101) and
    # the oracle, whose sequential exp sum over the vocabulary drifts by ~1e-5
    keep = t != O.IGNORE_INDEX
    l64 = l[keep].astype(np.float64)
    m64 = l64.max(1, keepdims=True)
    lse = np.log(np.exp(l64 - m64).sum(1)) + m64[:, 0]
    want64 = float((lse - l64[np.arange(l64.shape[0]), t[keep]]).mean())
    assert abs(loss - want64) <= 1e-5 * (1 + abs(want64))
    assert abs(loss - want) <= 1e-4 * (1 + abs(want))
    # dlogits likewise: at least as close to the f64 gradient as the oracle's
    d64 = np.zeros((rows, vocab))
    p64 = np.exp(l64 - m64)
    p64 /= p64.sum(1, keepdims=True)
    p64[np.arange(l64.shape[0]), t[keep]] -= 1.0
    d64[keep] = p64 / keep.sum()
    assert metric(host(gd), d64) <= max(1e-5, metric(d, d64))
    assert metric(host(gd), d) <= 1e-4
    assert np.all(host(gd)[::5] == 0.0)  # ignored rows
    # in place: dlogits may be the logits buffer
    gl = dev(l)
    loss2 = ops().cross_entropy_fwd_bwd(gl, dev(t), gl, rows, vocab)
    assert loss2 == loss and np.array_equal(host(gl), host(gd))


def test_cross_entropy_edge_cases():
    P = ops()
    l = rnd((2, 5), 15)
    g = torch.ones(2, 5, device=DEV)
    assert P.cross_entropy_fwd_bwd(dev(l), dev(np.array([-100, -100])), g, 2, 5) == 0.0
    assert torch.all(g == 0)
    assert abs(P.cross_entropy_fwd_bwd(torch.full((4, 50), 0.7, device=DEV), dev(np.array([3, 10, 0, 49])),
                                       torch.empty(4, 50, device=DEV), 4, 50) - np.log(50)) < 1e-5
    big = dev(l + np.float32(1000.0))
    assert np.isfinite(P.cross_entropy_fwd_bwd(big, dev(np.array([1, 2])), torch.empty(2, 5, device=DEV), 2, 5))
    from cpuforge_amd import CfattnError
    with pytest.raises(CfattnError, match="target 5 out of range for vocab 5"):
        P.cross_entropy_fwd_bwd(dev(l), dev(np.array([1, 5])), torch.empty(2, 5, device=DEV), 2, 5)


@pytest.mark.parametrize("chunk_bytes", [512 << 20, 3 * 1000 * 4])
def test_lm_head_ce_matches_oracle(chunk_bytes):
    print(f"lm_head_ce chunk_bytes={chunk_bytes}", flush=True)
    P = ops()
    t, d, vocab = 70, 48, 1000
    hn, head = rnd((t, d), 16), rnd((vocab, d), 17, 0.2)
    tg = _targets(t, vocab, 18, ignore_every=7)
    logits = np.zeros((t, vocab), np.float32)
    O.gemm_strided(hn, d, 1, head, 1, d, logits, vocab, 1, t, d, vocab, 0)
    dl = np.zeros_like(logits)
    want = O.cross_entropy_fwd_bwd(logits, tg, dl, t, vocab)
    dhn = dl.astype(np.float64) @ head.astype(np.float64)
    dhead0 = rnd((vocab, d), 19, 0.1)
    dhead = dhead0 + dl.T.astype(np.float64) @ hn.astype(np.float64)
    P.set_head_chunk_limit(chunk_bytes)
    try:
        g_dhn, g_dhead = torch.full((t, d), float("nan"), device=DEV), dev(dhead0)
        loss = P.lm_head_ce(dev(hn), dev(head), dev(tg), t, d, vocab, g_dhn, g_dhead)
    finally:
        P.set_head_chunk_limit(512 << 20)
    assert abs(loss - want) <= 1e-5 * (1 + abs(want))
    assert metric(host(g_dhn), dhn) <= 1e-5
    assert metric(host(g_dhead), dhead) <= 1e-5


# ------------------------------------------------------- matmul, Linear
@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (3, 5, 7), (17, 33, 9), (130, 70, 90), (512, 300, 400)])
def test_matmul_matches_f64(m, k, n):  # matmul.rs:200-282 SHAPES and tolerance
    P = ops()
    a, b = rnd((m, k), 20), rnd((k, n), 21)
    want = a.astype(np.float64) @ b.astype(np.float64)
    c0 = rnd((m, n), 22)
    for fn, A, B in ((P.matmul_nn, a, b), (P.matmul_nt, a, np.ascontiguousarray(b.T)),
                     (P.matmul_tn, np.ascontiguousarray(a.T), b)):
        c = torch.full((m, n), float("nan"), device=DEV)
        fn(dev(A), dev(B), c, m, k, n, False)
        assert np.max(np.abs(host(c) - want) / (1 + np.abs(want))) <= 1e-4
        c = dev(c0)
        fn(dev(A), dev(B), c, m, k, n, True)
        assert np.max(np.abs(host(c) - (want + c0)) / (1 + np.abs(want + c0))) <= 1e-4


def test_matmul_is_repeatable():
    """The same GEMM twice gives the same bits (no split-K atomics), at the
    SmolLM-135M LoRA-gradient shape (m=16, k=4096, n=576) and the LM head."""
    P = ops()
    for m, k, n, fn in ((16, 4096, 576, P.matmul_tn), (4096, 576, 49152 // 8, P.matmul_nt)):
        a = dev(rnd((k, m) if fn is P.matmul_tn else (m, k), 50))
        b = dev(rnd((k, n) if fn is P.matmul_tn else (n, k), 51))
        c1, c2 = torch.zeros(m, n, device=DEV), torch.zeros(m, n, device=DEV)
        fn(a, b, c1, m, k, n, True)
        fn(a, b, c2, m, k, n, True)
        assert torch.equal(c1, c2)


def test_matmul_k0_zeroes_or_keeps():  # matmul.rs:58-67
    P = ops()
    c = torch.full((3, 4), float("nan"), device=DEV)
    P.matmul_nn(torch.empty(0, device=DEV), torch.empty(0, device=DEV), c, 3, 0, 4, False)
    assert torch.all(c == 0)
    c = torch.ones(3, 4, device=DEV)
    P.matmul_nn(torch.empty(0, device=DEV), torch.empty(0, device=DEV), c, 3, 0, 4, True)
    assert torch.all(c == 1)


LINEAR_CASES = [  # (name, lora, rank, t, frozen adapters): SmolLM-135M q projection shapes
    ("plain", False, 16, 512, False),
    ("lora_r16", True, 16, 512, False),  # fused adapter kernels
    ("lora_r8_ragged", True, 8, 509, False),
    ("lora_r4", True, 4, 256, False),
    ("lora_r3_gemm", True, 3, 512, False),  # a rank the fused kernels do not take: the GEMM path
    ("lora_r16_frozen", True, 16, 300, True),  # no adapter gradients, dx only
]


@pytest.mark.parametrize("case", LINEAR_CASES, ids=[c[0] for c in LINEAR_CASES])
def test_linear_matches_oracle(case):
    name, lora, r, t, frozen = case
    print(f"linear {name}", flush=True)
    P = ops()
    inn, out, scale = 576, 576, 2.0
    x, w, a, b, dy = rnd((t, inn), 23), rnd((out, inn), 24, 0.02), rnd((r, inn), 25, 0.04), rnd((out, r), 26, 0.1), \
        rnd((t, out), 27)
    A, B = (a, b) if lora else (None, None)
    y, xs = np.zeros((t, out), np.float32), np.zeros((t, r), np.float32)
    O.linear_forward(x, w, A, B, scale, t, inn, out, r, y, xs if lora else None)
    gy, gxs = torch.full((t, out), float("nan"), device=DEV), torch.full((t, r), float("nan"), device=DEV)
    gA = dev(a) if lora else None
    gB = dev(b) if lora else None
    P.linear_forward(dev(x), dev(w), t, inn, out, gy, gA, gB, scale, gxs if lora else None)
    assert metric(host(gy), y) <= 1e-4
    if lora:
        assert metric(host(gxs), xs) <= 1e-4
    dx, gw, ga, gb = (rnd(s, 28 + i, 0.1) for i, s in enumerate(((t, inn), (out, inn), (r, inn), (out, r))))
    wdx, wgw, wga, wgb = dx.copy(), gw.copy(), ga.copy(), gb.copy()
    grads = lora and not frozen
    O.linear_backward(x, xs if lora else None, dy, w, A, B, scale, t, inn, out, r, wdx, wgw,
                      wga if grads else None, wgb if grads else None)
    g = [dev(dx), dev(gw), dev(ga), dev(gb)]
    P.linear_backward(dev(x), dev(xs) if lora else None, dev(dy), dev(w), t, inn, out, g[0], g[1],
                      g[2] if grads else None, g[3] if grads else None, gA, gB, scale)
    # f64 gradients of the same f32 inputs (linear.rs:75-90)
    f = lambda z: z.astype(np.float64)  # noqa: E731
    r_dx = f(dx) + f(dy) @ f(w)
    r_gw = f(gw) + f(dy).T @ f(x)
    if lora:
        dxa = scale * (f(dy) @ f(b))
        r_dx = r_dx + dxa @ f(a)
        r_ga = f(ga) + dxa.T @ f(x)
        r_gb = f(gb) + f(dy).T @ f(xs)
    got = [host(t_) for t_ in g]
    errs = {"dx": (metric(got[0], r_dx), metric(wdx, r_dx)), "gw": (metric(got[1], r_gw), metric(wgw, r_gw))}
    if grads:
        errs["ga"] = (metric(got[2], r_ga), metric(wga, r_ga))
        errs["gb"] = (metric(got[3], r_gb), metric(wgb, r_gb))
    elif lora:  # frozen adapters: their gradient buffers are untouched
        assert np.array_equal(got[2], ga) and np.array_equal(got[3], gb)
    print("gpu / oracle metric vs f64:", {k: f"{a_:.2e} / {b_:.2e}" for k, (a_, b_) in errs.items()}, flush=True)
    for k, (e_gpu, e_orc) in errs.items():
        assert e_gpu <= max(1e-4, 2 * e_orc), k


def test_lora_linear_is_bitwise_repeatable():
    """The fused adapter kernels sum in a fixed order: the same inputs give the
    same bits (the checkpoint-recompute contract of the layer)."""
    P = ops()
    t, inn, out, r = 700, 1536, 576, 16
    x, w, a, b, dy = (dev(rnd(s, 60 + i, sd)) for i, (s, sd) in
                      enumerate((((t, inn), 1.0), ((out, inn), 0.02), ((r, inn), 0.04), ((out, r), 0.1),
                                 ((t, out), 1.0))))
    outs = []
    for _ in range(2):
        y, xs = torch.empty(t, out, device=DEV), torch.empty(t, r, device=DEV)
        P.linear_forward(x, w, t, inn, out, y, a, b, 2.0, xs)
        dx, ga, gb = torch.zeros(t, inn, device=DEV), torch.zeros(r, inn, device=DEV), torch.zeros(out, r, device=DEV)
        P.linear_backward(x, xs, dy, w, t, inn, out, dx, None, ga, gb, a, b, 2.0)
        outs.append([host(z) for z in (y, xs, dx, ga, gb)])
    for u, v in zip(*outs):
        assert np.array_equal(u, v)


# ---------------------------------------------------------------- AdamW
@pytest.mark.parametrize("n", [1_000_003, 4096, 3])
def test_adamw_is_bitwise_the_reference(n):
    print(f"adamw n={n}", flush=True)
    p, m, v = rnd(n, 40), np.zeros(n, np.float32), np.zeros(n, np.float32)
    gp, gm, gv = dev(p), dev(m), dev(v)
    for t in range(1, 4):
        g = rnd(n, 40 + t)
        O.adamw_update(p, g, m, v, t, 1e-3, 0.9, 0.95, 1e-8, 0.1)
        ops().adamw_update(gp, dev(g), gm, gv, t, 1e-3, 0.9, 0.95, 1e-8, 0.1)
    assert np.array_equal(host(gp), p) and np.array_equal(host(gm), m) and np.array_equal(host(gv), v)
