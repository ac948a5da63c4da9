"""Pins the layer-op oracle (oracle/oracle_layer.c) before it is trusted as the
checker of include/cfops.h.  Each test restates one of the reference's own
tests (cited) or checks what the mathematics fixes: f64 closed forms, central
finite differences of an independent f64 forward, hand-computed optimizer
steps, identities.  CPU only."""
import numpy as np
import pytest

from oracle import oracle as O


def numeric_grad(f, x, eps=1e-6):  # core/src/gradcheck.rs:7-23
    x = np.array(x, dtype=np.float64, copy=True)
    g = np.zeros_like(x)
    for i in range(x.size):
        o = x[i]
        x[i] = o + eps
        hi = f(x)
        x[i] = o - eps
        lo = f(x)
        x[i] = o
        g[i] = (hi - lo) / (2 * eps)
    return g


def close(a, want, tol):  # gradcheck.rs:31-53
    return O.grad_close_metric(a, want)[0] <= tol


# --------------------------------------------------------------- SwiGLU
def _swiglu_data(n, seed):  # swiglu.rs:44-50
    r = O.Rng(seed)
    g = np.array([r.normal() * 2.0 for _ in range(n)], np.float32)
    u = np.array([r.normal() for _ in range(n)], np.float32)
    d = np.array([r.normal() for _ in range(n)], np.float32)
    return g, u, d


def _swiglu_ref(g, u):  # swiglu.rs:40-42
    return g / (1.0 + np.exp(-g)) * u


def test_swiglu_forward_matches_f64_reference():  # swiglu.rs:52-58
    g, u, _ = _swiglu_data(100, 1)
    h = np.zeros(100, np.float32)
    O.silu_mul_forward(g, u, h)
    assert close(h, _swiglu_ref(g.astype(np.float64), u.astype(np.float64)), 1e-5)


def test_swiglu_backward_matches_finite_differences():  # swiglu.rs:60-71
    n = 40
    g, u, dh = _swiglu_data(n, 2)
    dg, du = np.zeros(n, np.float32), np.zeros(n, np.float32)
    O.silu_mul_backward(dh, g, u, dg, du)
    g64, u64, d64 = g.astype(np.float64), u.astype(np.float64), dh.astype(np.float64)
    ng = numeric_grad(lambda gs: float(_swiglu_ref(gs, u64) @ d64), g64)
    nu = numeric_grad(lambda us: float(_swiglu_ref(g64, us) @ d64), u64)
    assert close(dg, ng, 5e-4) and close(du, nu, 5e-4)


def test_swiglu_backward_accumulates():
    g, u, dh = _swiglu_data(33, 3)
    dg, du = np.full(33, 0.25, np.float32), np.full(33, -1.0, np.float32)
    O.silu_mul_backward(dh, g, u, dg, du)
    dg1, du1 = np.zeros(33, np.float32), np.zeros(33, np.float32)
    O.silu_mul_backward(dh, g, u, dg1, du1)
    np.testing.assert_allclose(dg, dg1 + 0.25, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(du, du1 - 1.0, rtol=1e-6, atol=1e-6)


# -------------------------------------------------------- cross-entropy
IG = O.IGNORE_INDEX


def _logits(rows, vocab, seed):  # loss.rs:77-80
    r = O.Rng(seed)
    return np.array([r.normal() * 3.0 for _ in range(rows * vocab)], np.float32)


def _ref_loss(l, t, rows, vocab):  # loss.rs:63-75
    tot, n = 0.0, 0
    for r in range(rows):
        if t[r] == IG:
            continue
        lr = l[r * vocab:(r + 1) * vocab]
        m = lr.max()
        tot += np.log(np.exp(lr - m).sum()) + m - lr[t[r]]
        n += 1
    return tot / n


def test_uniform_logits_give_ln_vocab():  # loss.rs:82-90
    rows, vocab = 4, 50
    d = np.zeros(rows * vocab, np.float32)
    loss = O.cross_entropy_fwd_bwd(np.full(rows * vocab, 0.7, np.float32), np.array([3, 10, 0, 49]), d, rows, vocab)
    assert abs(loss - np.log(vocab)) < 1e-5


def test_loss_matches_f64_reference():  # loss.rs:92-101
    rows, vocab = 6, 23
    l = _logits(rows, vocab, 1)
    t = np.array([0, 5, IG, 22, 7, 7])
    d = np.zeros_like(l)
    loss = O.cross_entropy_fwd_bwd(l, t, d, rows, vocab)
    assert abs(loss - _ref_loss(l.astype(np.float64), t, rows, vocab)) < 1e-5


def test_ce_gradient_matches_finite_differences():  # loss.rs:103-114
    rows, vocab = 5, 11
    l = _logits(rows, vocab, 2)
    t = np.array([1, IG, 4, 10, 0])
    d = np.zeros_like(l)
    O.cross_entropy_fwd_bwd(l, t, d, rows, vocab)
    n = numeric_grad(lambda ls: _ref_loss(ls, t, rows, vocab), l.astype(np.float64))
    assert close(d, n, 5e-4)
    assert np.all(d[vocab:2 * vocab] == 0.0)


def test_ce_gradient_rows_sum_to_zero():  # loss.rs:116-127
    rows, vocab = 3, 17
    l = _logits(rows, vocab, 3)
    d = np.zeros_like(l)
    O.cross_entropy_fwd_bwd(l, np.array([2, 3, 4]), d, rows, vocab)
    for r in range(rows):
        assert abs(float(d[r * vocab:(r + 1) * vocab].sum())) < 1e-6


def test_ce_stable_for_huge_logits():  # loss.rs:129-141
    rows, vocab = 2, 8
    l = _logits(rows, vocab, 4) + np.float32(1000.0)
    d = np.zeros_like(l)
    loss = O.cross_entropy_fwd_bwd(l, np.array([1, 2]), d, rows, vocab)
    assert np.isfinite(loss) and np.all(np.isfinite(d))


def test_ce_all_ignored_is_zero():  # loss.rs:143-150
    d = np.ones(10, np.float32)
    loss = O.cross_entropy_fwd_bwd(_logits(2, 5, 5), np.array([IG, IG]), d, 2, 5)
    assert loss == 0.0 and np.all(d == 0.0)


def test_ce_target_out_of_range_panics():  # loss.rs:35
    d = np.zeros(10, np.float32)
    with pytest.raises(ValueError, match="target 5 out of range for vocab 5"):
        O.cross_entropy_fwd_bwd(_logits(2, 5, 6), np.array([1, 5]), d, 2, 5)


# ---------------------------------------------------------------- AdamW
def test_powi_matches_repeated_multiplication_and_f64_pow():
    for a in (0.9, 0.999, 0.5, 1.5):
        a32 = np.float32(a)
        for t in range(0, 9):
            want = np.float32(1.0)
            for _ in range(t):
                want = np.float32(want * a32)
            # square-and-multiply equals repeated multiplication where the
            # partial products are exact, and is always within a few ulp
            assert abs(O.powi_f32(a, t) - float(want)) <= 4 * np.spacing(np.float32(want))
        for t in (10, 100, 1000, 12345) if a < 1 else (10, 100):
            want = float(a32) ** t
            # each squaring at most doubles the relative error: ~t ulp in all
            assert abs(O.powi_f32(a, t) - want) <= 2.0 * t * 2.0 ** -24 * want + 1e-30
    assert O.powi_f32(2.0, -3) == 0.125
    assert O.powi_f32(3.0, 5) == 243.0


def test_adamw_first_step_moves_by_lr_in_the_gradient_direction():  # optim.rs:80-89
    p = np.array([1.0, 1.0], np.float32)
    m, v = np.zeros(2, np.float32), np.zeros(2, np.float32)
    O.adamw_update(p, np.array([0.5, -3.0], np.float32), m, v, 1, 0.1, 0.9, 0.999, 1e-8, 0.0)
    assert abs(p[0] - 0.9) < 1e-5 and abs(p[1] - 1.1) < 1e-5


def test_adamw_matches_a_hand_computed_second_step():  # optim.rs:91-107
    b1, b2, eps, lr = 0.9, 0.999, 1e-8, 0.01
    p = np.array([2.0], np.float32)
    m, v = np.zeros(1, np.float32), np.zeros(1, np.float32)
    O.adamw_update(p, np.array([1.0], np.float32), m, v, 1, lr, b1, b2, eps, 0.0)
    O.adamw_update(p, np.array([0.5], np.float32), m, v, 2, lr, b1, b2, eps, 0.0)
    p64, m64, v64 = 2.0, 0.0, 0.0
    for t, g in ((1, 1.0), (2, 0.5)):
        m64 = 0.9 * m64 + 0.1 * g
        v64 = 0.999 * v64 + 0.001 * g * g
        mh, vh = m64 / (1 - 0.9 ** t), v64 / (1 - 0.999 ** t)
        p64 -= 0.01 * mh / (np.sqrt(vh) + 1e-8)
    assert abs(float(p[0]) - p64) < 1e-6


def test_adamw_weight_decay_is_decoupled_from_the_gradient():  # optim.rs:109-115
    p = np.array([10.0], np.float32)
    m, v = np.zeros(1, np.float32), np.zeros(1, np.float32)
    O.adamw_update(p, np.array([0.0], np.float32), m, v, 1, 0.1, 0.9, 0.999, 1e-8, 0.5)
    assert abs(p[0] - 9.5) < 1e-5


def test_adamw_many_steps_track_an_f64_restatement():
    r = np.random.default_rng(0)
    n = 257
    p = r.standard_normal(n).astype(np.float32)
    m, v = np.zeros(n, np.float32), np.zeros(n, np.float32)
    p64, m64, v64 = p.astype(np.float64), np.zeros(n), np.zeros(n)
    for t in range(1, 21):
        g = r.standard_normal(n).astype(np.float32)
        O.adamw_update(p, g, m, v, t, 1e-3, 0.9, 0.95, 1e-8, 0.1)
        m64 = 0.9 * m64 + 0.1 * g
        v64 = 0.95 * v64 + 0.05 * g.astype(np.float64) ** 2
        p64 -= 1e-3 * (m64 / (1 - 0.9 ** t) / (np.sqrt(v64 / (1 - 0.95 ** t)) + 1e-8) + 0.1 * p64)
    np.testing.assert_allclose(p, p64, rtol=0, atol=2e-6)


# --------------------------------------------------------------- Linear
def _lin_setup(t, inn, out, r, seed):
    g = np.random.default_rng(seed)
    f = lambda *s: g.standard_normal(s).astype(np.float32)  # noqa: E731
    return f(t, inn), f(out, inn), f(r, inn), f(out, r), f(t, out)


@pytest.mark.parametrize("lora", [False, True])
def test_linear_forward_matches_closed_form(lora):  # linear.rs:1-3
    t, inn, out, r, scale = 7, 12, 9, 3, 2.5
    x, w, a, b, _ = _lin_setup(t, inn, out, r, 1)
    y = np.full((t, out), np.nan, np.float32)
    xs = np.full((t, r), np.nan, np.float32)
    O.linear_forward(x, w, a if lora else None, b if lora else None, scale, t, inn, out, r, y, xs if lora else None)
    x64 = x.astype(np.float64)
    want = x64 @ w.T.astype(np.float64)
    if lora:
        xs_want = scale * (x64 @ a.T.astype(np.float64))
        want = want + xs_want @ b.T.astype(np.float64)
        np.testing.assert_allclose(xs, xs_want, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(y, want, rtol=1e-5, atol=1e-5)


def test_linear_backward_matches_finite_differences():
    t, inn, out, r, scale = 5, 6, 4, 2, 1.5
    x, w, a, b, dy = _lin_setup(t, inn, out, r, 2)
    xs = np.zeros((t, r), np.float32)
    y = np.zeros((t, out), np.float32)
    O.linear_forward(x, w, a, b, scale, t, inn, out, r, y, xs)
    dx, gw = np.zeros_like(x), np.zeros_like(w)
    ga, gb = np.zeros_like(a), np.zeros_like(b)
    O.linear_backward(x, xs, dy, w, a, b, scale, t, inn, out, r, dx, gw, ga, gb)
    d64 = dy.astype(np.float64)

    def loss(x_=x, w_=w, a_=a, b_=b):
        return float(((x_ @ w_.T + scale * (x_ @ a_.T) @ b_.T) * d64).sum())
    f64 = lambda z: z.astype(np.float64)  # noqa: E731
    for got, arr, key in ((dx, x, "x_"), (gw, w, "w_"), (ga, a, "a_"), (gb, b, "b_")):
        n = numeric_grad(lambda v: loss(**{key: v.reshape(arr.shape)}), f64(arr).reshape(-1))
        assert close(got.reshape(-1), n, 1e-4), key


def test_linear_backward_accumulates_and_skips_frozen():
    t, inn, out, r, scale = 4, 5, 3, 2, 2.0
    x, w, a, b, dy = _lin_setup(t, inn, out, r, 3)
    xs, y = np.zeros((t, r), np.float32), np.zeros((t, out), np.float32)
    O.linear_forward(x, w, a, b, scale, t, inn, out, r, y, xs)
    dx1 = np.zeros_like(x)
    O.linear_backward(x, xs, dy, w, a, b, scale, t, inn, out, r, dx1)  # base and adapter frozen
    dx2 = np.ones_like(x)
    ga = np.zeros_like(a)
    O.linear_backward(x, xs, dy, w, a, b, scale, t, inn, out, r, dx2, None, ga, None)
    np.testing.assert_allclose(dx2, dx1 + 1.0, rtol=1e-6, atol=1e-6)
    assert np.any(ga != 0)
