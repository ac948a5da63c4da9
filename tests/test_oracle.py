"""Pins the C oracle (oracle/cforge_oracle.c) before it is trusted as the
checker of the HIP kernels.  CPU only.

Each oracle function is checked against something that does not share its
code: golden vectors written by tests/golden/make_golden.py (pure-Python RNG,
torch float64 autograd), closed forms, finite differences, and the
invariants the reference's own tests assert.  Test names follow the
reference tests they restate.
"""
import json
import math
import os
import struct

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.cases import CASES, case

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def bits(x: float) -> int:
    return struct.unpack("I", struct.pack("f", x))[0]


# ------------------------------------------------------------------ Rng
def test_rng_matches_golden_stream():
    """u64 stream, uniform and Box-Muller normal vs the pure-Python restatement."""
    g = json.load(open(os.path.join(GOLDEN, "rng.json")))
    for seed, d in g.items():
        r = O.Rng(int(seed))
        assert [str(r.next_u64()) for _ in range(8)] == d["u64"], seed
        r = O.Rng(int(seed))
        assert [bits(r.uniform()) for _ in range(8)] == d["uniform_bits"], seed
        r = O.Rng(int(seed))
        assert [bits(r.normal()) for _ in range(8)] == d["normal_bits"], seed


def test_rng_deterministic():  # rng.rs:51-57
    a, b = O.Rng(7), O.Rng(7)
    assert [a.next_u64() for _ in range(100)] == [b.next_u64() for _ in range(100)]


def test_rng_normal_has_sane_moments():  # rng.rs:59-70
    xs = O.rand(20000, 1)
    assert abs(xs.mean()) < 0.05
    assert abs(xs.var() - 1.0) < 0.08


def test_rng_zero_seed_is_not_stuck():
    # seed ^ golden | 1 can never be zero (rng.rs:11-13)
    r = O.Rng(0x9E3779B97F4A7C15)
    assert r.next_u64() != 0


# ----------------------------------------------------------------- GEMM
SHAPES = [(1, 1, 1), (3, 5, 7), (17, 33, 9), (64, 128, 257), (130, 7, 300)]


@pytest.mark.parametrize("m,k,n", SHAPES)
def test_gemm_layouts_match_numpy(m, k, n):
    """nn / nt / tn strided views vs numpy float64 (matmul.rs:200-282, tol 1e-4*(1+|y|))."""
    rng = np.random.default_rng(m * 1000 + n)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    want = a.astype(np.float64) @ b.astype(np.float64)
    c = np.zeros(m * n, np.float32)
    O.gemm_strided(a.reshape(-1), k, 1, b.reshape(-1), n, 1, c, n, 1, m, k, n, False)
    assert np.all(np.abs(c.reshape(m, n) - want) <= 1e-4 * (1 + np.abs(want)))
    bt = np.ascontiguousarray(b.T)  # B stored [n, k]
    c2 = np.zeros(m * n, np.float32)
    O.gemm_strided(a.reshape(-1), k, 1, bt.reshape(-1), 1, k, c2, n, 1, m, k, n, False)
    assert np.all(np.abs(c2.reshape(m, n) - want) <= 1e-4 * (1 + np.abs(want)))
    at = np.ascontiguousarray(a.T)  # A stored [k, m]
    c3 = np.zeros(n * m, np.float32)  # column-major C
    O.gemm_strided(at.reshape(-1), 1, m, b.reshape(-1), n, 1, c3, 1, m, m, k, n, False)
    assert np.all(np.abs(c3.reshape(n, m).T - want) <= 1e-4 * (1 + np.abs(want)))


def test_gemm_overwrite_ignores_nan_accumulate_adds_and_k0():
    a = np.ones(6, np.float32)
    b = np.ones(6, np.float32)
    c = np.full(4, np.nan, np.float32)
    O.gemm_strided(a, 3, 1, b, 2, 1, c, 2, 1, 2, 3, 2, False)  # overwrite: NaN ignored
    assert np.all(c == 3.0)
    O.gemm_strided(a, 3, 1, b, 2, 1, c, 2, 1, 2, 3, 2, True)  # accumulate
    assert np.all(c == 6.0)
    O.gemm_strided(a, 3, 1, b, 2, 1, c, 2, 1, 2, 0, 2, True)  # k == 0, acc: untouched
    assert np.all(c == 6.0)
    O.gemm_strided(a, 3, 1, b, 2, 1, c, 2, 1, 2, 0, 2, False)  # k == 0, overwrite: zeroed
    assert np.all(c == 0.0)


# ------------------------------------------------------------ attention
def _torch_attn(q, k, v, seq, nh, nkv, hd):
    group = nh // nkv
    qt = q.view(seq, nh, hd).transpose(0, 1)
    kt = k.view(seq, nkv, hd).transpose(0, 1).repeat_interleave(group, 0)
    vt = v.view(seq, nkv, hd).transpose(0, 1).repeat_interleave(group, 0)
    o = torch.nn.functional.scaled_dot_product_attention(qt[None], kt[None], vt[None], is_causal=True)[0]
    return o.transpose(0, 1).reshape(-1)


def test_attention_cases_match_golden():
    """Oracle f32 forward/backward and f64 reference vs torch float64 golden vectors."""
    gz = np.load(os.path.join(GOLDEN, "attn_cases.npz"))
    for i, (seq, nh, nkv, hd, qb) in enumerate(CASES):
        p = f"c{i}_fwd_"
        q, k, v = case(seq, nh, nkv, hd, 10 + i)
        # the oracle's inputs are bit-identical to the fixture's (same RNG)
        assert np.array_equal(q, gz[p + "q"]) and np.array_equal(v, gz[p + "v"])
        o = np.zeros_like(q)
        lse = np.zeros(nh * seq, np.float32)
        O.attention_forward_blocked(q, k, v, o, lse, seq, nh, nkv, hd, qb)
        assert O.grad_close_metric(o, gz[p + "o"])[0] <= 1e-4
        assert O.grad_close_metric(lse, gz[p + "lse"])[0] <= 1e-4
        o64, l64 = O.attn_ref_f64(q, k, v, seq, nh, nkv, hd)
        assert np.abs(o64 - gz[p + "o"]).max() < 1e-12
        assert np.abs(l64 - gz[p + "lse"]).max() < 1e-12
        p = f"c{i}_bwd_"
        q, k, v = gz[p + "q"], gz[p + "k"], gz[p + "v"]
        g = gz[p + "g"]
        o = np.zeros_like(q)
        lse = np.zeros(nh * seq, np.float32)
        O.attention_forward_blocked(q, k, v, o, lse, seq, nh, nkv, hd, qb)
        dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
        O.attention_backward_blocked(g, q, k, v, o, lse, dq, dk, dv, seq, nh, nkv, hd, qb)
        for name, a in (("dq", dq), ("dk", dk), ("dv", dv)):
            assert O.grad_close_metric(a, gz[p + name])[0] <= 1e-4, (i, name)
        wq, wk, wv = O.attn_bwd_ref_f64(g, q, k, v, seq, nh, nkv, hd)
        for name, a in (("dq", wq), ("dk", wk), ("dv", wv)):
            assert np.abs(a - gz[p + name]).max() < 1e-10, (i, name)


def test_forward_matches_f64_reference():  # attention.rs:324-334
    for i, (seq, nh, nkv, hd, qb) in enumerate(CASES):
        q, k, v = case(seq, nh, nkv, hd, 10 + i)
        o = np.zeros_like(q)
        lse = np.zeros(nh * seq, np.float32)
        O.attention_forward_blocked(q, k, v, o, lse, seq, nh, nkv, hd, qb)
        want, _ = O.attn_ref_f64(q, k, v, seq, nh, nkv, hd)
        assert O.grad_close_metric(o, want)[0] <= 1e-4


def test_block_size_does_not_change_result():  # attention.rs:336-354
    q, k, v = case(37, 4, 2, 8, 30)
    outs = []
    for qb in (1, 16, 1000):
        o = np.zeros_like(q)
        lse = np.zeros(4 * 37, np.float32)
        O.attention_forward_blocked(q, k, v, o, lse, 37, 4, 2, 8, qb)
        outs.append((o, lse))
    for o, lse in outs[1:]:
        assert np.abs(o - outs[0][0]).max() < 1e-5 and np.abs(lse - outs[0][1]).max() < 1e-5


def test_first_token_attends_only_to_itself():  # attention.rs:356-368
    q, k, v = case(5, 2, 1, 4, 40)
    o = np.zeros_like(q)
    lse = np.zeros(10, np.float32)
    O.attention_forward_blocked(q, k, v, o, lse, 5, 2, 1, 4, 128)
    for h in range(2):
        assert np.abs(o[h * 4:(h + 1) * 4] - v[:4]).max() < 1e-6


def test_backward_matches_finite_differences():  # attention.rs:370-393
    for i, (seq, nh, nkv, hd, qb) in enumerate(CASES):
        q, k, v = case(seq, nh, nkv, hd, 50 + i)
        g = O.rand(seq * nh * hd, 70 + i)
        o = np.zeros_like(q)
        lse = np.zeros(nh * seq, np.float32)
        O.attention_forward_blocked(q, k, v, o, lse, seq, nh, nkv, hd, qb)
        dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
        O.attention_backward_blocked(g, q, k, v, o, lse, dq, dk, dv, seq, nh, nkv, hd, qb)
        q64, k64, v64, g64 = (x.astype(np.float64) for x in (q, k, v, g))
        for which, a in enumerate((dq, dk, dv)):
            base = [q64, k64, v64]
            num = np.zeros_like(base[which])
            for j in range(num.size):
                hi = [x.copy() for x in base]
                lo = [x.copy() for x in base]
                hi[which][j] += 1e-6
                lo[which][j] -= 1e-6
                fh = np.dot(O.attn_ref_f64(*hi, seq, nh, nkv, hd)[0], g64)
                fl = np.dot(O.attn_ref_f64(*lo, seq, nh, nkv, hd)[0], g64)
                num[j] = (fh - fl) / 2e-6
            assert O.grad_close_metric(a, num)[0] <= 1e-3, (i, which)


@pytest.mark.parametrize("seq,nh,nkv,hd", [(70, 6, 2, 16), (129, 4, 4, 8), (33, 8, 1, 12)])
def test_oracle_matches_torch_f64_autograd(seq, nh, nkv, hd):
    """Larger shapes than CASES, several q blocks: torch float64 SDPA + autograd."""
    q, k, v = case(seq, nh, nkv, hd, 500 + seq)
    g = O.rand(q.size, 900 + seq)
    o = np.zeros_like(q)
    lse = np.zeros(nh * seq, np.float32)
    O.attention_forward_blocked(q, k, v, o, lse, seq, nh, nkv, hd, 32)
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    O.attention_backward_blocked(g, q, k, v, o, lse, dq, dk, dv, seq, nh, nkv, hd, 32)
    tq, tk, tv = (torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in (q, k, v))
    to = _torch_attn(tq, tk, tv, seq, nh, nkv, hd)
    (to * torch.tensor(g, dtype=torch.float64)).sum().backward()
    assert np.abs(o - to.detach().numpy()).max() < 1e-5
    for a, t in ((dq, tq), (dk, tk), (dv, tv)):
        assert np.abs(a - t.grad.numpy()).max() < 1e-4


def test_head_range_restricts_the_per_head_loop():
    """heads=(h0,h1) equals the full op on those heads; dk/dv get only their share."""
    seq, nh, nkv, hd = 40, 6, 2, 8
    q, k, v = case(seq, nh, nkv, hd, 77)
    g = O.rand(q.size, 78)
    o = np.zeros_like(q)
    lse = np.zeros(nh * seq, np.float32)
    O.attention_forward_blocked(q, k, v, o, lse, seq, nh, nkv, hd, 16)
    o2 = np.zeros_like(q)
    l2 = np.zeros_like(lse)
    O.attention_forward_blocked(q, k, v, o2, l2, seq, nh, nkv, hd, 16, heads=(3, 6))
    assert np.array_equal(o.reshape(seq, nh, hd)[:, 3:], o2.reshape(seq, nh, hd)[:, 3:])
    assert np.all(o2.reshape(seq, nh, hd)[:, :3] == 0)
    dk_full, dk_a, dk_b = (np.zeros_like(k) for _ in range(3))
    for dk, heads in ((dk_full, None), (dk_a, (0, 3)), (dk_b, (3, 6))):
        O.attention_backward_blocked(g, q, k, v, o, lse, np.zeros_like(q), dk, np.zeros_like(v), seq, nh, nkv, hd,
                                     16, heads=heads)
    assert np.abs(dk_full - (dk_a + dk_b)).max() < 1e-5


def test_delta_identity_and_row_sums():
    """delta_t = sum dO*O = sum_j P_tj dP_tj, and sum_j dS_tj = 0 per row."""
    seq, nh, nkv, hd = 30, 2, 1, 8
    q, k, v = case(seq, nh, nkv, hd, 91)
    g = O.rand(q.size, 92)
    qt, kt, vt = (torch.tensor(x, dtype=torch.float64) for x in (q, k, v))
    o = _torch_attn(qt, kt, vt, seq, nh, nkv, hd).numpy().reshape(seq, nh, hd)
    q3, k3, v3, g3 = q.reshape(seq, nh, hd), k.reshape(seq, nkv, hd), v.reshape(seq, nkv, hd), g.reshape(seq, nh, hd)
    for h in range(nh):
        s = q3[:, h].astype(np.float64) @ k3[:, 0].T.astype(np.float64) / math.sqrt(hd)
        s[np.triu_indices(seq, 1)] = -np.inf
        p = np.exp(s - s.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        dp = g3[:, h].astype(np.float64) @ v3[:, 0].T.astype(np.float64)
        delta = (g3[:, h] * o[:, h]).sum(1)
        assert np.abs(delta - (p * dp).sum(1)).max() < 1e-10
        ds = p * (dp - delta[:, None])
        assert np.abs(ds.sum(1)).max() < 1e-10


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(10000).astype(np.float32) * 10.0 ** rng.integers(-5, 5, 10000),
                        np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -1.0 - 2 ** -8, 65504.0, 3.0e38, 0.0, -0.0],
                                 np.float32)]).astype(np.float32)
    want = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(O.round_bf16(x), want)


# ------------------------------------------------------------------ RoPE
def _rope_ref(x, seq, heads, hd, pos0, theta, scaling=None):  # rope.rs:98-114
    half = hd // 2
    y = x.astype(np.float64).copy()
    for t in range(seq):
        for i in range(half):
            f = theta ** (-(2.0 * i) / hd)
            if scaling:
                f = O.llama3_scale(f, *scaling)
            ang = (pos0 + t) * f
            c, s = math.cos(ang), math.sin(ang)
            for h in range(heads):
                b = (t * heads + h) * hd
                x1, x2 = float(x[b + i]), float(x[b + half + i])
                y[b + i] = x1 * c - x2 * s
                y[b + half + i] = x2 * c + x1 * s
    return y


def test_rope_tables_match_golden():
    gz = np.load(os.path.join(GOLDEN, "rope.npz"))
    cos, sin = O.rope_table(16, 32, 10000.0)
    assert np.array_equal(cos, gz["plain_cos"].reshape(-1)) and np.array_equal(sin, gz["plain_sin"].reshape(-1))
    cos, sin = O.rope_table(64, 40, 500000.0, (32.0, 1.0, 4.0, 8192.0))
    assert np.array_equal(cos, gz["llama3_cos"].reshape(-1)) and np.array_equal(sin, gz["llama3_sin"].reshape(-1))


def test_rope_forward_matches_f64_reference():  # rope.rs:121-131
    seq, heads, hd, theta = 6, 3, 16, 10000.0
    cos, sin = O.rope_table(hd, 32, theta)
    x = O.rand(seq * heads * hd, 1)
    y = x.copy()
    O.rope_apply(cos, sin, 32, hd, y, seq, heads, 4, False)
    want = _rope_ref(x, seq, heads, hd, 4, theta)
    assert O.grad_close_metric(y, want)[0] <= 1e-5


L32 = (32.0, 1.0, 4.0, 8192.0)


def test_llama3_scaling_keeps_fast_dims_divides_slow_ones_and_blends_between():  # rope.rs:134-151
    hd, theta = 64, 500000.0
    freqs = [theta ** (-(2.0 * i) / hd) for i in range(hd // 2)]
    scaled = [O.llama3_scale(f, *L32) for f in freqs]
    assert scaled[0] == freqs[0]
    assert abs(scaled[-1] - freqs[-1] / 32.0) < 1e-15
    for s, f in zip(scaled, freqs):
        assert f / 32.0 * (1 - 1e-12) <= s <= f * (1 + 1e-12)
    assert any(f / 32.0 * 1.01 < s < f * 0.99 for s, f in zip(scaled, freqs))
    assert all(b <= a for a, b in zip(scaled, scaled[1:]))


def test_scaled_cache_matches_reference_rotation_with_scaled_frequencies():  # rope.rs:153-178
    seq, heads, hd, theta = 5, 2, 16, 500000.0
    cos, sin = O.rope_table(hd, 32, theta, L32)
    x = O.rand(seq * heads * hd, 9)
    y = x.copy()
    O.rope_apply(cos, sin, 32, hd, y, seq, heads, 3, False)
    assert O.grad_close_metric(y, _rope_ref(x, seq, heads, hd, 3, theta, L32))[0] <= 1e-5


def test_rope_position_zero_is_identity():  # rope.rs:180-187
    cos, sin = O.rope_table(8, 4, 10000.0)
    x = O.rand(16, 2)
    y = x.copy()
    O.rope_apply(cos, sin, 4, 8, y, 1, 2, 0, False)
    assert np.array_equal(x, y)


def test_rotation_preserves_norm_and_inverse_roundtrips():  # rope.rs:189-203
    seq, heads, hd = 10, 2, 32
    cos, sin = O.rope_table(hd, 64, 500000.0)
    x = O.rand(seq * heads * hd, 3)
    y = x.copy()
    O.rope_apply(cos, sin, 64, hd, y, seq, heads, 7, False)
    assert abs((x * x).sum() - (y * y).sum()) / (x * x).sum() < 1e-5
    O.rope_apply(cos, sin, 64, hd, y, seq, heads, 7, True)
    assert np.abs(x - y).max() < 1e-4


def test_rope_backward_matches_finite_differences():  # rope.rs:205-222
    seq, heads, hd, theta = 4, 2, 8, 10000.0
    cos, sin = O.rope_table(hd, 16, theta)
    x = O.rand(seq * heads * hd, 4)
    g = O.rand(seq * heads * hd, 5)
    dx = g.copy()
    O.rope_apply(cos, sin, 16, hd, dx, seq, heads, 2, True)
    num = np.zeros(x.size)
    for j in range(x.size):
        hi, lo = x.astype(np.float64).copy(), x.astype(np.float64).copy()
        hi[j] += 1e-6
        lo[j] -= 1e-6
        num[j] = (np.dot(_rope_ref(hi, seq, heads, hd, 2, theta), g) - np.dot(_rope_ref(lo, seq, heads, hd, 2, theta),
                                                                              g)) / 2e-6
    assert O.grad_close_metric(dx, num)[0] <= 5e-4


def test_rope_position_out_of_cache_is_rejected():  # rope.rs:73
    cos, sin = O.rope_table(8, 4, 10000.0)
    x = np.zeros(5 * 8, np.float32)
    with pytest.raises(ValueError):
        O.rope_apply(cos, sin, 4, 8, x, 5, 1, 0, False)


# --------------------------------------------------------------- RMSNorm
def _setup_norm(rows, dim, seed):  # rmsnorm.rs:88-94
    r = O.Rng(seed)
    x = np.array([r.normal() * 1.5 + 0.3 for _ in range(rows * dim)], np.float32)
    w = np.array([1.0 + 0.5 * r.normal() for _ in range(dim)], np.float32)
    g = np.array([r.normal() for _ in range(rows * dim)], np.float32)
    return x, w, g


def _rmsnorm_ref(x, w, rows, dim, eps):  # rmsnorm.rs:75-86
    x = x.reshape(rows, dim).astype(np.float64)
    inv = 1.0 / np.sqrt((x * x).mean(1, keepdims=True) + eps)
    return (x * inv * w.astype(np.float64)).reshape(-1)


def test_rmsnorm_forward_matches_f64_reference():  # rmsnorm.rs:96-105
    rows, dim, eps = 5, 37, 1e-5
    x, w, _ = _setup_norm(rows, dim, 1)
    y = np.zeros_like(x)
    rstd = np.zeros(rows, np.float32)
    O.rmsnorm_forward(x, w, y, rstd, rows, dim, eps)
    assert O.grad_close_metric(y, _rmsnorm_ref(x, w, rows, dim, eps))[0] <= 1e-5


def test_rmsnorm_output_has_unit_rms_when_weight_is_one():  # rmsnorm.rs:107-119
    rows, dim = 4, 64
    x, _, _ = _setup_norm(rows, dim, 2)
    y = np.zeros_like(x)
    rstd = np.zeros(rows, np.float32)
    O.rmsnorm_forward(x, np.ones(dim, np.float32), y, rstd, rows, dim, 1e-8)
    assert np.abs((y.reshape(rows, dim) ** 2).mean(1) - 1.0).max() < 1e-4


def test_rmsnorm_backward_matches_finite_differences():  # rmsnorm.rs:121-144
    rows, dim, eps = 3, 16, 1e-5
    x, w, g = _setup_norm(rows, dim, 3)
    y = np.zeros_like(x)
    rstd = np.zeros(rows, np.float32)
    O.rmsnorm_forward(x, w, y, rstd, rows, dim, eps)
    dx = np.zeros_like(x)
    dw = np.zeros_like(w)
    O.rmsnorm_backward(g, x, w, rstd, dx, dw, rows, dim)
    for a, wrt in ((dx, "x"), (dw, "w")):
        base = x if wrt == "x" else w
        num = np.zeros(base.size)
        for j in range(base.size):
            hi, lo = base.astype(np.float64).copy(), base.astype(np.float64).copy()
            hi[j] += 1e-6
            lo[j] -= 1e-6
            if wrt == "x":
                fh, fl = _rmsnorm_ref(hi, w, rows, dim, eps), _rmsnorm_ref(lo, w, rows, dim, eps)
            else:
                fh, fl = _rmsnorm_ref(x, hi, rows, dim, eps), _rmsnorm_ref(x, lo, rows, dim, eps)
            num[j] = (np.dot(fh, g) - np.dot(fl, g)) / 2e-6
        assert O.grad_close_metric(a, num)[0] <= 5e-4, wrt


def test_rmsnorm_backward_accumulates():  # rmsnorm.rs:146-168
    rows, dim, eps = 2, 8, 1e-5
    x, w, g = _setup_norm(rows, dim, 4)
    y = np.zeros_like(x)
    rstd = np.zeros(rows, np.float32)
    O.rmsnorm_forward(x, w, y, rstd, rows, dim, eps)
    dx1, dw1 = np.zeros_like(x), np.zeros_like(w)
    O.rmsnorm_backward(g, x, w, rstd, dx1, dw1, rows, dim)
    dx2, dw2 = dx1.copy(), dw1.copy()
    O.rmsnorm_backward(g, x, w, rstd, dx2, dw2, rows, dim)
    assert np.abs(dx2 - 2 * dx1).max() < 1e-5 and np.abs(dw2 - 2 * dw1).max() < 1e-5


# ------------------------------------------------------------ layer chain
def test_layer_prologue_chain_matches_torch_autograd():
    """q/k norm -> RoPE forward and its backward chain (layer.rs:104-116,
    191-206) vs torch float64 autograd of the same composition."""
    seq, nh, nkv, hd, theta, eps = 9, 4, 2, 16, 1e6, 1e-6
    cos, sin = O.rope_table(hd, 16, theta)
    qp, kp = O.rand(seq * nh * hd, 11), O.rand(seq * nkv * hd, 12)
    qw = (1.0 + O.rand(hd, 13, 0.02)).astype(np.float32)
    kw = (1.0 + O.rand(hd, 14, 0.02)).astype(np.float32)
    gq, gk = O.rand(seq * nh * hd, 15), O.rand(seq * nkv * hd, 16)
    q, k, qr, kr = O.layer_prologue_forward(qp, kp, seq, nh, nkv, hd, cos, sin, 16, 0, qw, kw, eps)
    dqp, dkp, dqw, dkw = O.layer_prologue_backward(gq, gk, qp, kp, seq, nh, nkv, hd, cos, sin, 16, 0, qw, kw, qr, kr)
    c = torch.tensor(cos.reshape(16, hd // 2)[:seq], dtype=torch.float64)
    s = torch.tensor(sin.reshape(16, hd // 2)[:seq], dtype=torch.float64)

    def chain(x, w, heads):
        x = x.view(seq, heads, hd)
        x = x * torch.rsqrt((x * x).mean(-1, keepdim=True) + eps) * w
        x1, x2 = x[..., : hd // 2], x[..., hd // 2:]
        cc, ss = c[:, None, :], s[:, None, :]
        return torch.cat([x1 * cc - x2 * ss, x2 * cc + x1 * ss], -1).reshape(-1)

    for pre, w, heads, out, g, dpre, dw in ((qp, qw, nh, q, gq, dqp, dqw), (kp, kw, nkv, k, gk, dkp, dkw)):
        tx = torch.tensor(pre, dtype=torch.float64, requires_grad=True)
        tw = torch.tensor(w, dtype=torch.float64, requires_grad=True)
        y = chain(tx, tw, heads)
        assert np.abs(out - y.detach().numpy()).max() < 1e-5
        (y * torch.tensor(g, dtype=torch.float64)).sum().backward()
        assert np.abs(dpre - tx.grad.numpy()).max() < 1e-4
        assert np.abs(dw - tw.grad.numpy()).max() < 1e-3
