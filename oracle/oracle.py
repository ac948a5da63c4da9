"""ctypes binding of the C attention and layer-op oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker.  The product package
(cpuforge_amd) never imports this module.

Every function mirrors one in cforge_oracle.c, oracle_layer.c or oracle_io.c, which cite the reference
file:line it restates.  Arrays are numpy, C-contiguous; the caller owns them,
as in the reference where callers lend slices.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(dtype=np.int64, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_sz = C.c_size_t


def build() -> None:
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        L.orc_rng_seed.restype = C.c_uint64
        L.orc_rng_seed.argtypes = [C.c_uint64]
        L.orc_rng_next_u64.restype = C.c_uint64
        L.orc_rng_next_u64.argtypes = [C.POINTER(C.c_uint64)]
        L.orc_rng_uniform.restype = C.c_float
        L.orc_rng_uniform.argtypes = [C.POINTER(C.c_uint64)]
        L.orc_rng_normal.restype = C.c_float
        L.orc_rng_normal.argtypes = [C.POINTER(C.c_uint64)]
        L.orc_fill_normal.restype = None
        L.orc_fill_normal.argtypes = [C.c_uint64, _f32p, _sz, C.c_float]
        L.orc_gemm_strided.restype = None
        L.orc_gemm_strided.argtypes = [C.c_void_p, C.c_long, C.c_long, C.c_void_p, C.c_long, C.c_long,
                                       C.c_void_p, C.c_long, C.c_long, _sz, _sz, _sz, C.c_int]
        L.orc_gemm_threads.restype = C.c_int
        L.orc_set_gemm_threads.argtypes = [C.c_int]
        L.orc_set_gemm_threads.restype = None
        L.orc_attention_forward_heads.restype = C.c_int
        L.orc_attention_forward_heads.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p] + [_sz] * 7
        L.orc_attention_backward_heads.restype = C.c_int
        L.orc_attention_backward_heads.argtypes = [_f32p] * 9 + [_sz] * 7
        L.orc_attn_ref_f64.restype = None
        L.orc_attn_ref_f64.argtypes = [_f64p] * 5 + [_sz] * 4 + [C.c_void_p]
        L.orc_attn_bwd_ref_f64.restype = None
        L.orc_attn_bwd_ref_f64.argtypes = [_f64p] * 7 + [_sz] * 6
        L.orc_llama3_scale.restype = C.c_double
        L.orc_llama3_scale.argtypes = [C.c_double] * 5
        L.orc_rope_table.restype = C.c_int
        L.orc_rope_table.argtypes = [_sz, _sz, C.c_double, C.c_void_p, _f32p, _f32p]
        L.orc_rope_apply.restype = C.c_int
        L.orc_rope_apply.argtypes = [_f32p, _f32p, _sz, _sz, _f32p, _sz, _sz, _sz, C.c_int]
        L.orc_rmsnorm_forward.restype = None
        L.orc_rmsnorm_forward.argtypes = [_f32p, _f32p, _f32p, _f32p, _sz, _sz, C.c_float]
        L.orc_rmsnorm_backward.restype = None
        L.orc_rmsnorm_backward.argtypes = [_f32p] * 6 + [_sz, _sz]
        L.orc_f32_to_bf16.restype = C.c_uint16
        L.orc_f32_to_bf16.argtypes = [C.c_float]
        L.orc_round_bf16.restype = None
        L.orc_round_bf16.argtypes = [_f32p, _f32p, _sz]
        L.orc_grad_close_metric.restype = C.c_double
        L.orc_grad_close_metric.argtypes = [_f32p, _f64p, _sz, C.POINTER(C.c_size_t)]
        for fn in (L.orc_bf16_to_f32, L.orc_f16_to_f32):
            fn.restype = None
            fn.argtypes = [_u16p, _f32p, _sz]
        L.orc_silu_mul_forward.restype = None
        L.orc_silu_mul_forward.argtypes = [_f32p] * 3 + [_sz]
        L.orc_silu_mul_backward.restype = None
        L.orc_silu_mul_backward.argtypes = [_f32p] * 5 + [_sz]
        L.orc_cross_entropy_fwd_bwd.restype = C.c_float
        L.orc_cross_entropy_fwd_bwd.argtypes = [_f32p, _i64p, _f32p, _sz, _sz, C.POINTER(C.c_long)]
        L.orc_powi_f32.restype = C.c_float
        L.orc_powi_f32.argtypes = [C.c_float, C.c_int]
        L.orc_adamw_update.restype = None
        L.orc_adamw_update.argtypes = [_f32p] * 4 + [_sz, C.c_uint64] + [C.c_float] * 5
        L.orc_linear_forward.restype = None
        L.orc_linear_forward.argtypes = [C.c_void_p] * 4 + [C.c_float] + [_sz] * 4 + [C.c_void_p] * 2
        L.orc_linear_backward.restype = None
        L.orc_linear_backward.argtypes = [C.c_void_p] * 6 + [C.c_float] + [_sz] * 4 + [C.c_void_p] * 5
        _lib = L
    return _lib


# ---------------------------------------------------------------- Rng
class Rng:
    """crates/core/src/rng.rs: xorshift64* with f32 Box-Muller."""

    def __init__(self, seed: int):
        self.state = C.c_uint64(lib().orc_rng_seed(seed))

    def next_u64(self) -> int:
        return lib().orc_rng_next_u64(C.byref(self.state))

    def uniform(self) -> float:
        return lib().orc_rng_uniform(C.byref(self.state))

    def normal(self) -> float:
        return lib().orc_rng_normal(C.byref(self.state))


def rand(n: int, seed: int, std: float = 1.0) -> np.ndarray:
    """`rand(n, seed, std)` of the reference tests: Rng::new(seed), n normals * std
    (core/src/ops/attention.rs:298-301)."""
    out = np.empty(n, dtype=np.float32)
    lib().orc_fill_normal(seed, out, n, std)
    return out


# --------------------------------------------------------------- GEMM
def gemm_strided(a, a_rs, a_cs, b, b_rs, b_cs, c, c_rs, c_cs, m, k, n, acc):
    """core/src/matmul.rs:37-98 semantics on flat float32 buffers."""
    for arr in (a, b, c):
        assert arr.dtype == np.float32 and arr.flags.c_contiguous
    lib().orc_gemm_strided(a.ctypes.data, a_rs, a_cs, b.ctypes.data, b_rs, b_cs, c.ctypes.data, c_rs, c_cs,
                           m, k, n, int(bool(acc)))


def gemm_threads() -> int:
    return lib().orc_gemm_threads()


def set_gemm_threads(n: int) -> None:
    """Threads the oracle GEMM uses from now on (n >= 1)."""
    lib().orc_set_gemm_threads(int(n))


# ---------------------------------------------------------- attention
def _chk(rc: int, what: str):
    if rc != 0:
        raise ValueError(f"{what}: oracle returned {rc}")


def attention_forward_blocked(q, k, v, o, lse, seq, nh, nkv, hd, q_block=128, heads=None):
    """core/src/ops/attention.rs:46-122; overwrites o and lse.  `heads=(h0,h1)`
    restricts the per-head loop to a sub-range."""
    h0, h1 = heads if heads is not None else (0, nh)
    _chk(lib().orc_attention_forward_heads(q, k, v, o, lse, seq, nh, nkv, hd, q_block, h0, h1), "forward")


def attention_backward_blocked(d_o, q, k, v, o, lse, dq, dk, dv, seq, nh, nkv, hd, q_block=128, heads=None):
    """core/src/ops/attention.rs:142-262; accumulates into dq, dk, dv."""
    h0, h1 = heads if heads is not None else (0, nh)
    _chk(lib().orc_attention_backward_heads(d_o, q, k, v, o, lse, dq, dk, dv, seq, nh, nkv, hd, q_block, h0, h1),
         "backward")


def attn_ref_f64(q, k, v, seq, nh, nkv, hd, row_mask=None):
    """Naive f64 attention (attention.rs:271-296) plus lse; returns (o, lse)."""
    q, k, v = (np.ascontiguousarray(x, dtype=np.float64) for x in (q, k, v))
    o = np.zeros(seq * nh * hd, dtype=np.float64)
    lse = np.zeros(nh * seq, dtype=np.float64)
    mptr = None
    if row_mask is not None:
        row_mask = np.ascontiguousarray(row_mask, dtype=np.uint8)
        mptr = row_mask.ctypes.data
    lib().orc_attn_ref_f64(q, k, v, o, lse, seq, nh, nkv, hd, mptr)
    return o, lse


def attn_bwd_ref_f64(d_o, q, k, v, seq, nh, nkv, hd, heads=None):
    """Closed-form f64 gradients of sum(dO * attn); returns (dq, dk, dv)."""
    h0, h1 = heads if heads is not None else (0, nh)
    d_o, q, k, v = (np.ascontiguousarray(x, dtype=np.float64) for x in (d_o, q, k, v))
    dq = np.zeros(seq * nh * hd)
    dk = np.zeros(seq * nkv * hd)
    dv = np.zeros(seq * nkv * hd)
    lib().orc_attn_bwd_ref_f64(d_o, q, k, v, dq, dk, dv, seq, nh, nkv, hd, h0, h1)
    return dq, dk, dv


# ---------------------------------------------------------------- RoPE
def llama3_scale(inv_freq, factor, low, high, orig):
    return lib().orc_llama3_scale(inv_freq, factor, low, high, orig)


def rope_table(head_dim, max_pos, theta, scaling=None):
    """RopeCache::with_scaling (core/src/ops/rope.rs:46-63); scaling is
    (factor, low_freq_factor, high_freq_factor, original_max_position)."""
    half = head_dim // 2
    cos = np.empty(max_pos * half, dtype=np.float32)
    sin = np.empty(max_pos * half, dtype=np.float32)
    sp = None
    if scaling is not None:
        s = np.asarray(scaling, dtype=np.float64)
        sp = s.ctypes.data
    _chk(lib().orc_rope_table(head_dim, max_pos, float(theta), sp, cos, sin), "rope_table")
    return cos, sin


def rope_apply(cos, sin, max_pos, head_dim, x, seq, heads, pos0, inverse):
    """RopeCache::apply (core/src/ops/rope.rs:71-89), in place on x."""
    _chk(lib().orc_rope_apply(cos, sin, max_pos, head_dim, x, seq, heads, pos0, int(bool(inverse))), "rope_apply")


# ------------------------------------------------------------- RMSNorm
def rmsnorm_forward(x, w, y, rstd, rows, dim, eps):
    lib().orc_rmsnorm_forward(x, w, y, rstd, rows, dim, eps)


def rmsnorm_backward(dy, x, w, rstd, dx, dw, rows, dim):
    lib().orc_rmsnorm_backward(dy, x, w, rstd, dx, dw, rows, dim)


# ----------------------------------------------- layer ops (oracle_layer.c)
IGNORE_INDEX = -100  # crates/core/src/ops/loss.rs:4


def silu_mul_forward(g, u, h):
    """crates/core/src/ops/swiglu.rs:10-16: h = silu(g) * u (overwrites h)."""
    lib().orc_silu_mul_forward(g, u, h, g.size)


def silu_mul_backward(dh, g, u, dg, du):
    """crates/core/src/ops/swiglu.rs:18-30: accumulates into dg, du."""
    lib().orc_silu_mul_backward(dh, g, u, dg, du, g.size)


def cross_entropy_fwd_bwd(logits, targets, dlogits, rows, vocab):
    """crates/core/src/ops/loss.rs:9-55: mean cross-entropy, dlogits
    overwritten.  Raises ValueError where the reference panics (a target out
    of range)."""
    bad = C.c_long(-1)
    loss = lib().orc_cross_entropy_fwd_bwd(logits, np.ascontiguousarray(targets, dtype=np.int64), dlogits, rows,
                                           vocab, C.byref(bad))
    if bad.value >= 0:
        raise ValueError(f"target {int(targets[bad.value])} out of range for vocab {vocab}")
    return float(loss)


def powi_f32(a: float, b: int) -> float:
    return lib().orc_powi_f32(a, b)


def adamw_update(p, g, m, v, t, lr, beta1, beta2, eps, weight_decay):
    """crates/train/src/optim.rs:9-30, in place on p, m, v."""
    lib().orc_adamw_update(p, g, m, v, p.size, t, lr, beta1, beta2, eps, weight_decay)


def _ptr(a):
    return None if a is None else a.ctypes.data


def linear_forward(x, w, a, b, scale, t, inn, out, r, y, xs):
    """Linear::forward (crates/model/src/linear.rs:56-71); a/b/xs None
    without an adapter."""
    lib().orc_linear_forward(_ptr(x), _ptr(w), _ptr(a), _ptr(b), scale, t, inn, out, r, _ptr(y), _ptr(xs))


def linear_backward(x, xs, dy, w, a, b, scale, t, inn, out, r, dx, gw=None, ga=None, gb=None):
    """Linear::backward (crates/model/src/linear.rs:73-91): accumulates into
    dx and every gradient given."""
    dxa = np.zeros(t * max(r, 1), dtype=np.float32)
    lib().orc_linear_backward(_ptr(x), _ptr(xs), _ptr(dy), _ptr(w), _ptr(a), _ptr(b), scale, t, inn, out, r, _ptr(dx),
                              _ptr(gw), _ptr(ga), _ptr(gb), _ptr(dxa))


# ---------------------------------------------------------------- bf16
def round_bf16(x: np.ndarray) -> np.ndarray:
    """RNE-round float32 values to bf16 and widen back to float32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().orc_round_bf16(x.reshape(-1), out.reshape(-1), x.size)
    return out


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    return (round_bf16(x).view(np.uint32) >> 16).astype(np.uint16)


def grad_close_metric(a: np.ndarray, n: np.ndarray):
    """core/src/gradcheck.rs:31-48: worst |a-n|/(1+|n|) and its index."""
    a = np.ascontiguousarray(a, dtype=np.float32).reshape(-1)
    n = np.ascontiguousarray(n, dtype=np.float64).reshape(-1)
    wi = C.c_size_t(0)
    w = lib().orc_grad_close_metric(a, n, a.size, C.byref(wi))
    return w, wi.value


# ------------------------------------------------------------ layer chain
def layer_prologue_forward(q_pre, k_pre, seq, nh, nkv, hd, cos, sin, max_pos, pos0=0, q_norm=None, k_norm=None,
                           eps=1e-6):
    """The attention prologue of Layer::forward (crates/model/src/layer.rs:104-116):
    optional per-head RMSNorm of q/k (Qwen3), then RoPE.  Returns
    (q, k, q_rstd, k_rstd); rstd are None without the norm."""
    q = np.array(q_pre, dtype=np.float32, copy=True)
    k = np.array(k_pre, dtype=np.float32, copy=True)
    q_rstd = k_rstd = None
    if q_norm is not None:
        q_rstd = np.zeros(seq * nh, dtype=np.float32)
        k_rstd = np.zeros(seq * nkv, dtype=np.float32)
        rmsnorm_forward(np.ascontiguousarray(q_pre, dtype=np.float32), q_norm, q, q_rstd, seq * nh, hd, eps)
        rmsnorm_forward(np.ascontiguousarray(k_pre, dtype=np.float32), k_norm, k, k_rstd, seq * nkv, hd, eps)
    rope_apply(cos, sin, max_pos, hd, q, seq, nh, pos0, False)
    rope_apply(cos, sin, max_pos, hd, k, seq, nkv, pos0, False)
    return q, k, q_rstd, k_rstd


def layer_prologue_backward(dq, dk, q_pre, k_pre, seq, nh, nkv, hd, cos, sin, max_pos, pos0=0, q_norm=None,
                            k_norm=None, q_rstd=None, k_rstd=None):
    """The chain after attention_backward in Layer::backward (layer.rs:191-206):
    inverse RoPE, then the per-head RMSNorm backward into fresh dq_pre/dk_pre
    and accumulated norm-weight gradients.  Returns (dq_pre, dk_pre, dqw, dkw)."""
    dq = np.array(dq, dtype=np.float32, copy=True)
    dk = np.array(dk, dtype=np.float32, copy=True)
    rope_apply(cos, sin, max_pos, hd, dq, seq, nh, pos0, True)
    rope_apply(cos, sin, max_pos, hd, dk, seq, nkv, pos0, True)
    if q_norm is None:
        return dq, dk, None, None
    dq_pre = np.zeros_like(dq)
    dk_pre = np.zeros_like(dk)
    dqw = np.zeros(hd, dtype=np.float32)
    dkw = np.zeros(hd, dtype=np.float32)
    rmsnorm_backward(dq, np.ascontiguousarray(q_pre, dtype=np.float32), q_norm, q_rstd, dq_pre, dqw, seq * nh, hd)
    rmsnorm_backward(dk, np.ascontiguousarray(k_pre, dtype=np.float32), k_norm, k_rstd, dk_pre, dkw, seq * nkv, hd)
    return dq_pre, dk_pre, dqw, dkw


# ---------------------------------------------------------------- on-disk formats
def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """crates/io/src/dtype.rs:3-5 over an array of uint16 patterns."""
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().orc_bf16_to_f32(bits.ravel(), out.ravel(), bits.size)
    return out


def f16_to_f32(bits: np.ndarray) -> np.ndarray:
    """crates/io/src/dtype.rs:7-33 over an array of uint16 patterns."""
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().orc_f16_to_f32(bits.ravel(), out.ravel(), bits.size)
    return out
