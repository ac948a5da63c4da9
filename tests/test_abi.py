"""CPU tests of the C ABI (no GPU needed): libcfattn.so loads, exports every
function include/cfattn.h, include/cfops.h and include/cfio.h declare, the ctypes table
covers them, and the host-only helpers agree with the oracle."""
import ctypes as C
import os
import re

import numpy as np
import pytest

from cpuforge_amd import _lib
from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("cfattn.h", "cfops.h", "cfio.h")]


def header_text():
    return re.sub(r"/\*.*?\*/", "", "\n".join(open(h).read() for h in HEADERS), flags=re.S)


def declared_functions():
    return sorted(set(re.findall(r"\b(cf(?:attn|ops|io)_\w+)\s*\(", header_text())))


def test_header_declares_the_reference_interface():
    names = declared_functions()
    for n in ("cfattn_attention_forward", "cfattn_attention_forward_blocked", "cfattn_attention_backward",
              "cfattn_attention_backward_blocked", "cfattn_fwd", "cfattn_bwd", "cfattn_fused_fwd",
              "cfattn_fused_bwd", "cfattn_rope_table", "cfattn_last_error"):
        assert n in names


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    missing = [n for n in declared_functions() if not hasattr(L, n)]
    assert not missing, f"libcfattn.so lacks {missing}"


def declared_arities():
    """Parameter count of every function the headers declare."""
    out = {}
    for name, params in re.findall(r"\b(cf(?:attn|ops|io)_\w+)\s*\(([^)]*)\)\s*;", header_text()):
        params = params.strip()
        out[name] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_ctypes_table_matches_header():
    assert sorted(_lib.SIGNATURES) == declared_functions()
    arity = declared_arities()
    assert sorted(arity) == declared_functions()
    # a missing trailing argument would make ctypes pass a 64-bit pointer as int
    wrong = {n: (len(args), arity[n]) for n, (_, args) in _lib.SIGNATURES.items() if len(args) != arity[n]}
    assert not wrong, f"ctypes argument counts differ from the header: {wrong}"


def test_layer_op_header_declares_the_reference_ops():
    names = declared_functions()
    for n in ("cfops_matmul", "cfops_rmsnorm_forward", "cfops_rmsnorm_backward", "cfops_silu_mul_forward",
              "cfops_silu_mul_backward", "cfops_cross_entropy_fwd_bwd", "cfops_lm_head_ce", "cfops_linear_forward",
              "cfops_linear_backward", "cfops_adamw_update"):
        assert n in names


def test_layer_ops_reject_a_null_context():
    L = _lib.lib()
    assert L.cfops_rmsnorm_forward(None, None, None, None, None, 1, 1, 1e-5, None) == _lib.ERR_ARG
    assert L.cfops_matmul(None, 0, None, None, None, 1, 1, 1, 0, None) == _lib.ERR_ARG
    loss = C.c_float(0)
    assert L.cfops_cross_entropy_fwd_bwd(None, None, None, None, 1, 1, C.byref(loss), None) == _lib.ERR_ARG


def test_rope_table_matches_oracle_bitwise():
    from cpuforge_amd import Llama3Scaling, RopeCache
    for hd, mp, theta, sc in ((64, 300, 1e4, None), (128, 200, 1e6, None), (64, 128, 5e5, (32.0, 1.0, 4.0, 8192.0))):
        r = RopeCache(hd, mp, theta, Llama3Scaling(*sc) if sc else None)
        cos, sin = O.rope_table(hd, mp, theta, sc)
        assert np.array_equal(r.cos.reshape(-1), cos) and np.array_equal(r.sin.reshape(-1), sin)


def test_llama3_scale_matches_oracle():
    from cpuforge_amd import Llama3Scaling
    sc = Llama3Scaling(32.0, 1.0, 4.0, 8192.0)
    for i in range(64):
        f = 500000.0 ** (-2.0 * i / 128)
        assert sc.apply(f) == O.llama3_scale(f, 32.0, 1.0, 4.0, 8192.0)


def test_odd_head_dim_rope_is_a_shape_error():  # rope.rs:47
    from cpuforge_amd import RopeCache
    with pytest.raises(AssertionError):
        RopeCache(7, 4, 1e4)


def test_flops_formula():
    s = _lib.Shape(8192, 32, 8, 128)
    assert _lib.lib().cfattn_flops_fwd_bwd(s, 1) == 7.0 * 32 * 128 * 8192 * 8193


def test_kernel_names():
    L = _lib.lib()
    names = [L.cfattn_kernel_name(i).decode() for i in range(L.cfattn_kernel_count())]
    assert "attn_fwd" in names and "attn_bwd_dkdv" in names and "attn_bwd_dq" in names
    assert L.cfattn_kernel_name(L.cfattn_kernel_count()) is None


def test_null_context_is_an_argument_error():
    L = _lib.lib()
    s = _lib.Shape(4, 2, 1, 8)
    assert L.cfattn_fwd(None, s, 1, 0, None, None, None, None, None, None) == _lib.ERR_ARG
    assert L.cfattn_attention_forward(None, None, 0, None, 0, None, 0, None, 0, None, 0, s) == _lib.ERR_ARG
    assert L.cfattn_destroy(None) == _lib.ERR_ARG
    assert L.cfattn_last_error(None) == b"null context"


def test_create_without_a_device_fails_cleanly():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    h = C.c_void_p()
    assert _lib.lib().cfattn_create(0, C.byref(h)) != _lib.OK
    assert not h.value
