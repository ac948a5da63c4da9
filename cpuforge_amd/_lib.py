"""Loads libcfattn.so (built in-tree by cpuforge_amd/build.py) and declares
the C ABI of include/cfattn.h, include/cfops.h and include/cfio.h for ctypes.

There is no fallback: if the library is missing the import of any compute
function raises, so nothing can silently run on the CPU instead of the GPU.
"""
from __future__ import annotations

import ctypes as C
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libcfattn.so")

OK, ERR_SHAPE, ERR_ARG, ERR_UNSUPPORTED, ERR_HIP, ERR_NOMEM, ERR_IO = range(7)
F32, BF16 = 0, 1

# Every function include/cfattn.h, include/cfops.h and include/cfio.h declare, with
# (restype, argtypes).
_sz = C.c_size_t
_vp = C.c_void_p
_fp = C.POINTER(C.c_float)


class Shape(C.Structure):
    """`cfattn_shape`, the C mirror of AttnShape (core/src/ops/attention.rs:20-26)."""
    _fields_ = [("seq", _sz), ("n_heads", _sz), ("n_kv", _sz), ("head_dim", _sz)]


class Llama3ScalingC(C.Structure):
    _fields_ = [("factor", C.c_double), ("low_freq_factor", C.c_double), ("high_freq_factor", C.c_double),
                ("original_max_position", C.c_double)]


class PrologueC(C.Structure):
    _fields_ = [("cos", _vp), ("sin", _vp), ("max_pos", _sz), ("pos0", _sz), ("q_norm", _vp), ("k_norm", _vp),
                ("eps", C.c_float)]


SIGNATURES = {
    "cfattn_create": (C.c_int, [C.c_int, C.POINTER(_vp)]),
    "cfattn_destroy": (C.c_int, [_vp]),
    "cfattn_last_error": (C.c_char_p, [_vp]),
    "cfattn_set_mode": (C.c_int, [_vp, C.c_int]),
    "cfattn_get_mode": (C.c_int, [_vp]),
    "cfattn_synchronize": (C.c_int, [_vp]),
    "cfattn_stream": (_vp, [_vp]),
    "cfattn_attention_forward": (C.c_int, [_vp, _vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz, Shape]),
    "cfattn_attention_forward_blocked": (C.c_int, [_vp, _vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz, _vp, _sz, Shape,
                                                   _sz]),
    "cfattn_attention_backward": (C.c_int, [_vp] + [_vp, _sz] * 9 + [Shape]),
    "cfattn_attention_backward_blocked": (C.c_int, [_vp] + [_vp, _sz] * 9 + [Shape, _sz]),
    "cfattn_fwd": (C.c_int, [_vp, Shape, _sz, C.c_int, _vp, _vp, _vp, _vp, _vp, _vp]),
    "cfattn_bwd": (C.c_int, [_vp, Shape, _sz, C.c_int] + [_vp] * 10),
    "cfattn_bwd_noalloc": (C.c_int, [_vp, Shape, _sz, C.c_int] + [_vp] * 10),
    "cfattn_prologue_fwd": (C.c_int, [_vp, Shape, _sz, C.c_int, C.POINTER(PrologueC)] + [_vp] * 7),
    "cfattn_prologue_bwd": (C.c_int, [_vp, Shape, _sz, C.POINTER(PrologueC)] + [_vp] * 11),
    "cfattn_fused_fwd": (C.c_int, [_vp, Shape, _sz, C.c_int, C.POINTER(PrologueC)] + [_vp] * 10),
    "cfattn_fused_bwd": (C.c_int, [_vp, Shape, _sz, C.c_int, C.POINTER(PrologueC)] + [_vp] * 16),
    "cfattn_rope_table": (C.c_int, [_sz, _sz, C.c_double, C.POINTER(Llama3ScalingC), _vp, _vp]),
    "cfattn_llama3_scale": (C.c_double, [C.POINTER(Llama3ScalingC), C.c_double]),
    "cfattn_f32_to_bf16": (C.c_int, [_vp, _vp, _vp, _sz, _vp]),
    "cfattn_set_ds_limit": (C.c_int, [_vp, _sz]),
    "cfattn_get_ds_limit": (_sz, [_vp]),
    "cfattn_profile_enable": (C.c_int, [_vp, C.c_int]),
    "cfattn_profile_select": (C.c_int, [_vp, C.c_uint]),
    "cfattn_profile_read": (C.c_int, [_vp, C.c_int, C.POINTER(C.c_double), C.POINTER(C.c_longlong)]),
    "cfattn_probe_mfma_peak": (C.c_int, [_vp, C.c_int, C.c_int, C.POINTER(C.c_double)]),
    "cfattn_probe_loop": (C.c_int, [_vp, C.c_int, C.c_int, C.POINTER(C.c_double)]),
    "cfattn_fwd_stats_enable": (C.c_int, [_vp, C.c_int]),
    "cfattn_fwd_stats_read": (C.c_int, [_vp, C.POINTER(C.c_longlong)]),
    "cfattn_kernel_name": (C.c_char_p, [C.c_int]),
    "cfattn_kernel_count": (C.c_int, []),
    "cfattn_flops_fwd_bwd": (C.c_double, [Shape, _sz]),
    "cfattn_version": (C.c_char_p, []),
    # include/cfops.h
    "cfops_matmul": (C.c_int, [_vp, C.c_int, _vp, _vp, _vp, _sz, _sz, _sz, C.c_int, _vp]),
    "cfops_rmsnorm_forward": (C.c_int, [_vp] * 5 + [_sz, _sz, C.c_float, _vp]),
    "cfops_rmsnorm_backward": (C.c_int, [_vp] * 7 + [_sz, _sz, _vp]),
    "cfops_silu_mul_forward": (C.c_int, [_vp] * 4 + [_sz, _vp]),
    "cfops_silu_mul_backward": (C.c_int, [_vp] * 6 + [_sz, _vp]),
    "cfops_cross_entropy_fwd_bwd": (C.c_int, [_vp] * 4 + [_sz, _sz, _fp, _vp]),
    "cfops_lm_head_ce": (C.c_int, [_vp] * 4 + [_sz, _sz, _sz, _vp, _vp, _fp, _vp]),
    "cfops_lm_head_ce_dev": (C.c_int, [_vp] * 4 + [_sz, _sz, _sz, _vp, _vp, _vp, _vp]),
    "cfops_set_head_chunk_limit": (C.c_int, [_vp, _sz]),
    "cfops_linear_forward": (C.c_int, [_vp] * 5 + [C.c_float] + [_sz] * 4 + [_vp] * 3),
    "cfops_linear_backward": (C.c_int, [_vp] * 7 + [C.c_float] + [_sz] * 4 + [_vp] * 5),
    "cfops_adamw_update": (C.c_int, [_vp] * 5 + [_sz, C.c_uint64] + [C.c_float] * 5 + [_vp]),
    # include/cfio.h
    "cfio_bf16_to_f32": (C.c_int, [_vp, _vp, _vp, _sz, _vp]),
    "cfio_f16_to_f32": (C.c_int, [_vp, _vp, _vp, _sz, _vp]),
    "cfio_st_open": (C.c_int, [C.c_char_p, C.POINTER(_vp), C.c_char_p, _sz]),
    "cfio_st_close": (C.c_int, [_vp]),
    "cfio_st_count": (_sz, [_vp]),
    "cfio_st_tensor": (C.c_int, [_vp, _sz, C.POINTER(C.c_char_p), C.POINTER(C.c_int), C.POINTER(_sz),
                                 C.POINTER(C.POINTER(_sz)), C.POINTER(_sz)]),
    "cfio_st_find": (C.c_longlong, [_vp, C.c_char_p]),
    "cfio_st_meta_count": (_sz, [_vp]),
    "cfio_st_meta": (C.c_int, [_vp, _sz, C.POINTER(C.c_char_p), C.POINTER(C.c_char_p)]),
    "cfio_dtype_name": (C.c_char_p, [C.c_int]),
    "cfio_st_read_f32": (C.c_int, [_vp, _vp, _sz, C.POINTER(_sz), C.POINTER(_vp), _vp]),
    "cfio_st_write": (C.c_int, [_vp, C.c_char_p, _sz, C.POINTER(C.c_char_p), C.POINTER(_sz),
                                C.POINTER(C.POINTER(_sz)), C.POINTER(_vp), _sz, C.POINTER(C.c_char_p),
                                C.POINTER(C.c_char_p), _vp]),
    "cfio_set_chunk_bytes": (C.c_int, [_vp, _sz]),
}

# dtype codes of include/cfio.h (the safetensors crate's Dtype order)
CFIO_DTYPES = ["BOOL", "F4", "F6_E2M3", "F6_E3M2", "U8", "I8", "F8_E5M2", "F8_E4M3", "F8_E8M0", "I16", "U16", "F16",
               "BF16", "I32", "U32", "F32", "C64", "F64", "I64", "U64"]

# matmul kinds of cfops_matmul (include/cfops.h)
NN, NT, TN = 0, 1, 2
IGNORE_INDEX = -100

_lib = None
_lock = threading.Lock()


class CfattnError(RuntimeError):
    """A failed libcfattn call; `code` is the CFATTN_ERR_* status."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"cfattn error {code}: {msg}")
        self.code = code


class ShapeError(CfattnError, AssertionError):
    """Where the reference panics on an assert (attention.rs:35-38, 55-58,
    155-158), the library returns CFATTN_ERR_SHAPE and this is raised."""


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise ImportError(f"{LIB_PATH} is missing: run `python -m cpuforge_amd.build` first "
                                      "(there is no CPU fallback)")
                # PyTorch-ROCm bundles its own HIP runtime with the same soname
                # (libamdhip64.so.7) as /opt/rocm's.  Two runtimes in one
                # process cannot both open the GPU, so when torch is present it
                # is loaded first and libcfattn.so binds to its runtime.
                try:
                    import torch  # noqa: F401
                except ImportError:
                    pass
                L = C.CDLL(LIB_PATH)
                for name, (res, args) in SIGNATURES.items():
                    fn = getattr(L, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = L
    return _lib


def check(rc: int, ctx=None) -> None:
    if rc == OK:
        return
    msg = ""
    if ctx is not None:
        raw = lib().cfattn_last_error(ctx)
        msg = raw.decode() if raw else ""
    if rc == ERR_SHAPE:
        raise ShapeError(rc, msg)
    raise CfattnError(rc, msg)
