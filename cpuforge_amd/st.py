"""safetensors files read into and written from device tensors
(crates/io/src/st.rs, crates/io/src/dtype.rs) through include/cfio.h.

    read_safetensors(path)          st.rs:19-45  -> Loaded(tensors, metadata)
    write_safetensors(path, ts, m)  st.rs:48-64  (temp file, then rename)
    bf16_to_f32 / f16_to_f32        dtype.rs:3-33, on the GPU

Tensors come back as float32 tensors on the context's device (bf16 and f16
files are widened on the GPU); a file's other dtypes are refused as the
reference refuses them.  Where the reference returns `Err(String)` these
functions raise `FormatError` whose text is that string.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass, field

import torch

from . import _lib
from .attention import Context, default_context


class FormatError(RuntimeError):
    """The reference's `Err(String)` of the I/O and state functions."""


@dataclass
class Loaded:
    """st.rs:12-15: every tensor of a file as f32, and its string metadata."""
    tensors: dict = field(default_factory=dict)
    metadata: dict = field(default_factory=dict)


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _device(ctx: Context) -> torch.device:
    return torch.device("cuda", ctx.device)


def _raise(ctx: Context, rc: int) -> None:
    raw = _lib.lib().cfattn_last_error(ctx.handle)
    msg = raw.decode("utf-8", "replace") if raw else f"status {rc}"
    if rc in (_lib.ERR_IO, _lib.ERR_ARG):
        raise FormatError(msg)
    raise _lib.CfattnError(rc, msg)


class StFile:
    """An open safetensors file: its validated header (cfio_st_open)."""

    def __init__(self, path):
        L = _lib.lib()
        self._lib = L
        self.handle = C.c_void_p()
        err = C.create_string_buffer(2048)
        rc = L.cfio_st_open(os.fsencode(path), C.byref(self.handle), err, len(err))
        if rc != _lib.OK:
            self.handle = None
            raise FormatError(err.value.decode("utf-8", "replace"))
        self.path = path

    def close(self):
        if self.handle:
            self._lib.cfio_st_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tensors(self) -> list:
        """[(name, dtype name, shape, numel)] in file order."""
        L, out = self._lib, []
        for i in range(L.cfio_st_count(self.handle)):
            name, dtype, ndim, shape, numel = C.c_char_p(), C.c_int(), C.c_size_t(), C.POINTER(C.c_size_t)(), C.c_size_t()
            _lib.check(L.cfio_st_tensor(self.handle, i, C.byref(name), C.byref(dtype), C.byref(ndim), C.byref(shape),
                                        C.byref(numel)))
            out.append((name.value.decode(), _lib.CFIO_DTYPES[dtype.value], [shape[d] for d in range(ndim.value)],
                        numel.value))
        return out

    def metadata(self) -> dict:
        L, out = self._lib, {}
        for i in range(L.cfio_st_meta_count(self.handle)):
            k, v = C.c_char_p(), C.c_char_p()
            _lib.check(L.cfio_st_meta(self.handle, i, C.byref(k), C.byref(v)))
            out[k.value.decode()] = v.value.decode()
        return out

    def read(self, indices, dsts, ctx: Context) -> None:
        n = len(indices)
        idx = (C.c_size_t * n)(*indices)
        ptrs = (C.c_void_p * n)(*[d.data_ptr() for d in dsts])
        rc = self._lib.cfio_st_read_f32(ctx.handle, self.handle, n, idx, ptrs, _stream())
        if rc != _lib.OK:
            _raise(ctx, rc)


def read_safetensors(path, ctx: Context | None = None) -> Loaded:
    """Every tensor of the file as a float32 device tensor (st.rs:19-45);
    bf16 and f16 tensors are widened on the GPU.  A tensor of any other dtype
    raises "tensor 'NAME' has unsupported dtype I64"."""
    ctx = ctx or default_context()
    with StFile(path) as f:
        infos = f.tensors()
        meta = f.metadata()
        dev = _device(ctx)
        outs = [torch.empty(shape, dtype=torch.float32, device=dev) for _, _, shape, _ in infos]
        f.read(list(range(len(infos))), outs, ctx)
    return Loaded({name: t for (name, _, _, _), t in zip(infos, outs)}, meta)


def write_safetensors(path, tensors, metadata: dict | None = None, ctx: Context | None = None) -> None:
    """st.rs:48-64: f32 tensors [(name, shape, device tensor)] and string
    metadata (an empty map writes no "__metadata__"), to PATH's temp file,
    then renamed into place."""
    ctx = ctx or default_context()
    L = _lib.lib()
    n = len(tensors)
    names = (C.c_char_p * n)()
    ndims = (C.c_size_t * n)()
    shapes = (C.POINTER(C.c_size_t) * n)()
    datas = (C.c_void_p * n)()
    keep = []
    for j, (name, shape, t) in enumerate(tensors):
        shape = [int(s) for s in shape]
        numel = 1
        for s in shape:
            numel *= s
        if not isinstance(t, torch.Tensor) or t.dtype != torch.float32 or not t.is_cuda:
            raise TypeError(f"tensor '{name}' must be a float32 device tensor")
        if t.numel() != numel:
            raise FormatError(f"tensor '{name}': shape {shape} does not match its {t.numel()} values")
        t = t.detach().contiguous()
        arr = (C.c_size_t * max(1, len(shape)))(*shape)
        keep += [t, arr]
        names[j] = name.encode()
        ndims[j] = len(shape)
        shapes[j] = C.cast(arr, C.POINTER(C.c_size_t))
        datas[j] = t.data_ptr() if numel else None
    items = list((metadata or {}).items())
    keys = (C.c_char_p * max(1, len(items)))(*[k.encode() for k, _ in items])
    vals = (C.c_char_p * max(1, len(items)))(*[v.encode() for _, v in items])
    rc = L.cfio_st_write(ctx.handle, os.fsencode(path), n, names, ndims, shapes, datas, len(items), keys, vals,
                         _stream())
    if rc != _lib.OK:
        _raise(ctx, rc)


def _widen(fn: str, src: torch.Tensor, out: torch.Tensor | None, ctx: Context | None) -> torch.Tensor:
    ctx = ctx or default_context()
    if not isinstance(src, torch.Tensor) or not src.is_cuda or src.element_size() != 2 or not src.is_contiguous():
        raise TypeError("src must be a contiguous 16-bit device tensor")
    if out is None:
        out = torch.empty(src.shape, dtype=torch.float32, device=src.device)
    elif out.dtype != torch.float32 or out.numel() != src.numel() or not out.is_contiguous():
        raise ValueError("out must be a contiguous float32 tensor of src's size")
    rc = getattr(_lib.lib(), fn)(ctx.handle, src.data_ptr(), out.data_ptr(), src.numel(), _stream())
    _lib.check(rc, ctx.handle)
    return out


def bf16_to_f32(src: torch.Tensor, out: torch.Tensor | None = None, ctx: Context | None = None) -> torch.Tensor:
    """dtype.rs:3-5 on the GPU: the f32 value of each bf16 pattern of `src`
    (any 16-bit dtype holding the raw patterns)."""
    return _widen("cfio_bf16_to_f32", src, out, ctx)


def f16_to_f32(src: torch.Tensor, out: torch.Tensor | None = None, ctx: Context | None = None) -> torch.Tensor:
    """dtype.rs:7-33 on the GPU: the f32 value of each IEEE half pattern,
    subnormals renormalised, inf / NaN payloads kept."""
    return _widen("cfio_f16_to_f32", src, out, ctx)


def set_chunk_bytes(nbytes: int, ctx: Context | None = None) -> None:
    ctx = ctx or default_context()
    _lib.check(_lib.lib().cfio_set_chunk_bytes(ctx.handle, nbytes), ctx.handle)
