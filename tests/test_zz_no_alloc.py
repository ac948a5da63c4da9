"""GPU test of cfattn_bwd_noalloc, the backward that allocates nothing (its
delta rows live in the library's fixed per-device scratch array).

Called through the C ABI on device tensors and compared with cfattn_bwd on
the same inputs, two calls in a row with the second on a smaller input (the
shared array keeps the first call's contents):
  - against cfattn_bwd with the stored-dS scratch off (the same kernels):
    bit for bit;
  - against cfattn_bwd with its defaults: bf16 max|a-r|/max|r| <= 2e-2, f32
    max abs <= 1e-4 (the attention parity bars).
A shape whose delta rows exceed the array is refused before any launch.
"""
import ctypes as C

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    import torch

    import cpuforge_amd as cf
    from cpuforge_amd import _lib
    from cpuforge_amd import device as D
    ctx = cf.Context(0)
    yield torch, cf, _lib, D, ctx
    ctx.close()


def _inputs(torch, shape, seed, mode):
    B, S, Hq, Hk, Dh = shape
    tdt = torch.bfloat16 if mode == "bf16" else torch.float32
    return [torch.from_numpy(np.stack([O.rand(S * h * Dh, seed + 16 * b + 2 * i, 1.0) for b in range(B)]))
            .view(B, S, h, Dh).to("cuda").to(tdt) for i, h in enumerate((Hq, Hk, Hk, Hq))]


def _noalloc(env, q, k, v, g, o, lse, init):
    torch, cf, _lib, D, ctx = env
    B, S, Hq, Dh = q.shape
    Hk = k.shape[2]
    dq, dk, dv = (x.clone() for x in init)
    dt = _lib.BF16 if q.dtype == torch.bfloat16 else _lib.F32
    rc = ctx._lib.cfattn_bwd_noalloc(ctx.handle, cf.AttnShape(S, Hq, Hk, Dh).c(), B, dt, g.data_ptr(), q.data_ptr(),
                                     k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(), dq.data_ptr(),
                                     dk.data_ptr(), dv.data_ptr(), torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, ctx.handle)
    return dq, dk, dv


class _DsLimit:
    def __init__(self, ctx, nbytes):
        self.ctx, self.nbytes = ctx, nbytes

    def __enter__(self):
        self.old = self.ctx.ds_limit
        self.ctx.ds_limit = self.nbytes

    def __exit__(self, *exc):
        self.ctx.ds_limit = self.old


@pytest.mark.parametrize("mode", ["bf16", "f32"])
def test_noalloc_backward_matches_bwd(env, mode):
    torch, cf, _lib, D, ctx = env
    # The second shape is smaller: the array still holds the first call's rows.
    for shape in ((2, 700, 8, 2, 128), (1, 130, 4, 1, 64)):
        B, S, Hq, Hk, Dh = shape
        print(f"noalloc {mode} {shape}", flush=True)
        q, k, v, g = _inputs(torch, shape, 1600, mode)
        init = [torch.from_numpy(O.rand(B * S * h * Dh, 1700 + 2 * i, 0.5)).view(B, S, h, Dh).to("cuda")
                for i, h in enumerate((Hq, Hk, Hk))]
        o, lse = D.fwd(q, k, v, ctx=ctx)
        got = _noalloc(env, q, k, v, g, o, lse, init)
        with _DsLimit(ctx, 0):
            same = D.bwd(g, q, k, v, o, lse, *(x.clone() for x in init), ctx=ctx)
        dflt = D.bwd(g, q, k, v, o, lse, *(x.clone() for x in init), ctx=ctx)
        torch.cuda.synchronize()
        for name, a, s_, d_ in zip(("dq", "dk", "dv"), got, same, dflt):
            a, s_, d_ = (x.cpu().numpy().astype(np.float64) for x in (a, s_, d_))
            assert np.array_equal(a, s_), f"{shape} {mode} {name}: differs from cfattn_bwd without stored dS"
            if mode == "bf16":
                e = np.abs(a - d_).max() / np.abs(d_).max()
                assert e <= 2e-2, f"{shape} {name}: {e}"
            else:
                e = np.abs(a - d_).max()
                assert e <= 1e-4, f"{shape} {name}: {e}"


def test_noalloc_refuses_shapes_over_its_scratch(env):
    torch, cf, _lib, D, ctx = env
    # 2^21 + 64 delta rows: refused on the host, before any launch, with
    # valid (unused) device buffers.
    B, S, Hq, Hk, Dh = 1, 65537, 32, 8, 64
    t = torch.zeros(16, dtype=torch.bfloat16, device="cuda")
    f = torch.zeros(16, dtype=torch.float32, device="cuda")
    rc = ctx._lib.cfattn_bwd_noalloc(ctx.handle, cf.AttnShape(S, Hq, Hk, Dh).c(), B, _lib.BF16, t.data_ptr(),
                                     t.data_ptr(), t.data_ptr(), t.data_ptr(), f.data_ptr(), f.data_ptr(),
                                     f.data_ptr(), f.data_ptr(), f.data_ptr(), None)
    assert rc == _lib.ERR_UNSUPPORTED
    assert b"scratch" in ctx._lib.cfattn_last_error(ctx.handle)
