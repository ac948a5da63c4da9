"""The measurement probes of the C ABI (cfattn_probe_mfma_peak,
cfattn_probe_loop): they run, report rates inside what the hardware allows,
and reject bad arguments with the library's error."""
import ctypes as C

import pytest

import cpuforge_amd as cf
from cpuforge_amd import _lib
from cpuforge_amd._lib import CfattnError

pytestmark = pytest.mark.gpu

# MI355X: 2516.6 TFLOP/s dense bf16 at 2.4 GHz; 256 CUs.
SPEC_BF16_TFLOPS = 2516.6


def test_mfma_probe_reports_a_rate_below_the_spec_peak():
    ctx = cf.Context(0)
    try:
        for zeros in (False, True):
            t = ctx.probe_mfma_peak(zeros, 2000)
            print(f"mfma probe zeros={zeros}: {t:.1f} TFLOP/s", flush=True)
            assert 100.0 < t <= SPEC_BF16_TFLOPS * 1.01
        with pytest.raises(CfattnError, match="iters must be positive"):
            ctx.probe_mfma_peak(False, 0)
    finally:
        ctx.close()


def test_loop_probes_report_rates_within_the_hardware_limits():
    ctx = cf.Context(0)
    try:
        lds = ctx.probe_loop("lds", 2000)
        valu = ctx.probe_loop("valu", 2000)
        m16 = ctx.probe_loop("mfma16", 2000)
        print(f"lds {lds / 1e12:.1f} TB/s, valu {valu / 1e12:.1f} T lane-op/s, "
              f"mfma 16x16x32 {m16 / 1e12:.1f} TFLOP/s", flush=True)
        # LDS: at most 256 B per clock per CU at 2.4 GHz on 256 CUs; VALU: at
        # most 64 lanes per clock per SIMD (1024 SIMDs) at 2.4 GHz; bf16 MFMA:
        # the dense spec peak, which both MFMA shapes share.
        assert 1e12 < lds <= 256 * 2.4e9 * 256
        assert 1e12 < valu <= 64 * 2.4e9 * 1024
        assert 100e12 < m16 <= SPEC_BF16_TFLOPS * 1e12 * 1.01
        with pytest.raises(CfattnError, match="unknown probe"):
            out = C.c_double()
            _lib.check(ctx._lib.cfattn_probe_loop(ctx.handle, 7, 10, C.byref(out)), ctx.handle)
        with pytest.raises(CfattnError, match="iters must be positive"):
            ctx.probe_loop("valu", -1)
    finally:
        ctx.close()
