"""The sustained-MFMA-rate probe (diagnostics, no reference counterpart): it runs through the
C-ABI, writes every output element, and the rate it implies lies between half the published
fp32 MFMA peak and that peak (one 32x32x2 MFMA per 64 clocks per SIMD, at most 2.4 GHz)."""
import time

import pytest
import torch

from piton_amd.runtime import mi355x as rt

pytestmark = pytest.mark.gpu


def test_probe_rate_is_plausible():
    cus = rt.device_info()["cu_count"]
    wgs, iters = 2 * cus, 400
    out = torch.full((wgs * 256,), float("nan"), device="cuda")
    rt.mfma_probe(out, wgs, iters)  # warm
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(5):
        rt.mfma_probe(out, wgs, iters)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / 5
    rate = wgs * 4 * iters * 32 * 4096 / dt
    assert torch.isfinite(out).all()
    peak = cus * 4 * 64 * 2.4e9  # flops per clock per SIMD x SIMDs x the peak engine clock
    assert 0.5 * peak < rate <= 1.02 * peak, (rate, peak)


def test_probe_rejects_bad_arguments():
    out = torch.empty(256, device="cuda")
    with pytest.raises(ValueError):
        rt.mfma_probe(out, 2, 1)  # out holds one workgroup's 256 floats only
    with pytest.raises(ValueError):
        rt.mfma_probe(out, 1, 0)
