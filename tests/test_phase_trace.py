"""The phase-trace diagnostics on the CPU: the per-launch summary arithmetic on synthetic
stamps, and the product library carries no trace entry points (they exist only in the
separately built traced copy)."""
import os
import subprocess

import pytest

from piton_amd import build, phase_trace


def test_summary_of_synthetic_launches():
    # three launches of two waves; stamps in 10 ns ticks: start, first data, end
    launches = [
        [(0, 100, 500), (10, 120, 520)],
        [(700, 790, 1300), (705, 800, 1310)],
        [(1500, 1600, 2000), (1510, 1620, 2010)],
    ]
    m = phase_trace._summary(launches, 3, nbytes=10_000_000)
    # only the middle launch counts: t0 = 700
    assert m["waves"] == 2
    assert m["last_wave_start"] == pytest.approx(0.05)
    assert m["first_data"] == pytest.approx(0.90)
    assert m["wave_wait"] == pytest.approx(0.925)
    assert m["end"] == pytest.approx(6.10)
    assert m["gap_to_next"] == pytest.approx(1.90)
    assert m["stream_tbs"] == pytest.approx(10e6 / ((6.10 - 0.90) * 1e-6) / 1e12)


def test_product_library_has_no_trace_entries():
    if not os.path.exists(build.LIB):
        pytest.skip("library not built")
    syms = subprocess.run(["nm", "-D", build.LIB], capture_output=True, text=True).stdout
    assert "piton_mi355x_matmul" in syms
    assert "piton_phase_" not in syms
