"""rocprofv3 summaries (piton_amd/profiling.py) on made-up counter files: the calibration scale
factors of the HBM traffic figures and the MFMA occupancy arithmetic."""
import csv
import os

import pytest

from piton_amd import profiling

GEMM = "void piton::gemm_direct_kernel<true, true, false, 4>(piton::GemmArgs)"  # 256 tiles, two a step
ADD = "void piton::add_vec4_kernel(float const*, float const*, float*, long)"
COLS = ["Dispatch_Id", "Kernel_Name", "Grid_Size", "Counter_Name", "Counter_Value", "Start_Timestamp",
        "End_Timestamp"]


def write_pmc(d, rows):
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, "run_counter_collection.csv"), "w", newline="") as f:
        w = csv.DictWriter(f, COLS)
        w.writeheader()
        for r in rows:
            w.writerow(dict(zip(COLS, r)))


def write_trace(d, rows):
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, "run_kernel_trace.csv"), "w", newline="") as f:
        w = csv.DictWriter(f, ["Kernel_Name", "Grid_Size_X", "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        for name, grid, t0, t1 in rows:
            w.writerow(dict(Kernel_Name=name, Grid_Size_X=grid, Start_Timestamp=t0, End_Timestamp=t1))


def test_traffic_is_scaled_by_the_calibration_add(tmp_path):
    kt, fe, wr = (str(tmp_path / n) for n in ("kt", "fetch", "write"))
    # two steps of two launches; the second step's launches take 300 us each
    write_trace(kt, [(GEMM, 65536, 1_000_000 * i, 1_000_000 * i + (200_000 if i < 2 else 300_000))
                     for i in range(4)])
    # the counters read half the calibration add's true bytes: the factors are 2
    write_pmc(fe, [(1, ADD, 64 * 2 ** 20 // 4, "FETCH_SIZE", profiling.CAL_READ / 2 / 1024, 0, 1),
                   (2, GEMM, 65536, "FETCH_SIZE", 100_000.0, 0, 1), (3, GEMM, 65536, "FETCH_SIZE", 120_000.0, 1, 2)])
    write_pmc(wr, [(1, ADD, 64 * 2 ** 20 // 4, "WRITE_SIZE", profiling.CAL_WRITE / 2 / 1024, 0, 1),
                   (2, GEMM, 65536, "WRITE_SIZE", 10_000.0, 0, 1), (3, GEMM, 65536, "WRITE_SIZE", 10_000.0, 1, 2)])
    stats, traffic, ff, fw = profiling.summarize(kt, fe, wr, timed_steps=1)
    assert ff == pytest.approx(2.0) and fw == pytest.approx(2.0)
    t = traffic["matmul 4096^3"]  # per step: two launches of the average dispatch
    assert t["fetch_bytes"] == pytest.approx(2 * 2 * 110_000 * 1024)
    assert t["write_bytes"] == pytest.approx(2 * 2 * 10_000 * 1024)
    assert t["algorithmic_bytes"] == 3 * 4096 * 4096 * 4
    assert stats[0]["calls"] == 4 and stats[0]["avg_ns"] == pytest.approx(250_000)
    steps = profiling.workload_steps(stats)["matmul 4096^3"]
    assert steps["step_ns"] == pytest.approx(2 * 250_000)
    assert steps["timed_step_ns"] == pytest.approx(2 * 300_000)  # the last step's two dispatches


def test_mfma_busy(tmp_path):
    d = str(tmp_path / "pmc")
    # 1 ms at 2.4 GHz on each of 8 XCDs with the 1024 SIMDs' MFMA pipes busy 90 % of it, then
    # 0.5 ms at 60 %: 80 % over both
    gui, gui2 = 8 * 2.4e6, 8 * 1.2e6
    busy, busy2 = 0.9 * 2.4e6 * 1024, 0.6 * 1.2e6 * 1024
    write_pmc(d, [(7, GEMM, 65536, "GRBM_GUI_ACTIVE", gui, 5_000, 1_005_000),
                  (7, GEMM, 65536, "SQ_VALU_MFMA_BUSY_CYCLES", busy, 5_000, 1_005_000),
                  (8, GEMM, 65536, "GRBM_GUI_ACTIVE", gui2, 1_005_000, 1_505_000),
                  (8, GEMM, 65536, "SQ_VALU_MFMA_BUSY_CYCLES", busy2, 1_005_000, 1_505_000),
                  (9, ADD, 1024, "GRBM_GUI_ACTIVE", 100.0, 0, 10)])
    m = profiling.mfma_busy(d)
    assert list(m) == ["matmul 4096^3"]
    assert m["matmul 4096^3"]["mfma_busy"] == pytest.approx(0.8)
    assert m["matmul 4096^3"]["dispatches"] == 2


def test_lds_occupancy(tmp_path):
    d = str(tmp_path / "pmc")
    att = "void piton::(anonymous namespace)::attn_fwd_fast<64, true>(piton::AttnArgs)"
    # 1e5 GUI cycles on each of 8 XCDs; two waves resident on each of the 1024 SIMDs all along
    # (SQ_WAVE_CYCLES counts units of 4 cycles); LDS active 3e7 cycles chip-wide, 1e7 of them
    # bank-conflict cycles: 0.5 conflict cycles per conflict-free cycle
    gui = 8 * 1e5
    waves = 2 * 1e5 * 1024 / 4
    write_pmc(d, [(3, att, 131072, "GRBM_GUI_ACTIVE", gui, 0, 1), (3, att, 131072, "SQ_WAVE_CYCLES", waves, 0, 1),
                  (3, att, 131072, "SQ_LDS_IDX_ACTIVE", 3e7, 0, 1), (3, att, 131072, "SQ_LDS_BANK_CONFLICT", 1e7, 0, 1),
                  (4, ADD, 1024, "GRBM_GUI_ACTIVE", 100.0, 0, 1)])
    m = profiling.lds_occupancy(d)
    assert list(m) == ["attention 32 x 1024 x 64 causal"]
    a = m["attention 32 x 1024 x 64 causal"]
    assert a["kernel"] == "attn_fwd_fast<64, true>" and a["dispatches"] == 1
    assert a["waves_per_simd"] == pytest.approx(2.0)
    assert a["lds_conflict_ratio"] == pytest.approx(0.5)


def test_mfma_busy_per_kernel_cycle_against_a_longer_counter_window(tmp_path):
    """The counter window (GRBM_GUI_ACTIVE) of the second dispatch is 1.25 times its own span:
    per GUI cycle the two dispatches are 2.88 / 3.9 busy, per kernel cycle at 2.4 GHz 0.8."""
    d = str(tmp_path / "pmc")
    gui, gui2 = 8 * 2.4e6, 8 * 1.5e6
    busy, busy2 = 0.9 * 2.4e6 * 1024, 0.6 * 1.2e6 * 1024
    write_pmc(d, [(7, GEMM, 65536, "GRBM_GUI_ACTIVE", gui, 5_000, 1_005_000),
                  (7, GEMM, 65536, "SQ_VALU_MFMA_BUSY_CYCLES", busy, 5_000, 1_005_000),
                  (8, GEMM, 65536, "GRBM_GUI_ACTIVE", gui2, 1_005_000, 1_505_000),
                  (8, GEMM, 65536, "SQ_VALU_MFMA_BUSY_CYCLES", busy2, 1_005_000, 1_505_000)])
    m = profiling.mfma_busy(d)["matmul 4096^3"]
    assert m["mfma_busy"] == pytest.approx(2.88 / 3.9)
    assert m["mfma_busy_kernel"] == pytest.approx(0.8)
    assert m["window_over_kernel"] == pytest.approx(3.9 / 3.6)
    assert m["kernel_us"] == pytest.approx(750.0)
