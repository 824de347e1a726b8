"""bench.py's contract on the CPU: one GPU only (any other --gpus is refused before a GPU is
touched), and the CPU baseline leg (the oracle's matmul over a bounded sample) reports a
positive throughput in the metric's unit with the threads it used, a one-thread figure, numpy's
float64 matmul, and the errors against float64."""
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


@pytest.mark.parametrize("n", ["2", "8"])
def test_more_than_one_gpu_is_refused(n):
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", n], cwd=ROOT,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""  # no JSON line


def test_cpu_baseline_on_a_small_sample():
    import bench
    rng = np.random.default_rng(0)
    a = torch.from_numpy(rng.uniform(-1, 1, (64, 96)).astype(np.float32))
    b = torch.from_numpy(rng.uniform(-1, 1, (96, 80)).astype(np.float32))
    c_rows = (a.numpy()[:16].astype(np.float64) @ b.numpy().astype(np.float64)).astype(np.float32)
    res = bench.cpu_baseline(a, b, budget_s=0.05, c_gpu=c_rows)
    assert res["unit"] == "TFLOP/s" and res["kind"] == "port"
    assert res["value"] > 0 and 1 <= res["cores"] <= 16
    assert "rows of C = A B at 64x80x96" in res["sample"]
    assert res["value_1_thread"] > 0 and res["numpy_fp64"]["value"] > 0
    # float32-rounded float64 products: a few ulp; the oracle's round-toward-zero chain: more
    err = res["err_vs_fp64"]
    assert err["rows"] == 16 and err["gpu"] < 1e-7 and 0 < err["oracle"] < 1e-5
