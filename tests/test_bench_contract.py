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


def test_cpu_legs_of_the_other_workloads_on_small_samples():
    """Each workload's CPU leg (the oracle at one and several threads, numpy float64, errors of
    the GPU's output and of the oracle's against float64) on a small synthetic sample, with the
    float64 result standing in for the GPU's."""
    import bench
    from oracle import fp64
    from piton_amd import digits
    rng = np.random.default_rng(1)
    n = 100
    x = (rng.standard_normal((19, n)) * 4).astype(np.float32)
    x[1, 5], x[2, 7], x[3] = np.inf, -np.inf, -np.inf
    sm = bench.cpu_softmax(n, (x, fp64.softmax(x).astype(np.float32)), budget_s=0.05)
    assert sm["oracle"]["value"] > 0 and sm["oracle_1_thread"]["threads"] == 1 and sm["numpy_fp64"]["value"] > 0
    assert sm["err_vs_fp64"]["rows"] == 16 and sm["err_vs_fp64"]["gpu"] < 1e-7 < sm["err_vs_fp64"]["oracle"] < 1e-5
    assert sm["special_rows_match_oracle"]

    q, k, v = (rng.standard_normal((2, 64, 16)).astype(np.float32) for _ in range(3))
    o = np.stack([fp64.attention_reference(q[h], k[h], v[h], True, 0.25) for h in range(2)]).astype(np.float32)
    at = bench.cpu_attention((q, k, v, o), budget_s=0.05)
    assert at["oracle"]["value"] > 0 and at["oracle"]["threads"] <= 2 and at["oracle_1_thread"]["value"] > 0
    assert at["err_vs_fp64"]["gpu"] < 1e-7 < at["err_vs_fp64"]["oracle"] < 1e-5

    layers = digits.he_normal_mlp(seed=1729)
    xd = rng.integers(0, 17, (200, 64)).astype(np.float32)
    h = xd.astype(np.float64)
    for i, (w, b) in enumerate(layers):
        h = fp64.dense(h, w, b, i < 2)
    ml = bench.cpu_mlp((layers, xd, h.astype(np.float32), np.argmax(h, 1).astype(np.int32)), budget_s=0.05)
    assert ml["oracle"]["value"] > 0 and ml["predictions_equal_oracle"] >= 198
    assert ml["err_vs_fp64"]["oracle"] < 1e-5
    assert bench.host_info()["cpu_count"] >= 1
