"""The performance suite and its A/B gate (piton_amd/perf_suite.py, piton_amd/ab.py; the
reference's perf/suite.py and perf/ab.py): the verdict rule on made-up results, the suite's
cases on the GPU, and an A/A run of the gate."""
import numpy as np
import pytest

from piton_amd import ab, perf_suite


def result(name, speedup, outputs="identical"):
    return dict(name=name, a_us=100.0, b_us=100.0 / speedup, speedup=speedup, outputs=outputs, errors=None)


def test_verdict_follows_the_reference_rule():
    assert ab.verdict([result("copy", 1.05), result("exp", 1.0)]) == (True, "faster: copy 1.050x")
    ok, why = ab.verdict([result("copy", 1.05), result("exp", 0.97)])
    assert not ok and why.startswith("slower: exp")
    ok, why = ab.verdict([result("copy", 1.05, "wrong")])
    assert not ok and why == "wrong: copy"
    ok, why = ab.verdict([result("copy", 1.01), result("exp", 0.99)])
    assert not ok and "no target" in why
    ok, why = ab.verdict([result("copy", 1.05), result("exp", 1.0)], targets=["exp"])
    assert not ok and "no target" in why


def test_compare_classifies_outputs():
    rows_a = {"copy": dict(ok=True), "exp": dict(ok=True), "log": dict(ok=True)}
    rows_b = {"copy": dict(ok=True), "exp": dict(ok=True), "log": dict(ok=False, error="3 outside tolerance")}
    sa = {"copy": np.arange(4.0), "exp": np.ones(3), "log": np.ones(2)}
    sb = {"copy": np.arange(4.0), "exp": np.ones(3) + 1e-7, "log": np.ones(2)}
    t = {"copy": 10.0, "exp": 10.0, "log": 10.0}
    res = {r["name"]: r for r in ab.compare(rows_a, rows_b, sa, sb, t, t)}
    assert res["copy"]["outputs"] == "identical"
    assert res["exp"]["outputs"] == "within tolerance"
    assert res["log"]["outputs"] == "wrong"


def test_suite_covers_the_reference_primitives():
    want = {"copy", "mul", "fma", "scaled_relu", "exp", "exp2", "log", "log2", "recip", "rsqrt", "sqrt", "idiv",
            "row_sum", "row_max", "transpose", "softmax", "matmul", "dense_relu"}
    assert want <= set(perf_suite.CASES)


@pytest.mark.gpu
def test_every_case_is_correct_at_reduced_sizes():
    rows, samples = perf_suite.run_cases(list(perf_suite.CASES), small=True, iters=2)
    bad = [(r["name"], r["error"]) for r in rows if not r["ok"]]
    assert not bad, bad
    assert set(samples) == set(perf_suite.CASES)
    assert all(r["us"] > 0 for r in rows)


@pytest.mark.gpu
def test_ab_gate_on_the_same_build_gives_identical_outputs(tmp_path):
    from piton_amd.runtime import mi355x
    lib = mi355x.library_path()
    ab.main(["--a", lib, "--b", lib, "copy", "exp", "softmax", "matmul", "--small", "--rounds", "1",
             "--json", str(tmp_path / "ab.json")])
    import json
    res = json.load(open(tmp_path / "ab.json"))
    assert all(r["outputs"] == "identical" for r in res["results"]), res
