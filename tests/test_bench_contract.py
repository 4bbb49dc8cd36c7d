"""CPU: the parts of bench.py's output contract that need no GPU -- the refusal of --gpus > 1,
the per-kernel accounting helpers and the roofline object."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


@pytest.mark.parametrize("n", [2, 8])
def test_more_than_one_gpu_is_refused_before_any_device_work(n):
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", str(n)], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "exactly one GPU" in r.stderr and f"asked for {n}" in r.stderr
    assert r.stdout == ""


def test_unlaunched_kernels_report_null_and_are_never_dominant():
    kms = bench.launched([0.66, 0.005, 0.029], [True, False, True])
    assert kms == [0.66, None, 0.029]
    assert bench.dominant(kms) == 0
    assert bench.dominant(bench.launched([0.005, 0.88, 0.001], [False, True, False])) == 1


def test_roofline_counts_compulsory_bytes_only():
    # R-MAT 2^20, K = 128: 6 B per entry + row pointers + B once + C once
    m = n = 1 << 20
    nnz, K = 31_409_164, 128
    alg = 6 * nnz + 4 * (m + 1) + 2 * n * K + 4 * m * K
    assert alg == 997_955_660
    roof = bench.roofline(alg, 116_935_568, 0.6633, "spmm_tasks", ["spmm_tasks", "spmm_mfma_win", "spmm_fixup"],
                          [0.6633, None, 0.0291], "rmat20_k128")
    assert roof["alg_bytes"] == alg and roof["impl_bytes"] == 116_935_568
    assert roof["achieved"] == pytest.approx(alg / 0.6633e-3 / 1e9, abs=0.1)
    assert roof["frac"] == pytest.approx(roof["achieved"] / 8000.0, abs=1e-4)
    assert roof["kernel_ms_all"] == {"spmm_tasks": 0.6633, "spmm_mfma_win": None, "spmm_fixup": 0.0291}
    # the traffic figure comes from the stored counter run and says so
    with open(os.path.join(ROOT, "profiles", "spmm_tasks_rmat20_k128_pmc.json")) as f:
        stored = json.load(f)
    assert roof["traffic"] == stored["hbm_bytes_per_launch"]
    assert "not this one" in roof["traffic_source"]


def test_workloads_without_a_counter_run_have_no_traffic():
    traffic, source = bench.load_traffic("spmm_tasks", "no_such_workload")
    assert traffic is None and source is None
