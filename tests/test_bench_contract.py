"""bench.py's contract that needs no GPU: the one-GPU refusal of --gpus N > 1, and the
committed rocprofv3 counter summaries that its JSON line quotes (each must carry the
machine-readable bench.* figures, or the line would silently lose traffic and MFMA use)."""
import os
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and "--gpus 2" in r.stderr


@pytest.mark.parametrize("workload", sorted(bench.COUNTERS_FILES))
def test_counter_summaries_carry_bench_figures(workload):
    path = bench.COUNTERS_FILES[workload]
    assert os.path.isfile(path), path
    figs = bench.read_profile_figures(path)
    for key in ("fwd_traffic_bytes", "bwd_traffic_bytes", "fwd_mfma_util_pct", "bwd_mfma_util_pct"):
        assert key in figs, (workload, key)
    assert 0 < figs["fwd_mfma_util_pct"] <= 100 and 0 < figs["bwd_mfma_util_pct"] <= 100
    assert figs["fwd_traffic_bytes"] > 0 and figs["bwd_traffic_bytes"] > 0


def test_read_profile_figures_ignores_prose(tmp_path):
    p = tmp_path / "summary.txt"
    p.write_text("# header\nbench.x: 1.5\nnot a figure: 3\nbench.y_total: 42\n")
    assert bench.read_profile_figures(str(p)) == {"x": 1.5, "y_total": 42.0}
    assert bench.read_profile_figures(str(tmp_path / "missing.txt")) == {}
