"""bench.py's contract on the CPU: the metric it reports is BASELINE.json's, it refuses more than one GPU with a
message before touching a GPU, and the HBM traffic summary its roofline reads is complete."""
import json
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))


def test_metric_is_baselines():
    import bench

    assert bench.METRIC == json.loads((ROOT / "BASELINE.json").read_text())["metric"]


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


def test_traffic_summary_matches_its_calibration():
    t = json.loads((ROOT / "profiles" / "hbm_traffic_config2.json").read_text())
    fetch, write = t["fetch_bytes_per_launch"], t["write_bytes_per_launch"]
    assert fetch > 0 and write > 0 and t["fetch_scale"] == 2.0 and t["write_scale"] == 1.0
    # HBM traffic within a few percent of the algorithmic bytes: the gather re-reads nothing
    assert 0.98 < (fetch + write) / t["algorithmic_bytes_per_launch"] < 1.05
