"""bench.py contract pieces that run without a GPU."""
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def test_cpu_baseline_leg_runs():
    import bench

    r = bench.cpu_baseline(seconds=0.05)
    assert r["kind"] == "port" and r["unit"] == "us/layer" and r["value"] > 0 and r["cores"] >= 1
    json.dumps(r)


def test_more_than_one_gpu_exits_with_message():
    p = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert p.returncode != 0 and "one GPU" in p.stderr


def test_committed_traffic_summary_parses():
    import bench

    t = bench.committed_traffic()
    assert t is None or t > 0
