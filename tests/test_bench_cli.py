"""bench.py's contract on the CPU: more than one GPU is refused with a
message before any GPU work, and the CPU baseline (the numpy oracle, a
bounded sample) reports the fields the bench line carries."""
import os
import subprocess
import sys

from conftest import REPO


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2", "--steps", "1"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_cpu_baseline_fields():
    sys.path.insert(0, REPO)
    try:
        import bench
    finally:
        sys.path.remove(REPO)
    cb = bench.cpu_baseline(budget_s=0.2)
    assert cb["unit"] == "tok/s" and cb["kind"] == "port" and cb["value"] > 0 and cb["cores"] >= 1
    assert "configuration 1" in cb["sample"]
    assert cb["one_thread"]["cores"] == 1 and cb["one_thread"]["value"] > 0
    assert cb["prefill"]["value"] > 0 and "configuration 2" in cb["prefill"]["sample"]
