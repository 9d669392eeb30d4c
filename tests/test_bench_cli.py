"""bench.py contract pieces that run without a GPU."""
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    msg = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in msg["error"]


def test_cpu_baseline_spends_its_budget_and_takes_the_median():
    import bench
    durations = iter([0.03, 0.01, 0.02] + [0.01] * 100)
    calls = []

    def fn():
        calls.append(1)
        time.sleep(next(durations))

    class Args:
        no_cpu_baseline = False

    r = bench._cpu_baseline(fn, 1e9, "GB/s", "a sample", 0.05, Args)
    runs = int(r["sample"].split("median of ")[1].split()[0])
    assert runs >= 3 and len(calls) == runs + 1  # one warm-up call
    assert r["kind"] == "port" and r["cores"] >= 1 and r["unit"] == "GB/s"
    assert 1 / 0.03 < r["value"] < 1 / 0.009  # 1 GB over the median run of 10-20 ms
    Args.no_cpu_baseline = True
    assert bench._cpu_baseline(fn, 1e9, "GB/s", "a sample", 0.05, Args) is None
