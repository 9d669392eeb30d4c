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


def test_cpu_baseline_runs_five_times_and_two_seconds_and_takes_the_median():
    """The CPU-baseline timer: one warm-up run, then at least 5 runs and at least
    2 s in all, reporting the median run."""
    import bench
    durations = iter([0.05, 0.3, 0.1, 0.2, 0.25, 0.15] + [0.3] * 100)
    calls = []

    def fn():
        calls.append(1)
        time.sleep(next(durations))

    class Args:
        no_cpu_baseline = False

    r = bench._cpu_baseline(fn, 1e9, "GB/s", "a sample", Args)
    runs = int(r["sample"].split("median of ")[1].split()[0])
    assert runs >= 5 and len(calls) == runs + 1  # one warm-up call
    assert runs == 9  # 0.3 + 0.1 + 0.2 + 0.25 + 0.15 + 4 x 0.3 >= 2 s
    assert r["kind"] == "port" and r["cores"] >= 1 and r["unit"] == "GB/s"
    assert 1 / 0.31 < r["value"] < 1 / 0.24  # 1 GB over the median run (0.25-0.3 s)
    assert "the job's CPU share" in r["sample"] and "op order" in r["sample"]
    Args.no_cpu_baseline = True
    assert bench._cpu_baseline(fn, 1e9, "GB/s", "a sample", Args) is None
