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


def test_cpu_baseline_timer_spends_its_budget_and_takes_the_median():
    import bench
    durations = iter([0.03, 0.01, 0.02] + [0.01] * 100)
    calls = []

    def fn():
        calls.append(1)
        time.sleep(next(durations))

    t, runs, total = bench._cpu_time(fn, min_reps=3, budget_s=0.05)
    assert runs >= 3 and total >= 0.05
    assert len(calls) == runs + 1  # one warm-up call
    assert 0.009 < t < 0.03
