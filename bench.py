#!/usr/bin/env python3
"""Benchmark of the attention hot path on one MI355X.

Headline metric: paged decode HBM GB/s + prefill TFLOP/s.
  value    : paged var-len GQA decode (config 3: B=32, Hq=32, Hkv=8, D=128,
             page 16, lengths U[256, 8192]) -- algorithmic HBM bytes per step
             / wall time per step, inputs resident in HBM.
  prefill  : causal GQA prefill (config 0: Q [8,64,1024,64], K/V [8,16,1024,64])
             -- algorithmic FLOPs / wall time per step.
A step is one call of the drop-in entry point on the synthetic batch.  Each
leg carries a roofline object for its dominant kernel (split-KV decode kernel,
prefill kernel): algorithmic bytes (FLOPs) per launch / the kernel's mean
duration from a HIP event pair that the runtime stamps with the dispatch's own
start and end (hipExtLaunchKernel on the launch stream), against MI355X's
published peak (8 TB/s HBM, 2.5 PFLOP/s dense fp16).  `traffic` is the HBM
bytes per launch from the committed rocprofv3 counter summary in profiles/.  The CPU
baseline is the repository's CPU restatement of the reference's naive path
(oracle/, fp32) timed on a bounded sample on this host.

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1]
Prints one JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2500.0
PROFILES = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles")


def _traffic(summary):
    """HBM bytes per launch of a kernel, from its committed counter summary.

    The summary records two rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE) of
    this script, scaled by what the counters read for a device copy of known
    size; it holds one line ``traffic_bytes_per_launch = N``.  None if absent.
    """
    path = os.path.join(PROFILES, summary)
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch"):
                    return float(line.split("=")[1])
    except OSError:
        pass
    return None


def _parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true",
                    help="skip the CPU baseline legs (for profiler runs)")
    ap.add_argument("--only", choices=["all", "paged", "prefill"], default="all")
    ap.add_argument("--chunk", type=int, default=0, help="split-KV chunk tokens (0 = auto)")
    ap.add_argument("--copy-calibration-mb", type=int, default=0,
                    help="also run one device-to-device copy of this many MiB "
                         "(reference kernel for HBM counter scaling)")
    return ap.parse_args()


def _log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _time_steps(fn, steps, warmup):
    """Wall time per step, and mean dominant-kernel time per step.

    The step time comes from a loop with nothing but the steps in it; the
    kernel time from a second loop of the same steps in which the library
    launches its dominant kernel with a HIP event pair stamped on the dispatch.
    """
    import torch
    from attention_kernel_triton_amd import _native
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    with _native.kernel_timer() as kt:
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
    if kt.launches != steps:
        raise RuntimeError(f"expected {steps} timed launches, got {kt.launches}")
    return wall / steps, kt.total_ms / 1e3 / steps


def _cpu_time(fn, reps):
    fn()  # warm-up
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    return ts[len(ts) // 2]


def bench_paged(args):
    import torch
    from attention_kernel_triton_amd import _ops
    from attention_kernel_triton_amd import synthetic as syn
    dev = torch.device("cuda:0")
    _log("generating config 3 (paged decode)")
    cfg = syn.paged_config()
    p = cfg.to(dev)
    nbytes = cfg.bytes()

    def step():
        return _ops.decode_paged(p.q, p.pool, p.indptr, p.indices, p.last_len,
                                 chunk_tokens=args.chunk)

    _log("timing paged decode")
    t_step, t_kern = _time_steps(step, args.steps, args.warmup)
    out = {
        "value": nbytes / t_step / 1e9,
        "ms_per_step": t_step * 1e3,
        "bytes_per_step": nbytes,
        "roofline": {"bound": "hbm", "achieved": nbytes / t_kern / 1e9, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": nbytes / t_kern / 1e9 / HBM_PEAK_GBS,
                     "traffic": _traffic("split_kernel_paged_decode_config3.md"),
                     "kernel": "split_kernel<128,4,kModePaged>",
                     "kernel_us": t_kern * 1e6},
        "tokens": sum(cfg.lens),
    }
    if not args.no_cpu_baseline:
        from oracle import naive
        _log("CPU baseline: oracle naive_paged_attention (fp32) on config 3")
        torch.set_num_threads(os.cpu_count() or 1)
        reps = 3
        t = _cpu_time(lambda: naive.naive_paged_attention(
            cfg.q, cfg.pool, cfg.indptr, cfg.indices, cfg.last_len, dtype=torch.float32), reps)
        out["cpu_baseline"] = {"value": nbytes / t / 1e9, "unit": "GB/s",
                               "cores": torch.get_num_threads(), "kind": "port",
                               "sample": f"full config 3 batch, median of {reps} runs "
                                         f"({t * 1e3:.0f} ms each), fp32 torch on CPU"}
    del p
    return out


def bench_prefill(args):
    import torch
    from attention_kernel_triton_amd import prefill_flash_attention as pre
    from attention_kernel_triton_amd import synthetic as syn
    dev = torch.device("cuda:0")
    _log("generating config 0 (causal prefill)")
    cfg = syn.prefill_config(0)
    c = cfg.to(dev)
    flops = cfg.flops()

    def step():
        return pre.flash_attention_prefill(c.Q, c.K, c.V, True, c.scale, c.group)

    _log("timing prefill")
    t_step, t_kern = _time_steps(step, args.steps, args.warmup)
    out = {
        "value": flops / t_step / 1e12,
        "unit": "TFLOP/s",
        "ms_per_step": t_step * 1e3,
        "flops_per_step": flops,
        "roofline": {"bound": "mfma", "achieved": flops / t_kern / 1e12, "peak": FP16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": flops / t_kern / 1e12 / FP16_PEAK_TFLOPS,
                     "traffic": _traffic("prefill_kernel_causal_config0.md"),
                     "kernel": "prefill_kernel<64,causal>",
                     "kernel_us": t_kern * 1e6},
    }
    if not args.no_cpu_baseline:
        from oracle import naive
        _log("CPU baseline: oracle prefill (fp32) on 2 of 8 batches of config 0")
        torch.set_num_threads(os.cpu_count() or 1)
        nb = 2
        reps = 3
        t = _cpu_time(lambda: naive.prefill(cfg.Q[:nb], cfg.K[:nb], cfg.V[:nb], True, cfg.scale,
                                            cfg.group, dtype=torch.float32), reps)
        out["cpu_baseline"] = {"value": flops * nb / 8 / t / 1e12, "unit": "TFLOP/s",
                               "cores": torch.get_num_threads(), "kind": "port",
                               "sample": f"2 of 8 batches of config 0, median of {reps} runs "
                                         f"({t * 1e3:.0f} ms each), fp32 torch on CPU"}
    return out


def copy_calibration(mb):
    import torch
    n = mb * (1 << 20)
    a = torch.empty(n, dtype=torch.uint8, device="cuda:0")
    b = torch.empty_like(a)
    a.fill_(1)
    torch.cuda.synchronize()
    b.copy_(a)
    torch.cuda.synchronize()
    _log(f"copy calibration: {n} bytes read, {n} bytes written")


def main():
    args = _parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; --gpus must be 1 "
                                   "(multi-GPU sharding is a design note, not a measured path)"}))
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no ROCm GPU visible"}))
        sys.exit(1)
    from attention_kernel_triton_amd import _native
    _native.load()
    res = {"metric": "paged decode HBM GB/s + prefill TFLOP/s (fp16, % MI355X peak), 1 GPU",
           "value": None, "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": None, "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "fp16 (fp32 accumulate)",
           "data": "synthetic (seeded N(0,1) fp16)",
           "config": {"workload": "paged var-len GQA decode, config 3", "batch": 32,
                      "num_q_heads": 32, "num_kv_heads": 8, "head_dim": 128, "page_size": 16,
                      "seq_len": "U[256, 8192]", "parallelism": "none (1 GPU)"}}
    if args.only in ("all", "paged"):
        pg = bench_paged(args)
        res["value"] = pg.pop("value")
        res["ms_per_step"] = pg.pop("ms_per_step")
        res["roofline"] = pg.pop("roofline")
        if "cpu_baseline" in pg:
            res["cpu_baseline"] = pg.pop("cpu_baseline")
        res["config"].update(pg)
        torch.cuda.empty_cache()
    if args.only in ("all", "prefill"):
        pf = bench_prefill(args)
        pf["config"] = {"workload": "causal GQA prefill, config 0", "batch": 8,
                        "num_q_heads": 64, "num_kv_heads": 16, "seq_len": 1024, "head_dim": 64}
        res["prefill"] = pf
        if res["value"] is None:
            res.update({"value": pf["value"], "unit": pf["unit"],
                        "ms_per_step": pf["ms_per_step"], "roofline": pf["roofline"]})
    if args.copy_calibration_mb:
        copy_calibration(args.copy_calibration_mb)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
