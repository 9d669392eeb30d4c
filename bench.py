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
    ap.add_argument("--only", choices=["all", "headline", "paged", "prefill", "legs"],
                    default="all",
                    help="all = paged (headline) + prefill + the other rows' legs; "
                         "headline = paged + prefill")
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


def _cpu_threads():
    """The host threads the CPU baseline uses: the OMP_NUM_THREADS share when the
    environment sets one (the GPU boxes do), else every core."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    return int(env) if env.isdigit() and int(env) > 0 else (os.cpu_count() or 1)


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


CPU_BUDGET_S = 10.0  # CPU work per baseline: at least 3 runs, then runs until this is spent


def _cpu_time(fn, min_reps=3, budget_s=CPU_BUDGET_S):
    """Median wall time of fn over runs totalling about budget_s (after a warm-up);
    returns (median seconds, runs, total seconds)."""
    fn()  # warm-up
    ts = []
    while len(ts) < min_reps or sum(ts) < budget_s:
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    total = sum(ts)
    ts.sort()
    return ts[len(ts) // 2], len(ts), total


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
        torch.set_num_threads(_cpu_threads())
        t, reps, total = _cpu_time(lambda: naive.naive_paged_attention(
            cfg.q, cfg.pool, cfg.indptr, cfg.indices, cfg.last_len, dtype=torch.float32))
        out["cpu_baseline"] = {"value": nbytes / t / 1e9, "unit": "GB/s",
                               "cores": torch.get_num_threads(), "kind": "port",
                               "sample": f"full config 3 batch, median of {reps} runs "
                                         f"({t * 1e3:.0f} ms each, {total:.1f} s in all), "
                                         f"fp32 torch on "
                                         f"{torch.get_num_threads()} threads of {_cpu_model()}"}
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
        torch.set_num_threads(_cpu_threads())
        nb = 2
        t, reps, total = _cpu_time(lambda: naive.prefill(
            cfg.Q[:nb], cfg.K[:nb], cfg.V[:nb], True, cfg.scale, cfg.group, dtype=torch.float32))
        out["cpu_baseline"] = {"value": flops * nb / 8 / t / 1e12, "unit": "TFLOP/s",
                               "cores": torch.get_num_threads(), "kind": "port",
                               "sample": f"2 of 8 batches of config 0, median of {reps} runs "
                                         f"({t * 1e3:.0f} ms each, {total:.1f} s in all), "
                                         f"fp32 torch on "
                                         f"{torch.get_num_threads()} threads of {_cpu_model()}"}
    return out


# --------------------------------------------------------------------------- other rows
# Secondary legs: one per remaining hot-path row, each with the roofline of its
# dominant kernel.  Inputs are rotated over several copies (or kept-index sets)
# whose total exceeds the 256 MB Infinity Cache, so HBM-bound legs are not
# measured out of the cache.
MALL_BYTES = 256 << 20


def _copies(nbytes_one, floor=2):
    return max(floor, -(-2 * MALL_BYTES // max(1, nbytes_one)))


def _leg(name, fn_list, work, unit, bound, kernel, args, note=""):
    """Time a leg that cycles through fn_list; work = algorithmic bytes or FLOPs per step."""
    i = [0]

    def step():
        fn_list[i[0] % len(fn_list)]()
        i[0] += 1

    steps = max(args.steps, len(fn_list))
    t_step, t_kern = _time_steps(step, steps, max(args.warmup, len(fn_list)))
    scale = 1e9 if unit == "GB/s" else 1e12
    peak = HBM_PEAK_GBS if bound == "hbm" else FP16_PEAK_TFLOPS
    out = {"value": work / t_step / scale, "unit": unit, "ms_per_step": t_step * 1e3,
           "work_per_step": work,
           "roofline": {"bound": bound, "achieved": work / t_kern / scale, "peak": peak,
                        "unit": unit, "frac": work / t_kern / scale / peak, "traffic": None,
                        "kernel": kernel, "kernel_us": t_kern * 1e6}}
    if note:
        out["note"] = note
    _log(f"{name}: {out['value']:.1f} {unit} (kernel {t_kern * 1e6:.1f} us, "
         f"frac {out['roofline']['frac']:.3f})")
    return out


def _sparse_bytes(ind, nnz, group, D, qo_rows):
    """Unique K/V rows per (batch, kv head) x 4D bytes + indices + q/o/lse."""
    import torch
    B, H, _ = ind.shape
    rows = 0
    for b in range(B):
        for g0 in range(0, H, group):
            sets = [ind[b, h, : int(nnz[b, h, 0])] for h in range(g0, g0 + group)]
            rows += int(torch.unique(torch.cat(sets)).numel())
    return rows * D * 2 * 2 + 4 * int(nnz.sum()) + qo_rows * (2 * D * 2 + 4)


def bench_legs(args):
    import torch
    from attention_kernel_triton_amd import _ops, kept_index
    from attention_kernel_triton_amd import synthetic as syn
    from attention_kernel_triton_amd.paged_kv import append_paged_kv
    from oracle.kept import kept_from_uniform
    dev = torch.device("cuda:0")
    legs = {}

    _log("leg: var-len causal prefill, config 1")
    c1 = syn.prefill_config(1)
    d1 = c1.to(dev)
    legs["prefill_varlen_config1"] = _leg(
        "config 1", [lambda: _ops.prefill(d1.Q, d1.K, d1.V, True, d1.scale, varlen=d1.varlen)],
        c1.flops(), "TFLOP/s", "mfma", "prefill_kernel<64,causal,varlen>", args,
        "FLOPs over each sequence's valid causal pairs")
    del d1
    torch.cuda.empty_cache()

    _log("leg: dense GQA decode, config 2")
    c2 = syn.decode_config()
    n2 = _copies(c2.bytes())
    d2 = [c2.to(dev) for _ in range(n2)]
    legs["decode_config2"] = _leg(
        "config 2", [lambda d=d: _ops.decode(d.q, d.K, d.V, d.scale) for d in d2], c2.bytes(),
        "GB/s", "hbm", "split_kernel<64,4,kModeDense>", args,
        f"inputs rotated over {n2} copies")
    del d2
    torch.cuda.empty_cache()

    _log("leg: sparse-token decode, config 4a")
    s4 = syn.sparse_config()
    B, H, N = s4.uniform.shape
    ind, nnz = kept_from_uniform(s4.uniform.reshape(B * H, N).numpy(), s4.kept_ratio, s4.l_max,
                                 s4.row_len.reshape(-1).numpy())
    ind = torch.from_numpy(ind).reshape(B, H, -1)
    nnz = torch.from_numpy(nnz).reshape(B, H, 1)
    b4 = _sparse_bytes(ind, nnz, s4.group, 128, B * H)
    n4 = _copies(s4.K.numel() * 4)
    kv4 = [(s4.K.to(dev), s4.V.to(dev)) for _ in range(n4)]
    q4, i4, z4 = s4.q.to(dev), ind.to(dev), nnz.to(dev)
    legs["sparse_config4a"] = _leg(
        "config 4a", [lambda kv=kv: _ops.sparse_decode(q4, kv[0], kv[1], i4, z4, s4.scale,
                                                      return_lse=True) for kv in kv4],
        b4, "GB/s", "hbm", "split_kernel<128,1,kModeSparseDense>", args,
        f"O + LSE; K/V rotated over {n4} copies; bytes = unique kept rows per kv head")
    del kv4
    torch.cuda.empty_cache()

    _log("leg: sparse paged + MagicPIG decode, config 4b")
    s5 = syn.sparse_paged_config()
    p5 = s5.paged.to(dev)
    B, H, N = s5.uniform.shape
    sets = []
    nsets = 0
    b5 = 0
    gen = torch.Generator(device=dev).manual_seed(7)
    while True:  # distinct kept-index sets until their gathered rows exceed 2x the cache
        u = torch.rand((B, H, N), generator=gen, device=dev)
        ind5, nnz5 = kept_index.select_kept(s5.l_max, uniform=u, kept_ratio=s5.kept_ratio,
                                            row_len=s5.row_len.to(dev))
        sets.append((ind5, nnz5))
        nsets += 1
        if nsets == 1:
            b5 = _sparse_bytes(ind5.cpu(), nnz5.cpu(), s5.group, 256, B * H) + \
                4 * (p5.indices.numel() + p5.indptr.numel())
        if nsets * b5 >= 2 * MALL_BYTES or nsets >= 64:
            break
    legs["sparse_paged_config4b"] = _leg(
        "config 4b", [lambda st=st: _ops.sparse_decode_paged(p5.q, p5.pool, p5.indptr, p5.indices,
                                                             st[0], st[1], return_lse=True)
                      for st in sets],
        b5, "GB/s", "hbm", "split_kernel<256,1,kModeSparsePaged>", args,
        f"O + LSE; {nsets} kept-index sets rotated")
    lk, ll = s5.lsh_k.to(dev), s5.lsh_l.to(dev)
    legs["magicpig_config4b"] = _leg(
        "config 4b MagicPIG", [lambda st=st: _ops.sparse_decode_paged(
            p5.q, p5.pool, p5.indptr, p5.indices, st[0], st[1], return_lse=True, lsh_k=lk,
            lsh_l=ll) for st in sets],
        b5, "GB/s", "hbm", "split_kernel<256,1,kModeSparsePaged,magicpig>", args,
        f"O + LSE with norm; {nsets} kept-index sets rotated")
    del p5, sets
    torch.cuda.empty_cache()

    _log("leg: LSE merge of partial states")
    rows, D, parts = 8 * 64 * 1024, 64, 2
    mo = torch.randn(parts, rows, D, device=dev).half()
    ml = torch.randn(parts, rows, device=dev)
    mb = parts * rows * (D * 2 + 4) + rows * (D * 2 + 4)
    legs["merge_states"] = _leg(
        "merge", [lambda: _ops.merge_states(mo, ml)], mb, "GB/s", "hbm", "merge_kernel<f16,f16>",
        args, f"{parts} fp16 parts of [{rows}, {D}] (config 0's rows) -> fp16")
    del mo, ml
    torch.cuda.empty_cache()

    _log("leg: paged KV append (prefill-sized)")
    Bq, Hkv, D, page, T = 32, 8, 128, 16, 1024
    pages = Bq * T // page
    pool = torch.zeros((pages, 2, Hkv, page, D), dtype=torch.float16, device=dev)
    perm = torch.randperm(pages, generator=torch.Generator().manual_seed(3)).to(torch.int32)
    indptr = torch.arange(0, pages + 1, T // page, dtype=torch.int32)
    last = torch.full((Bq,), page, dtype=torch.int32)
    ap = torch.arange(0, Bq * T + 1, T, dtype=torch.int32)
    kn = torch.randn(Bq * T, Hkv, D, device=dev).half()
    vn = torch.randn(Bq * T, Hkv, D, device=dev).half()
    t_dev = [x.to(dev) for x in (ap, indptr, perm, last)]
    legs["paged_append"] = _leg(
        "append", [lambda: append_paged_kv(kn, vn, t_dev[0], pool, t_dev[1], t_dev[2], t_dev[3])],
        8 * Bq * T * Hkv * D + 4 * (pages + 2 * Bq + 2), "GB/s", "hbm", "paged_append_kernel",
        args, f"{Bq} sequences x {T} tokens into random pages")
    return legs


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
    if args.only in ("all", "headline", "paged"):
        pg = bench_paged(args)
        res["value"] = pg.pop("value")
        res["ms_per_step"] = pg.pop("ms_per_step")
        res["roofline"] = pg.pop("roofline")
        if "cpu_baseline" in pg:
            res["cpu_baseline"] = pg.pop("cpu_baseline")
        res["config"].update(pg)
        torch.cuda.empty_cache()
    if args.only in ("all", "headline", "prefill"):
        pf = bench_prefill(args)
        pf["config"] = {"workload": "causal GQA prefill, config 0", "batch": 8,
                        "num_q_heads": 64, "num_kv_heads": 16, "seq_len": 1024, "head_dim": 64}
        res["prefill"] = pf
        if res["value"] is None:
            res.update({"value": pf["value"], "unit": pf["unit"],
                        "ms_per_step": pf["ms_per_step"], "roofline": pf["roofline"]})
    if args.only in ("all", "legs"):
        res["legs"] = bench_legs(args)
    if args.copy_calibration_mb:
        copy_calibration(args.copy_calibration_mb)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
