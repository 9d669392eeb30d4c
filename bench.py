#!/usr/bin/env python3
"""Benchmark of the attention hot path on one MI355X.

Headline metric: paged decode HBM GB/s + prefill TFLOP/s.
  value    : paged var-len GQA decode (config 3: B=32, Hq=32, Hkv=8, D=128,
             page 16, lengths U[256, 8192]) -- algorithmic HBM bytes per step
             / wall time per step, inputs resident in HBM.
  prefill  : causal GQA prefill (config 0: Q [8,64,1024,64], K/V [8,16,1024,64])
             -- algorithmic FLOPs / wall time per step.
  legs     : one leg per other hot-path row (configs 1, 2, 4a, 4b, MagicPIG,
             the LSE merge, the paged-KV append and kept-index selection).

A step is one call of the drop-in entry point on the synthetic batch, and every
entry point runs exactly one kernel.  Each leg first repeats its step, untimed,
for --settle-ms of wall time (MI355X's clocks ramp up over tens of
milliseconds of sustained load: config 0's prefill runs 115 us per step after
10 cold steps and 95 us once settled), then does W untimed warm-up steps,
then times K steps bracketed by torch.cuda.synchronize(): ms_per_step is the
wall clock over them, and roofline.kernel_us is the GPU time of the same K
launches from a HIP event pair recorded on the launch stream around them (so
kernel_us <= ms_per_step; it includes the sub-microsecond gaps between
back-to-back launches).  roofline.achieved is algorithmic bytes (FLOPs) per
step / kernel_us against MI355X's published peak (8 TB/s HBM, 2.5 PFLOP/s
dense fp16); roofline.traffic is the HBM bytes per launch from the committed
rocprofv3 counter summary in profiles/, where one exists.  Legs whose working
set is under twice the 256 MB Infinity Cache rotate over copies of their
inputs.  cpu_baseline is the repository's CPU restatement of the reference's
naive path in its fp16 op order (oracle/ref_order.py) timed on a bounded
sample on this host.

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
MALL_BYTES = 256 << 20
PROFILES = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles")


def _traffic(summary, key=None):
    """HBM bytes per launch of a kernel, from its committed counter summary.

    The summary records two rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE) of
    this script, scaled by what the counters read for a device copy of known
    size; it holds a line ``traffic_bytes_per_launch = N`` (or, for a summary
    of several legs, ``traffic_bytes_per_launch[key] = N``).  None if absent.
    """
    path = os.path.join(PROFILES, summary)
    tag = "traffic_bytes_per_launch" + (f"[{key}]" if key else "")
    try:
        with open(path) as f:
            for line in f:
                head, _, val = line.partition("=")
                if head.strip() == tag:
                    return float(val)
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
    ap.add_argument("--settle-ms", type=float, default=200.0,
                    help="untimed repetitions of each leg's step before its warm-up steps, "
                         "in milliseconds of wall time (0: none)")
    ap.add_argument("--copy-calibration-mb", type=int, default=0,
                    help="also run one device-to-device copy of this many MiB "
                         "(reference kernel for HBM counter scaling)")
    return ap.parse_args()


def _log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# --------------------------------------------------------------------------- timing
def _settle(fns, seconds):
    """Repeats the step, untimed, for `seconds` of wall time (GPU clocks ramp up
    under sustained load); returns the number of steps run."""
    import torch
    n, i = len(fns), 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(8):
            fns[i % n]()
            i += 1
        torch.cuda.synchronize()
    return i


def _time_steps(fns, steps, warmup, settle_s=0.0):
    """(wall seconds per step, GPU seconds per step, settle steps) over `steps`
    calls cycling through fns (one kernel each), after `settle_s` seconds of
    untimed steps and then `warmup` untimed calls."""
    import torch
    n = len(fns)
    settled = _settle(fns, settle_s) if settle_s > 0 else 0
    for i in range(warmup):
        fns[i % n]()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for i in range(steps):
        fns[i % n]()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu = e0.elapsed_time(e1) / 1e3
    if gpu > wall:  # the events are recorded inside the wall-clock window
        raise RuntimeError(f"GPU time {gpu} s exceeds the wall time {wall} s of its own steps")
    return wall / steps, gpu / steps, settled


def _leg(name, fns, work, unit, kernel, args, traffic=None, note=""):
    """Time a leg; work = algorithmic bytes or FLOPs per step."""
    steps = max(args.steps, len(fns))
    t_step, t_kern, settled = _time_steps(fns, steps, max(args.warmup, len(fns)),
                                          args.settle_ms / 1e3)
    scale = 1e9 if unit == "GB/s" else 1e12
    bound = "hbm" if unit == "GB/s" else "mfma"
    peak = HBM_PEAK_GBS if bound == "hbm" else FP16_PEAK_TFLOPS
    out = {"value": work / t_step / scale, "unit": unit, "ms_per_step": t_step * 1e3,
           "work_per_step": work, "steps": steps,
           "settle": {"ms": args.settle_ms, "steps": settled},
           "roofline": {"bound": bound, "achieved": work / t_kern / scale, "peak": peak,
                        "unit": unit, "frac": work / t_kern / scale / peak, "traffic": traffic,
                        "kernel": kernel, "kernel_us": t_kern * 1e6}}
    if note:
        out["note"] = note
    _log(f"{name}: {out['value']:.1f} {unit} per step ({t_step * 1e6:.1f} us), kernel "
         f"{t_kern * 1e6:.1f} us, frac {out['roofline']['frac']:.3f}")
    return out


def _copies(nbytes_one, floor=1):
    """Input sets to rotate so that their total exceeds twice the Infinity Cache."""
    return max(floor, -(-2 * MALL_BYTES // max(1, nbytes_one)))


# --------------------------------------------------------------------------- CPU baseline
def _cpu_threads():
    """Host threads for the CPU baseline: the job's CPU share (OMP_NUM_THREADS,
    16 on the GPU boxes) when the environment sets one, else os.cpu_count().
    On a GPU box os.cpu_count() reports every core of the host, most of which
    belong to other jobs, so it is recorded but not used there."""
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


def _cpu_baseline(fn, work, unit, sample, args, kind="port", order="fp16, the reference's op order"):
    """Times fn (the reference's naive path restated on a bounded sample of the
    leg's workload, `work` units of it) on the host CPU: one warm-up run, then
    at least 5 runs and at least 2 s, and the median (and mean) reported; a
    single run when one takes over 30 s."""
    if args.no_cpu_baseline:
        return None
    import torch
    threads = _cpu_threads()
    torch.set_num_threads(threads)
    t0 = time.perf_counter()
    fn()  # warm-up
    first = time.perf_counter() - t0
    ts = [first] if first > 30.0 else []
    while first <= 30.0 and (len(ts) < 5 or sum(ts) < 2.0):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    t = ts[len(ts) // 2]
    mean = sum(ts) / len(ts)
    scale = 1e9 if unit == "GB/s" else 1e12
    return {"value": work / t / scale, "unit": unit, "cores": torch.get_num_threads(),
            "kind": kind,
            "sample": f"{sample}; {order}; median of {len(ts)} runs ({t * 1e3:.1f} ms, mean "
                      f"{mean * 1e3:.1f} ms){' (one run: over 30 s)' if len(ts) == 1 else ''}; "
                      f"{torch.get_num_threads()} threads (the job's CPU share; os.cpu_count() = "
                      f"{os.cpu_count()}) of {_cpu_model()}"}


# --------------------------------------------------------------------------- headline legs
def bench_paged(args):
    import torch
    from attention_kernel_triton_amd import decode_flash_attention_redundant_var_len_paged as pg
    from attention_kernel_triton_amd import _ops
    from attention_kernel_triton_amd import synthetic as syn
    dev = torch.device("cuda:0")
    _log("generating config 3 (paged decode)")
    cfg = syn.paged_config()
    nbytes = cfg.bytes()  # 472 MB per step: under twice the Infinity Cache, so rotated
    sets = [cfg.to(dev) for _ in range(_copies(nbytes))]  # each .to() is a fresh device copy

    def make(p):
        if args.chunk:
            return lambda: _ops.decode_paged(p.q, p.pool, p.indptr, p.indices, p.last_len,
                                             chunk_tokens=args.chunk)
        return lambda: pg.flash_attention_decode_paged(p.q, p.pool, p.indptr, p.indices,
                                                       p.last_len)

    _log(f"timing paged decode ({len(sets)} input sets rotated)")
    kernel = "split_kernel<128,4,kModePaged>" if args.chunk else "paged_stream_kernel<128,4>"
    profile = ("split_kernel_paged_decode_config3.md" if args.chunk
               else "paged_stream_kernel_config3.md")
    out = _leg("config 3", [make(p) for p in sets], nbytes, "GB/s", kernel, args,
               traffic=_traffic(profile))
    out["tokens"] = sum(cfg.lens)
    out["input_sets"] = len(sets)
    out["ceilings"] = _ceilings(cfg, sets, args)
    del sets

    def cpu():
        from oracle import ref_order
        ref_order.naive_paged_attention(cfg.q, cfg.pool, cfg.indptr, cfg.indices, cfg.last_len)

    _log("CPU baseline: the reference's naive_paged_attention (fp16 op order) on config 3")
    out["cpu_baseline"] = _cpu_baseline(cpu, nbytes, "GB/s", "the full config 3 batch", args)
    return out


def _ceilings(cfg, sets, args):
    """Read-rate ceilings of the headline's bytes on this device: the diagnostic
    kernels of csrc/diag.hip read exactly the (page, kv head) K and V blocks
    the paged decode reads (a gather over the same page tables), and the same
    number of bytes in order (a linear read of each pool), with no arithmetic,
    over the same rotated input sets and with the same settling and timing."""
    import torch
    from attention_kernel_triton_amd import _native as N
    lib = N.load()
    dev = sets[0].pool.device
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    P, _, Hkv, page, D = cfg.pool.shape
    total = cfg.indices.numel()
    gather_bytes = total * Hkv * page * D * 2 * 2 + 4 * total
    pool_bytes = cfg.pool.numel() * 2

    def gather(p):
        N.check(lib.akt_diag_paged_gather(N.ptr(p.pool), N.ptr(p.indices), total, Hkv, D, page, P,
                                          N.strides(p.pool), N.ptr(sink), N.stream_of(p.pool)),
                "akt_diag_paged_gather")

    def stream(p):
        N.check(lib.akt_diag_stream_read(N.ptr(p.pool), pool_bytes, N.ptr(sink),
                                         N.stream_of(p.pool)), "akt_diag_stream_read")

    _log("ceiling legs: gather of config 3's blocks, linear read of its pool")
    out = {
        "ceiling_gather_config3": _leg(
            "gather ceiling", [lambda p=p: gather(p) for p in sets], gather_bytes, "GB/s",
            "paged_gather_kernel<4>", args,
            traffic=_traffic("legs_hbm_traffic.md", "ceiling_gather_config3"),
            note=f"reads every (page, kv head) K and V block of config 3's page table "
                 f"({total} pages x {Hkv} kv heads x 8 KB) and nothing else; {len(sets)} input "
                 "sets rotated"),
        "ceiling_stream_read_config3": _leg(
            "stream ceiling", [lambda p=p: stream(p) for p in sets], pool_bytes, "GB/s",
            "stream_read_kernel", args,
            traffic=_traffic("legs_hbm_traffic.md", "ceiling_stream_read_config3"),
            note=f"reads each {pool_bytes} B pool in order; {len(sets)} pools rotated"),
    }
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
    _log("timing prefill")
    out = _leg("config 0", [lambda: pre.flash_attention_prefill(c.Q, c.K, c.V, True, c.scale,
                                                                c.group)],
               flops, "TFLOP/s", "prefill_kernel<64,causal>", args,
               traffic=_traffic("prefill_kernel_causal_config0.md"))
    del c
    nb = 2

    def cpu():
        from oracle import ref_order
        ref_order.prefill(cfg.Q[:nb], cfg.K[:nb], cfg.V[:nb], True, cfg.scale, cfg.group)

    _log("CPU baseline: the reference's prefill (fp16 op order) on 2 of 8 batches of config 0")
    out["cpu_baseline"] = _cpu_baseline(cpu, flops * nb // 8, "TFLOP/s",
                                        "2 of the 8 batches of config 0", args)
    return out


# --------------------------------------------------------------------------- other rows
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
    dev = torch.device("cuda:0")
    legs = {}

    # ---- config 1: var-len causal prefill (compute-bound: no rotation)
    _log("leg: var-len causal prefill, config 1")
    c1 = syn.prefill_config(1)
    d1 = c1.to(dev)
    legs["prefill_varlen_config1"] = _leg(
        "config 1", [lambda: _ops.prefill(d1.Q, d1.K, d1.V, True, d1.scale, varlen=d1.varlen)],
        c1.flops(), "TFLOP/s", "prefill_kernel<64,causal,varlen>", args,
        note="FLOPs over each sequence's valid causal pairs")
    del d1
    torch.cuda.empty_cache()
    lens1 = [int(x) for x in c1.varlen.tolist()]

    def cpu1():
        from oracle import ref_order
        ref_order.prefill_varlen(c1.Q[:2], c1.K[:2], c1.V[:2], True, c1.scale, c1.group,
                                 c1.varlen[:2])

    fl1 = 4 * 64 * 64 * sum(L * (L + 1) // 2 for L in lens1[:2])
    legs["prefill_varlen_config1"]["cpu_baseline"] = _cpu_baseline(
        cpu1, fl1, "TFLOP/s", f"the first 2 of 8 sequences of config 1 (lengths {lens1[:2]}; "
        "the reference computes all 1024 rows and zeroes the padding)", args)

    # ---- config 2: dense GQA decode (33.7 MB: rotated)
    _log("leg: dense GQA decode, config 2")
    c2 = syn.decode_config()
    n2 = _copies(c2.bytes())
    d2 = [c2.to(dev) for _ in range(n2)]
    legs["decode_config2"] = _leg(
        "config 2", [lambda d=d: _ops.decode(d.q, d.K, d.V, d.scale) for d in d2], c2.bytes(),
        "GB/s", "split_kernel<64,4,kModeDense>", args, note=f"inputs rotated over {n2} copies")
    del d2
    torch.cuda.empty_cache()

    def cpu2():
        from oracle import ref_order
        ref_order.decode(c2.q, c2.K, c2.V, c2.scale, c2.group)

    legs["decode_config2"]["cpu_baseline"] = _cpu_baseline(
        cpu2, c2.bytes(), "GB/s", "the full config 2 batch", args)

    # ---- config 4a: sparse-token decode + LSE (K/V rotated)
    _log("leg: sparse-token decode, config 4a")
    s4 = syn.sparse_config()
    B, H, N = s4.uniform.shape
    ind4, nnz4 = kept_index.select_kept(s4.l_max, uniform=s4.uniform.to(dev),
                                        kept_ratio=s4.kept_ratio, row_len=s4.row_len.to(dev))
    ind4c, nnz4c = ind4.cpu(), nnz4.cpu()
    b4 = _sparse_bytes(ind4c, nnz4c, s4.group, 128, B * H)
    n4 = _copies((s4.K.numel() + s4.V.numel()) * 2)
    kv4 = [(s4.K.to(dev), s4.V.to(dev)) for _ in range(n4)]
    q4 = s4.q.to(dev)
    legs["sparse_config4a"] = _leg(
        "config 4a", [lambda kv=kv: _ops.sparse_decode(q4, kv[0], kv[1], ind4, nnz4, s4.scale,
                                                      return_lse=True) for kv in kv4],
        b4, "GB/s", "split_kernel<128,1,kModeSparseDense>", args,
        note=f"O + LSE; K/V rotated over {n4} copies; bytes = unique kept rows per kv head")
    del kv4
    torch.cuda.empty_cache()

    def cpu4():
        from oracle import ref_order
        ref_order.sparsetoken_naive_decode(s4.q, s4.K, s4.V, ind4c, nnz4c, s4.scale, s4.group)

    legs["sparse_config4a"]["cpu_baseline"] = _cpu_baseline(
        cpu4, b4, "GB/s", "the full config 4a batch", args,
        order="fp16, the reference's (b, h) loop and index gathers")

    # ---- config 4b: sparse paged + MagicPIG decode (kept-index sets rotated)
    _log("leg: sparse paged + MagicPIG decode, config 4b")
    s5 = syn.sparse_paged_config()
    p5 = s5.paged.to(dev)
    B, H, N = s5.uniform.shape
    sets = []
    b5 = 0
    gen = torch.Generator(device=dev).manual_seed(7)
    while True:  # distinct kept-index sets until their gathered rows exceed 2x the cache
        u = torch.rand((B, H, N), generator=gen, device=dev)
        sets.append(kept_index.select_kept(s5.l_max, uniform=u, kept_ratio=s5.kept_ratio,
                                           row_len=s5.row_len.to(dev)))
        if len(sets) == 1:
            b5 = _sparse_bytes(sets[0][0].cpu(), sets[0][1].cpu(), s5.group, 256, B * H) + \
                4 * (p5.indices.numel() + p5.indptr.numel())
        if len(sets) * b5 >= 2 * MALL_BYTES or len(sets) >= 64:
            break
    legs["sparse_paged_config4b"] = _leg(
        "config 4b", [lambda st=st: _ops.sparse_decode_paged(p5.q, p5.pool, p5.indptr, p5.indices,
                                                             st[0], st[1], return_lse=True)
                      for st in sets],
        b5, "GB/s", "split_kernel<256,1,kModeSparsePaged>", args,
        note=f"O + LSE; {len(sets)} kept-index sets rotated")
    lk, ll = s5.lsh_k.to(dev), s5.lsh_l.to(dev)
    legs["magicpig_config4b"] = _leg(
        "config 4b MagicPIG", [lambda st=st: _ops.sparse_decode_paged(
            p5.q, p5.pool, p5.indptr, p5.indices, st[0], st[1], return_lse=True, lsh_k=lk,
            lsh_l=ll) for st in sets],
        b5, "GB/s", "split_kernel<256,1,kModeSparsePaged,magicpig>", args,
        note=f"O + LSE with norm; {len(sets)} kept-index sets rotated")
    ind5, nnz5 = sets[0][0].cpu(), sets[0][1].cpu()
    del p5, sets
    torch.cuda.empty_cache()
    pc = s5.paged

    def cpu5():
        from oracle import ref_order
        ref_order.sparsetoken_naive_paged_attention(pc.q, pc.pool, pc.indptr, pc.indices, ind5,
                                                    nnz5)

    def cpu6():
        from oracle import ref_order
        ref_order.magicpig_sparsetoken_naive_paged_attention(pc.q, pc.pool, pc.indptr, pc.indices,
                                                             ind5, nnz5, s5.lsh_k, s5.lsh_l)

    per_token = "fp16 (MagicPIG: fp32 scores) in the reference's per-token gather loop"
    legs["sparse_paged_config4b"]["cpu_baseline"] = _cpu_baseline(
        cpu5, b5, "GB/s", "the full config 4b batch (first kept-index set)", args,
        order=per_token)
    legs["magicpig_config4b"]["cpu_baseline"] = _cpu_baseline(
        cpu6, b5, "GB/s", "the full config 4b batch (first kept-index set)", args,
        order=per_token)

    # ---- kept-index selection over config 4b's keep draws (sets rotated)
    _log("leg: kept-index selection, config 4b draws")
    rl = s5.row_len.to(dev)
    lens5 = [int(x) for x in s5.row_len.reshape(-1).tolist()]
    bk = 4 * sum(lens5) + 4 * B * H * s5.l_max + 4 * B * H
    nk = _copies(bk + 4 * B * H * N)
    draws = [torch.rand((B, H, N), generator=gen, device=dev) for _ in range(nk)]
    legs["kept_index_config4b"] = _leg(
        "kept index", [lambda u=u: kept_index.select_kept(s5.l_max, uniform=u,
                                                          kept_ratio=s5.kept_ratio, row_len=rl)
                       for u in draws],
        bk, "GB/s", "kept_index_kernel", args,
        note=f"{B * H} rows of up to {N} fp32 draws; {nk} draw sets rotated; bytes = draws "
             f"read + padded index rows and counts written")
    del draws
    torch.cuda.empty_cache()
    u5 = s5.uniform.reshape(B * H, N).numpy()
    rl5 = s5.row_len.reshape(-1).numpy()

    def cpu7():
        from oracle.kept import kept_from_uniform
        kept_from_uniform(u5, s5.kept_ratio, s5.l_max, rl5)

    legs["kept_index_config4b"]["cpu_baseline"] = _cpu_baseline(
        cpu7, bk, "GB/s", "all 96 rows of config 4b's draws", args,
        order="the harness's rand < p, nonzero and -1 padding, restated in numpy")

    # ---- LSE merge of two fp16 partial states over config 0's rows (rotated)
    _log("leg: LSE merge of partial states")
    rows, D, parts = 8 * 64 * 1024, 64, 2
    mb = parts * rows * (D * 2 + 4) + rows * (D * 2 + 4)
    nm = _copies(mb)
    mins = [(torch.randn(parts, rows, D, device=dev).half(), torch.randn(parts, rows, device=dev))
            for _ in range(nm)]
    legs["merge_states"] = _leg(
        "merge", [lambda m=m: _ops.merge_states(m[0], m[1]) for m in mins], mb, "GB/s",
        "merge_kernel<f16,f16>", args,
        note=f"{parts} fp16 parts of [{rows}, {D}] (config 0's rows) -> fp16; {nm} input sets "
             f"rotated")
    mo_c, ml_c = mins[0][0][:, : rows // 16].cpu(), mins[0][1][:, : rows // 16].cpu()
    del mins
    torch.cuda.empty_cache()

    def cpu8():
        from oracle import naive
        naive.merge_states(mo_c, ml_c, dtype=torch.float32)

    legs["merge_states"]["cpu_baseline"] = _cpu_baseline(
        cpu8, mb // 16, "GB/s", "1/16 of the rows", args,
        order="fp32 log-sum-exp merge in torch (no reference counterpart)")

    # ---- paged KV append: 32 sequences x 1024 tokens into random pages (rotated)
    _log("leg: paged KV append (prefill-sized)")
    Bq, Hkv, D, page, T = 32, 8, 128, 16, 1024
    pages = Bq * T // page
    perm = torch.randperm(pages, generator=torch.Generator().manual_seed(3)).to(torch.int32)
    indptr = torch.arange(0, pages + 1, T // page, dtype=torch.int32)
    last = torch.full((Bq,), page, dtype=torch.int32)
    ap = torch.arange(0, Bq * T + 1, T, dtype=torch.int32)
    t_dev = [x.to(dev) for x in (ap, indptr, perm, last)]
    ab = 8 * Bq * T * Hkv * D + 4 * (pages + 2 * Bq + 2)
    na = _copies(ab)
    asets = [(torch.randn(Bq * T, Hkv, D, device=dev).half(),
              torch.randn(Bq * T, Hkv, D, device=dev).half(),
              torch.zeros((pages, 2, Hkv, page, D), dtype=torch.float16, device=dev))
             for _ in range(na)]
    legs["paged_append"] = _leg(
        "append", [lambda a=a: append_paged_kv(a[0], a[1], t_dev[0], a[2], t_dev[1], t_dev[2],
                                               t_dev[3]) for a in asets],
        ab, "GB/s", "paged_append_kernel", args,
        note=f"{Bq} sequences x {T} tokens into random pages; {na} input sets rotated; bytes = "
             f"new K/V rows read and written once")
    nb_cpu = 2
    kn_c = asets[0][0][: nb_cpu * T].cpu().numpy()
    vn_c = asets[0][1][: nb_cpu * T].cpu().numpy()
    del asets
    torch.cuda.empty_cache()
    pool_c = torch.zeros((pages, 2, Hkv, page, D), dtype=torch.float16).numpy()

    def cpu9():
        from oracle.kept import paged_append
        paged_append(pool_c, kn_c, vn_c, ap[: nb_cpu + 1].numpy(),
                     indptr[: nb_cpu + 1].numpy(), perm.numpy(), last[:nb_cpu].numpy())

    legs["paged_append"]["cpu_baseline"] = _cpu_baseline(
        cpu9, 8 * nb_cpu * T * Hkv * D, "GB/s", f"{nb_cpu} of the {Bq} sequences", args,
        order="numpy, one token at a time (no reference counterpart)")
    # HBM bytes per launch of each leg's kernel, from the committed counter summary.
    for key, leg in legs.items():
        if leg["roofline"]["traffic"] is None:
            leg["roofline"]["traffic"] = _traffic("legs_hbm_traffic.md", key)
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
    _native.torch_ext()
    res = {"metric": "paged decode HBM GB/s + prefill TFLOP/s (fp16, % MI355X peak), 1 GPU",
           "value": None, "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": None, "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
           "data": "synthetic (seeded N(0,1) fp16)",
           "config": {"workload": "paged var-len GQA decode, config 3", "batch": 32,
                      "num_q_heads": 32, "num_kv_heads": 8, "head_dim": 128, "page_size": 16,
                      "seq_len": "U[256, 8192]", "parallelism": "none (1 GPU)"}}
    if args.only in ("all", "headline", "paged"):
        pg = bench_paged(args)
        res["value"] = pg.pop("value")
        res["ms_per_step"] = pg.pop("ms_per_step")
        res["roofline"] = pg.pop("roofline")
        cb = pg.pop("cpu_baseline", None)
        if cb:
            res["cpu_baseline"] = cb
        pg.pop("unit", None)
        res["config"].update({"bytes_per_step": pg.pop("work_per_step"), "tokens": pg["tokens"]})
        # Untimed steps before the W warm-up steps (GPU clocks ramp up under load).
        res["settle"] = pg.pop("settle")
        res.setdefault("legs", {}).update(pg.pop("ceilings"))
        torch.cuda.empty_cache()
    if args.only in ("all", "headline", "prefill"):
        pf = bench_prefill(args)
        pf["config"] = {"workload": "causal GQA prefill, config 0", "batch": 8,
                        "num_q_heads": 64, "num_kv_heads": 16, "seq_len": 1024, "head_dim": 64}
        res["prefill"] = pf
        if res["value"] is None:
            res.update({"value": pf["value"], "unit": pf["unit"],
                        "ms_per_step": pf["ms_per_step"], "roofline": pf["roofline"]})
        torch.cuda.empty_cache()
    if args.only in ("all", "legs"):
        res.setdefault("legs", {}).update(bench_legs(args))
    if args.copy_calibration_mb:
        copy_calibration(args.copy_calibration_mb)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
