"""The decode workspace contract of the C ABI (include/akt_amd.h): only the
first min(AKT_WORKSPACE_ZERO_BYTES, size) bytes of a workspace must be zero
before its first use, and every call leaves them zero again.

Each case fills a workspace with 0xFF, zeroes exactly that prefix, calls the
paged decode entry point through the C ABI twice in a row on it, and compares
both results bit for bit with the drop-in wrapper (which runs the same kernels
on a workspace zeroed whole).
"""
import math

import pytest
import torch

from attention_kernel_triton_amd import _native as N
from attention_kernel_triton_amd import _ops
from attention_kernel_triton_amd import synthetic as syn

pytestmark = pytest.mark.gpu


def _dirty_workspace(nbytes, dev):
    ws = torch.full((nbytes,), 0xFF, dtype=torch.uint8, device=dev)
    ws[: min(N.WORKSPACE_ZERO_BYTES, nbytes)] = 0
    return ws


def _paged_capi(p, ws):
    lib = N.load()
    B, Hq, D = p.q.shape[0], p.q.shape[1], p.q.shape[-1]
    P, _, Hkv, page, _ = p.pool.shape
    o = torch.empty((B, Hq, D), dtype=torch.float16, device=p.q.device)
    lse = torch.empty((B, Hq), dtype=torch.float32, device=p.q.device)
    rc = lib.akt_decode_paged_fwd(N.ptr(p.q), N.ptr(p.pool), N.ptr(p.indptr), N.ptr(p.indices),
                                  N.ptr(p.last_len), N.ptr(o), N.ptr(lse), B, Hq, Hkv, D, page,
                                  p.indices.numel(), P, N.strides(p.q), N.strides(p.pool),
                                  1.0 / math.sqrt(D), 0, N.ptr(ws), ws.numel(),
                                  N.stream_of(p.q))
    N.check(rc, "akt_decode_paged_fwd")
    return o, lse


def _need(p):
    B, Hq, D = p.q.shape[0], p.q.shape[1], p.q.shape[-1]
    _, _, Hkv, page, _ = p.pool.shape
    return N.load().akt_decode_paged_workspace_size(B, Hq, Hkv, D, page, p.indices.numel(), 0)


@pytest.mark.parametrize("case", ["config3", "over_32768_units"])
def test_paged_decode_needs_only_the_documented_zero_prefix(dev, case):
    if case == "config3":
        p = syn.paged_config().to(dev)  # 256 units, persistent split kernel
    else:
        # 1100 sequences x 32 kv heads = 35200 units: past the fixed counter
        # area, so the call zero-fills its extra counters itself (and, past
        # 1024 sequences, runs the non-persistent split kernel).
        g = torch.Generator().manual_seed(13)
        B, Hkv, D, page = 1100, 32, 64, 16
        lens = torch.randint(257, 321, (B,), generator=g).tolist()
        indptr, indices, last, P = syn.block_table(g, lens, page)
        gd = torch.Generator(device=dev).manual_seed(14)
        pool = torch.randn(P, 2, Hkv, page, D, generator=gd, device=dev, dtype=torch.float16)
        q = torch.randn(B, Hkv, 1, D, generator=gd, device=dev, dtype=torch.float16)
        p = syn.Paged(q, pool, indptr.to(dev), indices.to(dev), last.to(dev), lens)
    need = _need(p)
    assert need > N.WORKSPACE_ZERO_BYTES
    ro, rl = _ops.decode_paged(p.q, p.pool, p.indptr, p.indices, p.last_len, return_lse=True)
    ws = _dirty_workspace(need, dev)
    for _ in range(2):
        o, lse = _paged_capi(p, ws)
        torch.cuda.synchronize(dev)
        assert torch.equal(o, ro) and torch.equal(lse, rl)
        # The counters are zero again after the call.
        assert int(ws[: N.WORKSPACE_ZERO_BYTES].count_nonzero()) == 0


# Small launches of the automatic (stream-K) path: more waves than groups
# (some waves empty) and fewer, units cut at many positions, paired
# (512-thread) and unpaired (256-thread) instances.
@pytest.mark.parametrize("lens,page,Hq,Hkv,D", [
    ([40, 300, 1], 16, 8, 2, 128),           # 46 groups, 48 waves: two empty waves
    ([360, 27, 4, 450, 140], 48, 8, 2, 128),  # 138 groups, 144 waves
    ([1, 16, 17, 33], 16, 8, 1, 128),        # G = 8 (256-thread instance): 7 groups, 8 waves
    ([700, 5, 1300], 16, 16, 4, 64),
    ([513, 2, 90], 64, 4, 2, 256),
    ([8192, 4000, 31, 6000], 16, 32, 8, 128),  # more groups than waves
])
def test_paged_auto_path_on_dirty_workspace_matches_oracle(dev, lens, page, Hq, Hkv, D):
    """Every unit's run of waves stores and counts its partials: the results
    match the oracle on a workspace whose partial area holds garbage, and the
    arrival counters are zero again after each of two calls."""
    from oracle import naive

    g = torch.Generator().manual_seed(sum(lens) + page + D)
    indptr, indices, last, P = syn.block_table(g, lens, page, 3)
    pool = torch.randn(P, 2, Hkv, page, D, generator=g).half()
    q = torch.randn(len(lens), Hq, 1, D, generator=g).half()
    ro, rl = naive.naive_paged_attention(q, pool, indptr, indices, last)
    p = syn.Paged(q.to(dev), pool.to(dev), indptr.to(dev), indices.to(dev), last.to(dev), lens)
    ws = _dirty_workspace(_need(p), dev)
    for _ in range(2):
        o, lse = _paged_capi(p, ws)
        torch.cuda.synchronize(dev)
        err = float((o.cpu().double() - ro).abs().max())
        lerr = float((lse.cpu().double() - rl).abs().max())
        assert err <= 2e-3 and lerr <= 1e-4, (err, lerr)
        assert int(ws[: N.WORKSPACE_ZERO_BYTES].count_nonzero()) == 0
