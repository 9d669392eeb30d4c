"""The no-allocation paged decode entry point, called through the C ABI.

akt_decode_paged_fwd_noalloc keeps its split-KV workspace in a device array of
the library instead of a caller workspace; it runs the same kernels as
akt_decode_paged_fwd, so its outputs must equal that entry point's bit for bit.
Two calls in a row, the second on a smaller input, check that the shared array
carries nothing from one call into the next.
"""
import math

import pytest
import torch

from attention_kernel_triton_amd import _native as N
from attention_kernel_triton_amd import _ops
from attention_kernel_triton_amd import synthetic as syn

pytestmark = pytest.mark.gpu


def _noalloc(p, return_lse=True):
    lib = N.load()
    B, Hq, D = p.q.shape[0], p.q.shape[1], p.q.shape[-1]
    P, _, Hkv, page, _ = p.pool.shape
    o = torch.empty((B, Hq, D), dtype=torch.float16, device=p.q.device)
    lse = torch.empty((B, Hq), dtype=torch.float32, device=p.q.device) if return_lse else None
    rc = lib.akt_decode_paged_fwd_noalloc(N.ptr(p.q), N.ptr(p.pool), N.ptr(p.indptr),
                                          N.ptr(p.indices), N.ptr(p.last_len), N.ptr(o),
                                          N.ptr(lse), B, Hq, Hkv, D, page, p.indices.numel(), P,
                                          N.strides(p.q), N.strides(p.pool),
                                          1.0 / math.sqrt(D), 0, N.stream_of(p.q))
    N.check(rc, "akt_decode_paged_fwd_noalloc")
    return o, lse


def test_noalloc_paged_decode_equals_workspace_entry_point(dev):
    big = syn.paged_config().to(dev)  # config 3
    small = syn.paged_config(seed=9, B=5, Hq=8, Hkv=2, D=128, min_len=1, max_len=3000).to(dev)
    for p in (big, small):
        ro, rl = _ops.decode_paged(p.q, p.pool, p.indptr, p.indices, p.last_len, return_lse=True)
        o, lse = _noalloc(p)
        torch.cuda.synchronize(dev)
        assert torch.equal(o, ro) and torch.equal(lse, rl)
