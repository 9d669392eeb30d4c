"""GPU parity of the paged KV write side (akt_paged_kv_append, PagedKVCache)."""
import math

import numpy as np
import pytest
import torch

from attention_kernel_triton_amd import decode_flash_attention_redundant_var_len_paged as pg
from attention_kernel_triton_amd.paged_kv import PagedKVCache, append_paged_kv
from helpers import assert_close
from oracle import naive
from oracle.kept import paged_append

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("page,D", [(16, 128), (1, 64), (48, 256)])
def test_append_kernel_is_bit_exact(dev, page, D):
    rng = np.random.default_rng(page + D)
    B, Hkv, P = 5, 4, 64
    lens = [0, 1, 37, 200, 129]
    counts = [0, 1, 17, 200, 5]
    perm = rng.permutation(P)
    indptr, indices, last, off = [0], [], [], 0
    for n in lens:
        npg = -(-n // page)
        indices += list(perm[off:off + npg])
        off += npg
        indptr.append(len(indices))
        last.append(0 if n == 0 else (n - 1) % page + 1)
    if len(indices) > 3:
        indices[3] = P + 7  # invalid page id: its tokens are skipped
    ap = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    pool = rng.standard_normal((P, 2, Hkv, page, D)).astype(np.float16)
    k_new = rng.standard_normal((ap[-1], Hkv, D)).astype(np.float16)
    v_new = rng.standard_normal((ap[-1], Hkv, D)).astype(np.float16)
    ref = paged_append(pool, k_new, v_new, ap, np.array(indptr), np.array(indices), np.array(last))
    gpool = torch.from_numpy(pool).to(dev)
    t = lambda a: torch.tensor(np.asarray(a), dtype=torch.int32, device=dev)  # noqa: E731
    append_paged_kv(torch.from_numpy(k_new).to(dev), torch.from_numpy(v_new).to(dev), t(ap), gpool,
                    t(indptr), t(indices), t(last))
    assert np.array_equal(gpool.cpu().numpy(), ref)


@pytest.mark.parametrize("B,Hkv,D,page", [(70, 2, 64, 16), (9, 3, 512, 8), (5, 5, 1024, 4)])
def test_append_many_sequences_and_wide_rows(dev, B, Hkv, D, page):
    """More sequences than a wave has lanes (the sequence search runs in
    64-sequence steps), runs of new tokens of 0 to 11 rows (sequence changes
    inside one wave's run of tokens), and token rows of 192 and 640 16-byte
    chunks (a partial last chunk column, and two passes over a row)."""
    rng = np.random.default_rng(B * 7 + D)
    counts = rng.integers(0, 12, size=B)
    counts[::5] = 0
    hist = rng.integers(0, 40, size=B)
    lens = hist + counts
    P = int(sum(-(-int(n) // page) for n in lens)) + 3
    perm = rng.permutation(P)
    indptr, indices, last, off = [0], [], [], 0
    for n in lens:
        npg = -(-int(n) // page)
        indices += [int(x) for x in perm[off:off + npg]]
        off += npg
        indptr.append(len(indices))
        last.append(0 if n == 0 else (int(n) - 1) % page + 1)
    ap = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    pool = rng.standard_normal((P, 2, Hkv, page, D)).astype(np.float16)
    k_new = rng.standard_normal((int(ap[-1]), Hkv, D)).astype(np.float16)
    v_new = rng.standard_normal((int(ap[-1]), Hkv, D)).astype(np.float16)
    ref = paged_append(pool, k_new, v_new, ap, np.array(indptr), np.array(indices), np.array(last))
    gpool = torch.from_numpy(pool).to(dev)
    t = lambda a: torch.tensor(np.asarray(a), dtype=torch.int32, device=dev)  # noqa: E731
    append_paged_kv(torch.from_numpy(k_new).to(dev), torch.from_numpy(v_new).to(dev), t(ap), gpool,
                    t(indptr), t(indices), t(last))
    assert np.array_equal(gpool.cpu().numpy(), ref)


def test_append_strided_new_rows(dev):
    """k_new / v_new given as views of a [total, 2, Hkv, D] projection output."""
    rng = np.random.default_rng(3)
    B, Hkv, D, page, P = 2, 2, 64, 16, 8
    kv = torch.from_numpy(rng.standard_normal((9, 2, Hkv, D)).astype(np.float16)).to(dev)
    indptr, indices, last = [0, 1, 2], [5, 2], [4, 5]
    ap = [0, 4, 9]
    pool = torch.zeros((P, 2, Hkv, page, D), dtype=torch.float16, device=dev)
    t = lambda a: torch.tensor(a, dtype=torch.int32, device=dev)  # noqa: E731
    append_paged_kv(kv[:, 0], kv[:, 1], t(ap), pool, t(indptr), t(indices), t(last))
    ref = paged_append(np.zeros(tuple(pool.shape), dtype=np.float16), kv[:, 0].cpu().numpy(),
                       kv[:, 1].cpu().numpy(), np.array(ap), np.array(indptr), np.array(indices),
                       np.array(last))
    assert np.array_equal(pool.cpu().numpy(), ref)


def test_paged_cache_prefill_then_decode_steps(dev):
    """Prefill chunks, then one token per step; decode over the cache after
    every step equals dense decode over each sequence's history."""
    g = torch.Generator().manual_seed(17)
    Hkv, G, D, page = 2, 4, 128, 16
    cache = PagedKVCache(num_pages=128, num_kv_heads=Hkv, page_size=page, head_dim=D, device=dev)
    seqs = [3, 11, 5]
    prefill = [300, 12, 0]
    hist_k = {s: torch.randn(n, Hkv, D, generator=g).half() for s, n in zip(seqs, prefill)}
    hist_v = {s: torch.randn(n, Hkv, D, generator=g).half() for s, n in zip(seqs, prefill)}
    cache.append(seqs, torch.cat([hist_k[s] for s in seqs]).to(dev),
                 torch.cat([hist_v[s] for s in seqs]).to(dev), prefill)
    for step in range(4):
        k1 = torch.randn(3, Hkv, D, generator=g).half()
        v1 = torch.randn(3, Hkv, D, generator=g).half()
        indptr, indices, last = cache.append(seqs, k1.to(dev), v1.to(dev), [1, 1, 1])
        for i, s in enumerate(seqs):
            hist_k[s] = torch.cat([hist_k[s], k1[i:i + 1]])
            hist_v[s] = torch.cat([hist_v[s], v1[i:i + 1]])
        q = torch.randn(3, Hkv * G, 1, D, generator=g).half()
        o = pg.flash_attention_decode_paged(q.to(dev), cache.pool, indptr, indices, last).cpu()
        for i, s in enumerate(seqs):
            K = hist_k[s].permute(1, 0, 2).unsqueeze(0).contiguous()
            V = hist_v[s].permute(1, 0, 2).unsqueeze(0).contiguous()
            ref, _ = naive.decode(q[i:i + 1], K, V, 1 / math.sqrt(D), G)
            assert_close(o[i], ref[0, :, 0], what=f"step {step} seq {s}")
    assert cache.seq_len(3) == 304 and cache.seq_len(5) == 4
    used = 128 - cache.free_pages
    cache.release(11)
    assert 128 - cache.free_pages == used - 1  # 16 tokens: one page back


def test_paged_cache_rejects_overflow(dev):
    cache = PagedKVCache(num_pages=2, num_kv_heads=1, page_size=4, head_dim=64, device=dev)
    with pytest.raises(MemoryError):
        cache.append([0], torch.zeros(9, 1, 64, dtype=torch.float16, device=dev),
                      torch.zeros(9, 1, 64, dtype=torch.float16, device=dev), [9])
