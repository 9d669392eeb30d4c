"""Paged KV cache write side (no reference module).

The reference reads paged caches (pool [P, 2, Hkv, page, D], CSR page table
kv_page_indptr / kv_page_indices / kv_last_page_len) but only builds them by
hand in its tests (decode_flash_attention_redundant_var_len_paged.py:349-353,
sparsetoken_decode_flash_attention_redundant_var_len_paged.py:321-330).
This module fills them:

- ``append_paged_kv`` runs the HIP kernel ``akt_paged_kv_append``: each
  sequence's new K/V rows become its last logical positions under an
  already-updated page table.
- ``PagedKVCache`` owns a pool and a free list on the host, grows each
  sequence's page list as tokens are appended (prefill chunks or one token
  per decode step), and hands out the page table the decode entry points
  take.  Page bookkeeping is host-side; only the copy runs on the GPU.
"""
from __future__ import annotations

import torch

from . import _native as N
from ._ops import _half_rows, _int32, _need_gpu, _same_device


def append_paged_kv(k_new, v_new, append_indptr, paged_kv_cache, kv_page_indptr,
                    kv_page_indices, kv_last_page_len) -> None:
    """Scatter k_new / v_new [total_new, Hkv, D] into paged_kv_cache [P, 2, Hkv, page, D].

    Sequence b's rows append_indptr[b]:append_indptr[b+1] become its last
    positions under the page table (which must already count them).  Runs
    asynchronously on the current stream.
    """
    pool = paged_kv_cache
    _need_gpu("paged_kv_cache", pool)
    if pool.dtype != torch.float16:
        raise TypeError(f"paged_kv_cache must be float16, got {pool.dtype}")
    if pool.stride(-1) != 1:
        raise ValueError("paged_kv_cache needs a unit head_dim stride (it is written in place)")
    dev = pool.device
    k_new = _half_rows("k_new", k_new)
    v_new = _half_rows("v_new", v_new)
    _same_device(dev, k_new=k_new, v_new=v_new)
    ap = _int32("append_indptr", append_indptr, dev).contiguous()
    indptr = _int32("kv_page_indptr", kv_page_indptr, dev).contiguous()
    indices = _int32("kv_page_indices", kv_page_indices, dev).contiguous()
    last = _int32("kv_last_page_len", kv_last_page_len, dev).contiguous()
    P, _, Hkv, page, D = pool.shape
    if k_new.dim() != 3 or k_new.shape[1:] != (Hkv, D) or v_new.shape != k_new.shape:
        raise ValueError(f"k_new / v_new must be [total_new, {Hkv}, {D}]")
    B = indptr.numel() - 1
    if ap.numel() != B + 1 or last.numel() != B:
        raise ValueError("append_indptr needs B+1 entries and kv_last_page_len B")
    lib = N.load()
    rc = lib.akt_paged_kv_append(N.ptr(k_new), N.ptr(v_new), N.ptr(ap), N.ptr(pool), N.ptr(indptr),
                                 N.ptr(indices), N.ptr(last), B, k_new.shape[0], Hkv, D, page, P,
                                 N.strides(k_new), N.strides(v_new), N.strides(pool),
                                 N.stream_of(pool))
    N.check(rc, "akt_paged_kv_append")


class PagedKVCache:
    """A page pool plus per-sequence page lists, in the reference's layout.

    >>> cache = PagedKVCache(num_pages=1024, num_kv_heads=8, page_size=16, head_dim=128)
    >>> cache.append([7, 9], k, v, [300, 12])       # prefill chunks
    >>> cache.append([7, 9], k1, v1, [1, 1])        # one decode step
    >>> indptr, indices, last = cache.page_table([7, 9])
    """

    def __init__(self, num_pages: int, num_kv_heads: int, page_size: int, head_dim: int,
                 device="cuda", dtype=torch.float16):
        self.page_size = page_size
        self.pool = torch.zeros((num_pages, 2, num_kv_heads, page_size, head_dim), dtype=dtype,
                                device=device)
        self._free = list(range(num_pages - 1, -1, -1))  # pop() hands out page 0 first
        self._pages: dict = {}
        self._len: dict = {}

    @property
    def free_pages(self) -> int:
        return len(self._free)

    def seq_len(self, seq_id) -> int:
        return self._len.get(seq_id, 0)

    def release(self, seq_id) -> None:
        """Return a sequence's pages to the free list."""
        self._free.extend(reversed(self._pages.pop(seq_id, [])))
        self._len.pop(seq_id, None)

    def _grow(self, seq_id, n: int) -> None:
        pages = self._pages.setdefault(seq_id, [])
        new_len = self._len.get(seq_id, 0) + n
        need = -(-new_len // self.page_size) - len(pages)
        if need > len(self._free):
            raise MemoryError(f"page pool exhausted: need {need} pages, {len(self._free)} free")
        for _ in range(need):
            pages.append(self._free.pop())
        self._len[seq_id] = new_len

    def page_table(self, seq_ids):
        """(kv_page_indptr, kv_page_indices, kv_last_page_len) int32 device tensors."""
        indptr, indices, last = [0], [], []
        for s in seq_ids:
            pages = self._pages.get(s, [])
            indices.extend(pages)
            indptr.append(len(indices))
            n = self._len.get(s, 0)
            last.append(0 if n == 0 else (n - 1) % self.page_size + 1)
        dev = self.pool.device
        mk = lambda v: torch.tensor(v, dtype=torch.int32, device=dev)  # noqa: E731
        return mk(indptr), mk(indices), mk(last)

    def append(self, seq_ids, k_new, v_new, counts):
        """Append counts[i] rows of k_new / v_new [sum(counts), Hkv, D] to seq_ids[i].

        Returns the batch's page table after the append.
        """
        if len(counts) != len(seq_ids):
            raise ValueError("one count per sequence")
        for s, n in zip(seq_ids, counts):
            if n < 0:
                raise ValueError("counts must be non-negative")
            self._grow(s, int(n))
        indptr, indices, last = self.page_table(seq_ids)
        ap = [0]
        for n in counts:
            ap.append(ap[-1] + int(n))
        append_paged_kv(k_new, v_new, torch.tensor(ap, dtype=torch.int32, device=self.pool.device),
                        self.pool, indptr, indices, last)
        return indptr, indices, last


__all__ = ["append_paged_kv", "PagedKVCache"]
