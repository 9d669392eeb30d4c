"""Drop-in for the reference module decode_flash_attention_redundant_var_len_paged.py.

``flash_attention_decode_paged`` keeps the reference signature, the FlashInfer
style CSR page table and the combined K/V pool layout
(decode_flash_attention_redundant_var_len_paged.py:228-274):
  q               [B, Hq, 1, D]
  paged_kv_cache  [num_pages, 2, Hkv, page_size, D]   (K = [:, 0], V = [:, 1])
  kv_page_indptr  [B + 1]  int32
  kv_page_indices [total_pages] int32
  kv_last_page_len[B]      int32
Sequence b holds (indptr[b+1] - indptr[b] - 1) * page_size + last_page_len[b]
tokens; the softmax scale is 1/sqrt(D) and G = Hq // Hkv as in the reference.
Differences: any page_size works (the reference asserts page_size % 16 == 0),
a sequence with no pages yields zeros (the reference kernel yields NaN), and
``return_lse=True`` also returns the fp32 log-sum-exp [B, Hq].
"""
from __future__ import annotations

from . import _ops

redundant_len = 16  # kept for import compatibility; the kernel does not replicate q


def flash_attention_decode_paged(q, paged_kv_cache, kv_page_indptr, kv_page_indices,
                                 kv_last_page_len, return_lse=False):
    """Returns O: [B, Hq, D] (and lse [B, Hq] when return_lse)."""
    return _ops.decode_paged(q, paged_kv_cache, kv_page_indptr, kv_page_indices,
                             kv_last_page_len, return_lse=return_lse)
