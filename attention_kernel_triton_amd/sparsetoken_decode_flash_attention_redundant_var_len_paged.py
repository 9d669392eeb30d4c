"""Drop-in for sparsetoken_decode_flash_attention_redundant_var_len_paged.py.

``sparsetoken_flash_attention_decode_paged`` keeps the reference signature
(sparsetoken_decode_flash_attention_redundant_var_len_paged.py:170-232).
Kept token t of sequence b is read from page kv_page_indices[kv_page_indptr[b]
+ t // page_size], slot t % page_size; the scale is 1/sqrt(D).  Tokens whose
logical page lies outside the sequence's page list are skipped, a head with
nnz == 0 yields zeros, and ``return_lse=True`` also returns the fp32
log-sum-exp [B, Hq].
"""
from __future__ import annotations

from . import _ops

redundant_len = 16  # kept for import compatibility; the kernel does not replicate q


def sparsetoken_flash_attention_decode_paged(q, paged_kv_cache, kv_page_indptr, kv_page_indices,
                                             sparse_ind, sparse_nnz, return_lse=False):
    """Returns O: [B, Hq, D] (and lse [B, Hq] when return_lse)."""
    return _ops.sparse_decode_paged(q, paged_kv_cache, kv_page_indptr, kv_page_indices,
                                    sparse_ind, sparse_nnz, return_lse=return_lse)
