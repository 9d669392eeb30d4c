"""Sparse-token decode with CSR kept-token indices (no reference module).

The reference passes kept tokens as ``sparse_ind`` rows padded with -1 to
L_max plus a count per row, and notes a second format, ``inds`` + ``ptr``,
that saves the padding (sparse_decode_flash_attention.py:13-15).  These entry
points take that format: row u = b * Hq + h keeps the tokens
``inds[ptr[u]:ptr[u + 1]]`` (int32 positions, int64 row pointer of
B * Hq + 1 entries).  They run the same split-KV kernels as the padded entry
points, so results are identical on the same kept tokens.
"""
from __future__ import annotations

from . import _ops


def sparsetoken_flash_attention_decode_csr(q, K, V, inds, ptr, softmax_scale, GQA_group_size,
                                           return_lse=False, max_nnz=None):
    """CSR counterpart of sparsetoken_flash_attention_decode: returns [B, Hq, 1, D]."""
    B, H, _, D = q.shape
    assert K.shape[1] * GQA_group_size == H and V.shape == K.shape
    return _ops.sparse_decode_csr(q, K, V, inds, ptr, softmax_scale, return_lse=return_lse,
                                  max_nnz=max_nnz)


def sparsetoken_flash_attention_decode_paged_csr(q, paged_kv_cache, kv_page_indptr,
                                                 kv_page_indices, inds, ptr, return_lse=False,
                                                 max_nnz=None):
    """CSR counterpart of sparsetoken_flash_attention_decode_paged: returns [B, Hq, D]."""
    return _ops.sparse_decode_paged_csr(q, paged_kv_cache, kv_page_indptr, kv_page_indices, inds,
                                        ptr, return_lse=return_lse, max_nnz=max_nnz)


def magicpig_sparsetoken_flash_attention_decode_paged_csr(q, paged_kv_cache, kv_page_indptr,
                                                          kv_page_indices, inds, ptr, K, L,
                                                          return_lse=False, max_nnz=None):
    """CSR counterpart of magicpig_sparsetoken_flash_attention_decode_paged."""
    return _ops.sparse_decode_paged_csr(q, paged_kv_cache, kv_page_indptr, kv_page_indices, inds,
                                        ptr, return_lse=return_lse, max_nnz=max_nnz,
                                        lsh_k=K.float(), lsh_l=L.float())


to_csr = _ops.padded_to_csr

__all__ = [
    "sparsetoken_flash_attention_decode_csr",
    "sparsetoken_flash_attention_decode_paged_csr",
    "magicpig_sparsetoken_flash_attention_decode_paged_csr",
    "to_csr",
]
