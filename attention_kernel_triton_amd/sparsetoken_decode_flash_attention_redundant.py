"""Drop-in for the reference module sparsetoken_decode_flash_attention_redundant.py.

``sparsetoken_flash_attention_decode`` keeps the reference signature
(sparsetoken_decode_flash_attention_redundant.py:127-170): query head h of
batch b attends only the kept tokens sparse_ind[b, h, :sparse_nnz[b, h]] of
its kv head h // GQA_group_size.  sparse_ind is int32 [B, Hq, L_max] (-1
padded), sparse_nnz int32 [B, Hq, 1].  Only the kept K/V rows are read.
Indices follow torch indexing as in the reference's PyTorch path (-S <= i < 0
names row S + i), and a head with nnz == 0 attends to its first index slot,
as that path does (:191-194: with -1 padding, the last token); the
reference's Triton kernel yields NaN there.  Indices outside [-S, S) are
skipped.  ``return_lse=True`` also returns the fp32 log-sum-exp [B, Hq].
"""
from __future__ import annotations

from . import _ops

redundant_len = 16  # kept for import compatibility; the kernel does not replicate q


def sparsetoken_flash_attention_decode(q, K, V, sparse_ind, sparse_nnz, softmax_scale,
                                       GQA_group_size, return_lse=False):
    """Returns O: [B, Hq, 1, D] (and lse [B, Hq] when return_lse)."""
    B, Hq = q.shape[0], q.shape[1]
    assert Hq % K.shape[1] == 0 and Hq // K.shape[1] == GQA_group_size
    return _ops.sparse_decode(q, K, V, sparse_ind, sparse_nnz, softmax_scale,
                              return_lse=return_lse)
