"""Drop-in for magicpig_sparsetoken_decode_flash_attention_redundant_var_len_paged_with_norm.py.

``magicpig_sparsetoken_flash_attention_decode_paged`` keeps the reference
signature (magicpig_..._with_norm.py:166-209) and its MagicPIG score
(magicpig_..._with_norm.py:110-148, eq. 11 of the MagicPIG paper):
  score_i = q.k_i / sqrt(D) - ln(u_i),
  u_i = 1 - (1 - p_i^K)^L - L p_i^K (1 - p_i^K)^(L-1),
  p_i = 1 - arccos(q.k_i / (|q| |k_i| + 1e-8)) / pi,
with the reference's clamps, and per-(batch, q head) K, L (fp32 [B, Hq]).
u_i is evaluated in fp32 in a cancellation-free form: for x = p_i^K >= 0.05,
u = -expm1((L - 1) log1p(-x) + log1p((L - 1) x)); below, the series
sum_{k>=2} (k - 1) C(L, k) (-x)^k.  (The direct formula cancels
catastrophically when x is small or L is near 1.)  The reference returns
only O; this build also returns the
normaliser when ``return_lse=True``: lse[b, h] = ln sum_i exp(score_i) (fp32).
A head with nnz == 0 yields zeros (as the reference, magicpig:51-53) and
lse = -inf.
"""
from __future__ import annotations

from . import _ops


def magicpig_sparsetoken_flash_attention_decode_paged(q, paged_kv_cache, kv_page_indptr,
                                                      kv_page_indices, sparse_ind, sparse_nnz,
                                                      K, L, return_lse=False):
    """Returns O: [B, Hq, D] (and lse [B, Hq] when return_lse)."""
    return _ops.sparse_decode_paged(q, paged_kv_cache, kv_page_indptr, kv_page_indices,
                                    sparse_ind, sparse_nnz, return_lse=return_lse,
                                    lsh_k=K.float(), lsh_l=L.float())
