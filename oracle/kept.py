"""Kept-index selection and page addressing on the CPU (test infrastructure).

Integer restatements, in numpy, of:
  * the reference harness's kept-index construction
    (sparsetoken_decode_flash_attention_redundant.py:283-295,
     sparsetoken_decode_flash_attention_redundant_var_len_paged.py:341-353,
     magicpig_..._with_norm.py:327-338): keep = u < p; if nothing is kept,
    keep index 0; indices ascending; -1 padding; nnz = count;
  * the paged address translation token t of sequence b ->
    (indices[indptr[b] + t // page], t % page)
    (decode_flash_attention_redundant_var_len_paged.py:168-178,
     sparsetoken_decode_flash_attention_redundant_var_len_paged.py:115-126).

Pinning (tests/test_oracle_kept.py): brute-force Python loops on small rows,
torch.nonzero agreement, and the reference's fixed page-table fixtures.
"""
from __future__ import annotations

import numpy as np


def kept_indices(keep: np.ndarray, l_max: int, row_len=None, ensure_nonempty: bool = True):
    """keep: bool [rows, N] -> (ind int32 [rows, l_max] -1 padded, nnz int32 [rows]).

    Only the first row_len[r] candidates of row r are considered.
    """
    keep = np.asarray(keep, dtype=bool)
    rows, n = keep.shape
    ind = np.full((rows, l_max), -1, dtype=np.int32)
    nnz = np.zeros(rows, dtype=np.int32)
    for r in range(rows):
        nr = n if row_len is None else int(min(max(row_len[r], 0), n))
        idx = np.flatnonzero(keep[r, :nr]).astype(np.int32)
        if idx.size == 0 and ensure_nonempty:
            idx = np.zeros(1, dtype=np.int32)
        m = min(idx.size, l_max)
        ind[r, :m] = idx[:m]
        nnz[r] = idx.size
    return ind, nnz


def kept_from_uniform(uniform: np.ndarray, kept_ratio: float, l_max: int, row_len=None,
                      ensure_nonempty: bool = True):
    """uniform float32 [rows, N]: keep where uniform < float32(kept_ratio)."""
    u = np.asarray(uniform, dtype=np.float32)
    return kept_indices(u < np.float32(kept_ratio), l_max, row_len, ensure_nonempty)


def paged_token_address(indptr: np.ndarray, indices: np.ndarray, b: int, t, page: int):
    """Physical (page id, slot) of logical token(s) t of sequence b."""
    t = np.asarray(t, dtype=np.int64)
    return indices[indptr[b] + t // page].astype(np.int64), t % page


def paged_seq_len(indptr: np.ndarray, last_len: np.ndarray, b: int, page: int) -> int:
    """Tokens of sequence b: (pages - 1) * page + last_page_len (0 without pages)."""
    n = int(indptr[b + 1] - indptr[b])
    if n <= 0:
        return 0
    return (n - 1) * page + int(min(max(last_len[b], 0), page))


def paged_append(pool: np.ndarray, k_new: np.ndarray, v_new: np.ndarray,
                 append_indptr: np.ndarray, indptr: np.ndarray, indices: np.ndarray,
                 last_len: np.ndarray) -> np.ndarray:
    """Write side of the paged layout (no reference counterpart; the reference's
    tests build page tables by hand, decode_flash_attention_redundant_var_len_paged.py:349-353).

    pool: [P, 2, Hkv, page, D]; k_new / v_new: [total_new, Hkv, D].  Sequence
    b's new rows append_indptr[b]:append_indptr[b+1] become its last logical
    positions under the (updated) table; positions / page ids outside the
    table or pool are skipped.  Returns the updated copy of the pool.
    """
    out = pool.copy()
    P, page = pool.shape[0], pool.shape[3]
    B = len(indptr) - 1
    for b in range(B):
        a0, a1 = int(append_indptr[b]), int(append_indptr[b + 1])
        n_new = a1 - a0
        length = paged_seq_len(indptr, last_len, b, page)
        for j in range(n_new):
            t = length - n_new + j
            if t < 0 or t >= length:
                continue
            pid, slot = paged_token_address(indptr, indices, b, t, page)
            pid, slot = int(pid), int(slot)
            if 0 <= pid < P:
                out[pid, 0, :, slot] = k_new[a0 + j]
                out[pid, 1, :, slot] = v_new[a0 + j]
    return out
