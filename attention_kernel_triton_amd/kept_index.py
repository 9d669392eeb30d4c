"""Device-side kept-token index selection.

The reference builds sparse index lists in its test harness with a Python loop
over (batch, head) (sparsetoken_decode_flash_attention_redundant.py:283-295,
sparsetoken_decode_flash_attention_redundant_var_len_paged.py:341-353):
keep = rand(n) < p; keep index 0 if nothing is kept; indices =
nonzero(keep) ascending, -1 padded to L_max; nnz = count.  ``select_kept``
produces the same int32 arrays in one kernel launch (csrc/kept_index.hip),
bit-exact with torch.nonzero.
"""
from __future__ import annotations

from . import _ops


def select_kept(l_max, mask=None, uniform=None, kept_ratio=None, row_len=None,
                ensure_nonempty=True):
    """Returns (sparse_ind int32 [..., l_max], sparse_nnz int32 [..., 1]).

    Pass either ``mask`` (bool/uint8 [..., N]) or ``uniform`` (float32 [..., N])
    with ``kept_ratio``.  ``row_len`` (int32, one per row) limits each row's
    candidates to its first row_len entries.
    """
    return _ops.kept_indices(l_max, mask=mask, uniform=uniform, kept_ratio=kept_ratio,
                             row_len=row_len, ensure_nonempty=ensure_nonempty)
