"""Drop-in for the reference module prefill_flash_attention_var_len_padding.py.

``flash_attention_prefill(..., varlen=)`` keeps the reference signature
(prefill_flash_attention_var_len_padding.py:348-391).  ``varlen`` is a device
int32/int64 tensor [B] of valid lengths of right-padded sequences.  As in the
reference, query rows are processed in 64-row blocks up to
ceil(varlen[b] / 64) * 64 and rows in later blocks are left unwritten; rows at
or beyond varlen[b] are unspecified.  With causal=True a valid row never sees
padding (padding K/V rows are never staged: zeros are read in their place, so
non-finite padding cannot leak through P.V either); with
causal=False every row attends all S keys, padding included, exactly like
the reference.
``varlen=None`` means every sequence has length S.
"""
from __future__ import annotations

from . import _ops


def flash_attention_prefill(Q, K, V, causal, softmax_scale, GQA_group_size=1, varlen=None, *,
                            return_lse=False):
    """Var-len padded prefill; see the module docstring for the padding contract.

    With the opt-in return_lse=True returns (O, LSE [B, H, S] fp32); LSE rows
    that O leaves unwritten are unwritten too.
    """
    B, H, S, D = Q.shape
    assert K.shape == (B, H // GQA_group_size, S, D)
    assert V.shape == (B, H // GQA_group_size, S, D)
    assert D % 64 == 0, "HEAD_DIM must be a multiple of 64?"
    return _ops.prefill(Q, K, V, causal, softmax_scale, varlen=varlen, return_lse=return_lse)
