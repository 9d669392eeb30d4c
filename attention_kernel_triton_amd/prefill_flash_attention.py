"""Drop-in for the reference module prefill_flash_attention.py.

``flash_attention_prefill`` keeps the reference signature, asserts and output
allocation (prefill_flash_attention.py:342-383); the work runs in the gfx950
MFMA kernel ``akt_prefill_fwd_ex`` (csrc/prefill.hip).  The reference's tile-size
environment variables (VAR_Q_SEQ_BLK_SIZE, VAR_KV_SEQ_BLK_SIZE) are accepted
and ignored: results never depend on them.
"""
from __future__ import annotations

from . import _ops


def flash_attention_prefill(Q, K, V, causal, softmax_scale, GQA_group_size=1, *,
                            return_lse=False):
    """O = softmax(softmax_scale * Q K^T [+ causal mask]) V.

    Q: [B, H, S, D]; K, V: [B, H // GQA_group_size, S, D]; fp16 on a ROCm GPU
    (the reference's type), or all three bf16 (bf16 MFMA, P rounded to bf16).
    Query head h attends kv head h // GQA_group_size (prefill_flash_attention.py:185).
    Returns O: [B, H, S, D] in Q's dtype; with the opt-in return_lse=True, the
    pair (O, LSE) where LSE [B, H, S] fp32 = ln sum_k exp(softmax_scale * q.k)
    (the quantity the reference's commented-out store at
    prefill_flash_attention.py:331-334 would have written).
    """
    B, H, S, D = Q.shape
    assert K.shape == (B, H // GQA_group_size, S, D)
    assert V.shape == (B, H // GQA_group_size, S, D)
    assert D % 64 == 0, "HEAD_DIM must be a multiple of 64?"
    return _ops.prefill(Q, K, V, causal, softmax_scale, return_lse=return_lse)
