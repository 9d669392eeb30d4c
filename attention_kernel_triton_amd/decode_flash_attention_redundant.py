"""Drop-in for the reference module decode_flash_attention_redundant.py.

``flash_attention_decode`` keeps the reference signature and result shape
(decode_flash_attention_redundant.py:233-271) but does not replicate q to 16
rows: the gfx950 split-KV kernel (csrc/decode.hip) serves all query heads of a
kv head from one read of K/V.  ``return_lse=True`` additionally returns the
natural-log softmax normaliser [B, Hq] (fp32) of the scaled scores.
"""
from __future__ import annotations

from . import _ops


def flash_attention_decode(q, K, V, softmax_scale, GQA_group_size=1, return_lse=False):
    """q: [B, Hkv*G, 1, D]; K, V: [B, Hkv, S, D] -> O: [B, Hkv*G, 1, D]."""
    B, H, S, D = K.shape
    assert q.shape == (B, H * GQA_group_size, 1, D)
    assert V.shape == (B, H, S, D)
    assert D % 64 == 0, "HEAD_DIM must be a multiple of 64?"
    return _ops.decode(q, K, V, softmax_scale, return_lse=return_lse)
