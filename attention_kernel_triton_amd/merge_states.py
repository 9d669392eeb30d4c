"""Log-sum-exp merge of partial attention states (no reference module).

The reference computes per-row softmax normalisers inside its kernels but
leaves their stores commented out (prefill_flash_attention.py:331-334,
decode_flash_attention_redundant.py:225-228).  This build returns them
(``return_lse=True`` on every prefill and decode entry point); ``merge_states``
joins results computed over disjoint key sets -- chunks of a long context,
or per-GPU shards -- into the result over their union:

    LSE = ln sum_i exp(LSE_i),   O = sum_i exp(LSE_i - LSE) O_i

It runs the HIP kernel ``akt_merge_states`` (csrc/merge.hip).
"""
from __future__ import annotations

from ._ops import merge_states

__all__ = ["merge_states"]
