"""gfx950 (MI355X) attention kernels with the reference's Python entry points.

Modules mirror the reference repository's files (KiritoHugh/attention_kernel_triton):

  prefill_flash_attention                       flash_attention_prefill
  prefill_flash_attention_var_len_padding       flash_attention_prefill(varlen=)
  decode_flash_attention_redundant              flash_attention_decode
  decode_flash_attention_redundant_var_len_paged  flash_attention_decode_paged
  sparsetoken_decode_flash_attention_redundant  sparsetoken_flash_attention_decode
  sparsetoken_decode_flash_attention_redundant_var_len_paged
                                                sparsetoken_flash_attention_decode_paged
  magicpig_sparsetoken_decode_flash_attention_redundant_var_len_paged_with_norm
                                                magicpig_sparsetoken_flash_attention_decode_paged
  kept_index                                    select_kept (device kept-index selection)
  merge_states                                  merge_states (LSE merge of partial results)
  sparse_csr                                    sparse decodes over CSR kept indices (inds + ptr)
  paged_kv                                      append_paged_kv, PagedKVCache (paged KV write side)

All of them run hand-written HIP kernels from libakt_amd.so (built by
``python -m attention_kernel_triton_amd.build``) through its C ABI.
"""
from . import _native  # noqa: F401

__all__ = [
    "prefill_flash_attention",
    "prefill_flash_attention_var_len_padding",
    "decode_flash_attention_redundant",
    "decode_flash_attention_redundant_var_len_paged",
    "sparsetoken_decode_flash_attention_redundant",
    "sparsetoken_decode_flash_attention_redundant_var_len_paged",
    "magicpig_sparsetoken_decode_flash_attention_redundant_var_len_paged_with_norm",
    "kept_index",
    "merge_states",
    "sparse_csr",
    "paged_kv",
]
