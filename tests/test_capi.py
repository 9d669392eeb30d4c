"""The C-ABI library loads, exports every declared symbol and validates arguments.

No test here launches a kernel: argument checks return before any GPU call.
"""
import ctypes as C
import re
from pathlib import Path

import pytest
import torch

from attention_kernel_triton_amd import _native as N

HEADER = Path(__file__).resolve().parents[1] / "include" / "akt_amd.h"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(akt_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_symbols()
    assert "akt_decode_paged_fwd" in names and "akt_prefill_fwd" in names
    assert set(names) == set(N.exported_symbols())


def test_library_exports_every_declared_symbol():
    lib = N.load()
    for name in declared_symbols():
        assert hasattr(lib, name), name
    assert lib.akt_abi_version() == N.ABI_VERSION == 2


def _i64(*v):
    return (C.c_int64 * len(v))(*v)


def test_prefill_rejects_unsupported_head_dim():
    lib = N.load()
    s = _i64(4 * 96, 96, 96, 1)
    rc = lib.akt_prefill_fwd(None, None, None, None, 1, 4, 2, 4, 96, s, s, s, s, 0.1, 1, None, 0,
                             None)
    assert rc == 2 and b"head_dim" in lib.akt_last_error()


def test_prefill_rejects_bad_gqa_and_strides():
    lib = N.load()
    s = _i64(64 * 64, 64, 64, 1)
    rc = lib.akt_prefill_fwd(None, None, None, None, 1, 6, 4, 4, 64, s, s, s, s, 0.1, 1, None, 0,
                             None)
    assert rc == 1 and b"multiple" in lib.akt_last_error()
    bad = _i64(64 * 64, 64, 64, 2)
    rc = lib.akt_prefill_fwd(None, None, None, None, 1, 4, 4, 4, 64, bad, s, s, s, 0.1, 1, None,
                             0, None)
    assert rc == 1 and b"stride" in lib.akt_last_error()


def test_decode_paged_requires_workspace():
    lib = N.load()
    need = lib.akt_decode_paged_workspace_size(4, 8, 2, 128, 16, 100, 0)
    assert need > 0
    qs = _i64(8 * 128, 128, 128, 1)
    ks = _i64(2 * 2 * 16 * 128, 2 * 16 * 128, 16 * 128, 128, 1)
    rc = lib.akt_decode_paged_fwd(C.c_void_p(16), C.c_void_p(16), None, None, None,
                                  C.c_void_p(16), None, 4, 8, 2, 128, 16, 100, 100, qs, ks, 0.1,
                                  0, None, 0, None)
    assert rc == 3 and b"workspace" in lib.akt_last_error()


def test_sparse_rejects_unaligned_rows():
    lib = N.load()
    qs = _i64(32 * 128, 128, 128, 1)
    ks = _i64(8 * 100 * 128, 100 * 128, 128, 1)
    rc = lib.akt_sparse_decode_fwd(C.c_void_p(8), C.c_void_p(16), C.c_void_p(16), None, None,
                                   C.c_void_p(16), None, 1, 32, 8, 100, 128, 10, qs, ks, ks,
                                   _i64(320, 10), _i64(32, 1), 0.1, 0, None, 0, None)
    assert rc == 1 and b"aligned" in lib.akt_last_error()


def _ws(units, parts, gt, D):
    """Split-KV workspace layout: a 256-byte counter header; with partials, at
    least 32768 int32 arrival counters (one per unit), fp32 partial outputs
    [parts, gt, D] and their (m, l, e, pad) rows [parts, gt, 4], each array
    padded to 256 bytes."""
    if parts == 0:
        return 256
    ru = lambda x: -(-x // 256) * 256  # noqa: E731
    return 256 + ru(max(units, 32768) * 4) + ru(parts * gt * D * 4) + parts * gt * 16


def test_workspace_sizes_scale_with_problem():
    lib = N.load()
    a = lib.akt_decode_paged_workspace_size(32, 32, 8, 128, 16, 8448, 0)
    b = lib.akt_decode_paged_workspace_size(32, 32, 8, 128, 16, 2 * 8448, 0)
    assert 0 < a <= b
    # partials only when a unit has several chunks (8 x 16 units of 4 heads here)
    assert lib.akt_decode_workspace_size(8, 64, 16, 512, 64, 512) == _ws(128, 0, 4, 64) == 256
    assert lib.akt_decode_workspace_size(8, 64, 16, 1024, 64, 512) == _ws(128, 256, 4, 64)
    assert lib.akt_decode_workspace_size(4000, 64, 16, 1024, 64, 512) == _ws(64000, 128000, 4, 64)
    assert lib.akt_sparse_decode_workspace_size(1, 32, 128, 3840, 1) == _ws(32, 0, 1, 128)
    assert lib.akt_sparse_decode_workspace_size(1, 32, 128, 3840, 8) == _ws(32, 256, 1, 128)
    # nothing to compute: no workspace
    assert lib.akt_sparse_decode_workspace_size(0, 32, 128, 3840, 0) == 0


def test_automatic_chunk_length():
    """Automatic paged decode (chunk_tokens 0) with pages of whole 16-token
    groups runs the stream-K kernel: its workspace holds one partial slot per
    (wave + unit), with the waves at their 4096 maximum where no device can be
    queried (this CPU-only process).  Explicit chunk lengths keep the chunked
    kernel's layout, and dense decode keeps choosing its chunk (512 tokens for
    config 2)."""
    lib = N.load()
    ws = lib.akt_decode_paged_workspace_size
    # config 3: 32 sequences x 8 kv heads = 256 units of 4 heads, D = 128
    assert ws(32, 32, 8, 128, 16, 7208, 0) == _ws(256, 4096 + 256, 4, 128)
    assert ws(32, 32, 8, 128, 16, 7208, 0) != ws(32, 32, 8, 128, 16, 7208, 640)
    # pages of 8 tokens (not whole groups) keep the chunked kernel at 256 tokens
    assert ws(32, 32, 8, 128, 8, 7208, 0) == ws(32, 32, 8, 128, 8, 7208, 256)
    # config 2 (dense, 8 x 1024 tokens, 16 kv heads) stays at 512
    dws = lib.akt_decode_workspace_size
    assert dws(8, 64, 16, 1024, 64, 0) == dws(8, 64, 16, 1024, 64, 512)


def test_automatic_sparse_split_count():
    """Sparse rows get as many splits as fit one round of ~512 resident workgroups,
    at most 8 and at most one per 64 index slots of l_max; the workspace size shows
    the count."""
    lib = N.load()
    ws = lib.akt_sparse_decode_workspace_size
    part = lambda rows, ns, D: _ws(rows, rows * ns if ns > 1 else 0, 1, D)  # noqa: E731
    assert ws(1, 32, 128, 3840, 0) == part(32, 8, 128)       # config 4a: 512 / 32 rows, capped at 8
    assert ws(1, 64, 128, 3840, 0) == part(64, 8, 128)       # 512 / 64 rows
    assert ws(3, 32, 256, 32768, 0) == part(96, 5, 256)      # config 4b: 512 / 96 rows
    assert ws(1, 32, 128, 200, 0) == part(32, 4, 128)        # capped at ceil(200 / 64)
    assert ws(64, 32, 128, 3840, 0) == part(2048, 1, 128)    # 2048 rows: one split, no partials


def test_kept_index_rejects_short_row_stride():
    lib = N.load()
    rc = lib.akt_kept_index_from_mask(C.c_void_p(16), 4, 100, 50, None, C.c_void_p(16), 10,
                                      C.c_void_p(16), 1, None)
    assert rc == 1


def test_python_entry_points_validate_before_launch():
    import torch
    from attention_kernel_triton_amd import (decode_flash_attention_redundant as dec,
                                             prefill_flash_attention as pre)
    Q = torch.zeros(1, 4, 8, 64, dtype=torch.float16)
    K = torch.zeros(1, 2, 8, 64, dtype=torch.float16)
    with pytest.raises(AssertionError):
        pre.flash_attention_prefill(Q, K[:, :1], K, True, 0.1, 2)  # reference shape assert
    with pytest.raises(ValueError):
        pre.flash_attention_prefill(Q, K, K, True, 0.1, 2)  # CPU tensors are not accepted
    with pytest.raises(AssertionError):
        dec.flash_attention_decode(Q[:, :, :2], K, K, 0.1, 2)


def test_merge_states_validates_arguments():
    lib = N.load()
    s2 = _i64(0, 0)
    rc = lib.akt_merge_states(None, 0, None, None, 0, None, 2, 4, 12, s2, s2, 12, 1, None)
    assert rc == 1 and b"multiple of 8" in lib.akt_last_error()
    rc = lib.akt_merge_states(None, 5, None, None, 0, None, 2, 4, 64, s2, s2, 64, 1, None)
    assert rc == 1 and b"dtype" in lib.akt_last_error()
    rc = lib.akt_merge_states(None, 0, None, None, 0, None, 2, 0, 64, s2, s2, 64, 1, None)
    assert rc == 0  # no rows: nothing to do


def test_prefill_lse_requires_output():
    lib = N.load()
    s = _i64(64 * 64, 64, 64, 1)
    rc = lib.akt_prefill_fwd_lse(None, None, None, None, None, 1, 4, 4, 4, 64, s, s, s, s,
                                 _i64(16, 4, 1), 0.1, 1, None, 0, None)
    assert rc == 1 and b"lse" in lib.akt_last_error()


def test_prefill_ex_checks_dtype_and_allows_no_lse():
    lib = N.load()
    s = _i64(64 * 64, 64, 64, 1)
    rc = lib.akt_prefill_fwd_ex(None, None, None, None, None, 1, 4, 4, 4, 64, s, s, s, s, None,
                                0.1, 1, None, 0, 1, None)  # AKT_DTYPE_F32: not a prefill type
    assert rc == 1 and b"dtype" in lib.akt_last_error()
    for dtype in (0, 2):  # fp16, bf16: an empty batch launches nothing
        rc = lib.akt_prefill_fwd_ex(None, None, None, None, None, 0, 4, 4, 4, 64, s, s, s, s,
                                    None, 0.1, 1, None, 0, dtype, None)
        assert rc == 0, lib.akt_last_error()


def test_csr_entry_points_require_row_pointer():
    lib = N.load()
    s = _i64(4 * 64, 64, 64, 1)
    rc = lib.akt_sparse_decode_csr_fwd(None, None, None, None, None, None, None, 1, 4, 4, 10, 64,
                                       8, s, s, s, 0.1, 0, None, 0, None)
    assert rc == 1 and b"row pointer" in lib.akt_last_error()
    s5 = _i64(2 * 16 * 64, 16 * 64, 16 * 64, 64, 1)
    rc = lib.akt_sparse_decode_paged_csr_fwd(None, None, None, None, None, None, None, None, None,
                                             None, 1, 4, 4, 64, 16, 1, 8, s, s5, 0, None, 0, None)
    assert rc == 1 and b"row pointer" in lib.akt_last_error()


def test_paged_append_validates_arguments():
    lib = N.load()
    s3 = _i64(2 * 64, 64, 1)
    s5 = _i64(2 * 2 * 16 * 64, 2 * 16 * 64, 16 * 64, 64, 1)
    rc = lib.akt_paged_kv_append(None, None, None, None, None, None, None, 1, 4, 2, 60, 16, 8, s3,
                                 s3, s5, None)
    assert rc == 1 and b"multiple of 8" in lib.akt_last_error()
    rc = lib.akt_paged_kv_append(None, None, None, None, None, None, None, 1, 4, 2, 64, 16, 8, s3,
                                 s3, s5, None)
    assert rc == 1 and b"pointers" in lib.akt_last_error()
    rc = lib.akt_paged_kv_append(None, None, None, None, None, None, None, 1, 0, 2, 64, 16, 8, s3,
                                 s3, s5, None)
    assert rc == 0  # nothing to append


@pytest.mark.parametrize("batch,hq,hkv,dim,pages,chunk", [
    (256, 32, 8, 128, 400000, 640),  # chunked kernel: partials grow with the pages
    (1000, 256, 64, 256, 1000, 0),   # stream-K kernel: partials grow with the units
])
def test_noalloc_paged_decode_rejects_workspace_past_its_array(batch, hq, hkv, dim, pages, chunk):
    """The no-allocation entry point refuses, before any GPU call, a problem whose
    split-KV workspace exceeds its fixed device array (32 MiB)."""
    lib = N.load()
    need = lib.akt_decode_paged_workspace_size(batch, hq, hkv, dim, 16, pages, chunk)
    assert need > 32 << 20
    qs = _i64(hq * dim, dim, dim, 1)
    kvs = _i64(2 * hkv * 16 * dim, hkv * 16 * dim, 16 * dim, dim, 1)
    rc = lib.akt_decode_paged_fwd_noalloc(C.c_void_p(16), C.c_void_p(16), C.c_void_p(16),
                                          C.c_void_p(16), C.c_void_p(16), C.c_void_p(16), None,
                                          batch, hq, hkv, dim, 16, pages, pages, qs, kvs, 0.088,
                                          chunk, None)
    assert rc == 1 and b"no-allocation" in lib.akt_last_error()


def test_host_layer_rejects_mismatched_k_and_v():
    """K and V must have one shape that agrees with Q (batch, head dim and, for
    prefill, sequence length) before any kernel sizes a read from them.  The
    compiled host layer checks shapes before devices, so CPU tensors show it."""
    from attention_kernel_triton_amd import _ops
    Q = torch.zeros(1, 4, 8, 64, dtype=torch.float16)
    K = torch.zeros(1, 2, 8, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="one shape"):
        _ops.prefill(Q, K, K[:, :, :4], True, 0.1)
    with pytest.raises(ValueError, match="does not match Q"):
        _ops.prefill(Q, K[:, :, :4], K[:, :, :4], True, 0.1)
    with pytest.raises(ValueError, match="does not match Q"):
        _ops.prefill(Q, K[..., :32], K[..., :32], True, 0.1)
    q = torch.zeros(1, 4, 1, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="one shape"):
        _ops.decode(q, K, K[:, :, :4], 0.1)
    with pytest.raises(ValueError, match="does not match Q"):
        _ops.decode(q, torch.zeros(2, 2, 8, 64, dtype=torch.float16),
                    torch.zeros(2, 2, 8, 64, dtype=torch.float16), 0.1)
    ind = torch.zeros(1, 4, 8, dtype=torch.int32)
    nnz = torch.ones(1, 4, 1, dtype=torch.int32)
    with pytest.raises(ValueError, match="one shape"):
        _ops.sparse_decode(q, K, K[:, :1], ind, nnz, 0.1)
