"""Tensor-level wrappers over the C ABI (include/akt_amd.h).

Each function validates devices, dtypes and layouts, allocates outputs and the
split-KV workspace through torch's caching allocator, and launches on the
current HIP stream of the input's device.  They never synchronise and never
fall back to another implementation.  The hot entry points run in the
compiled host layer (_akt_torch); the rest bind the C ABI through ctypes.
"""
from __future__ import annotations


import torch

from . import _native as N


def _need_gpu(name: str, t: torch.Tensor) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if not t.is_cuda:
        raise ValueError(f"{name} must be on a ROCm GPU device, got {t.device}")


def _half_rows(name: str, t: torch.Tensor) -> torch.Tensor:
    """fp16 tensor with unit innermost stride and 16-byte aligned rows."""
    _need_gpu(name, t)
    if t.dtype != torch.float16:
        raise TypeError(f"{name} must be float16, got {t.dtype}")
    ok = t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all(
        (s * 2) % 16 == 0 for s in t.stride()[:-1])
    return t if ok else t.contiguous()


def _int32(name: str, t: torch.Tensor, device) -> torch.Tensor:
    _need_gpu(name, t)
    if t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")
    if t.dtype != torch.int32:
        raise TypeError(f"{name} must be int32, got {t.dtype}")
    return t


def _same_device(dev, **tensors) -> None:
    for name, t in tensors.items():
        if t.device != dev:
            raise ValueError(f"{name} is on {t.device}, expected {dev}")


# --------------------------------------------------------------------------- hot paths
# prefill, decode, decode_paged, sparse_decode and sparse_decode_paged run in
# the compiled host layer (csrc/torch_ops.cpp): the same checks, allocation,
# stream and workspace handling as the wrappers below, at a few microseconds
# of host time per call.  The first call of each name binds this module's
# attribute to the compiled function.
_HOT = ("prefill", "decode", "decode_paged", "sparse_decode", "sparse_decode_paged")


def _hot(name):
    ext = N.torch_ext()
    g = globals()
    for n in _HOT:
        g[n] = getattr(ext, n)
    return getattr(ext, name)


def prefill(Q, K, V, causal, softmax_scale, varlen=None, return_lse=False):
    """O = softmax(scale * Q K^T [+ causal mask]) V for Q [B,Hq,S,D], K/V [B,Hkv,S,D].

    varlen: optional device int32/int64 [B] of valid lengths.  With
    return_lse, also the fp32 natural-log normaliser [B, Hq, S] of every
    computed row (rows a var-len call leaves unwritten stay uninitialised).
    """
    return _hot("prefill")(Q, K, V, causal, softmax_scale, varlen=varlen, return_lse=return_lse)


# --------------------------------------------------------------------------- merge
_DTYPE_CODE = {torch.float16: 0, torch.float32: 1}


def merge_states(o, lse, out_dtype=None):
    """Log-sum-exp merge of N partial attention states.

    o: [N, ..., D] fp16 or fp32 partial outputs over disjoint key sets;
    lse: [N, ...] fp32 natural-log normalisers.  Returns (o_merged [..., D]
    in out_dtype (default o's dtype), lse_merged [...] fp32).
    """
    _need_gpu("o", o)
    _need_gpu("lse", lse)
    _same_device(o.device, lse=lse)
    if o.dtype not in _DTYPE_CODE:
        raise TypeError(f"o must be float16 or float32, got {o.dtype}")
    if lse.dtype != torch.float32:
        raise TypeError(f"lse must be float32, got {lse.dtype}")
    if o.dim() < 2 or tuple(lse.shape) != tuple(o.shape[:-1]):
        raise ValueError(f"lse shape {tuple(lse.shape)} must equal o.shape[:-1] = "
                         f"{tuple(o.shape[:-1])}")
    out_dtype = o.dtype if out_dtype is None else out_dtype
    if out_dtype not in _DTYPE_CODE:
        raise TypeError(f"out_dtype must be float16 or float32, got {out_dtype}")
    n, D = o.shape[0], o.shape[-1]
    rest = tuple(o.shape[1:-1])
    rows = 1
    for r in rest:
        rows *= r
    o3 = o.reshape(n, rows, D)
    esz = o.element_size()
    if (o3.stride(-1) != 1 or o3.data_ptr() % 16 or any((s * esz) % 16 for s in o3.stride()[:2])):
        o3 = o3.contiguous()
    l2 = lse.reshape(n, rows)
    out = torch.empty(rest + (D,), dtype=out_dtype, device=o.device)
    lse_out = torch.empty(rest, dtype=torch.float32, device=o.device)
    lib = N.load()
    rc = lib.akt_merge_states(N.ptr(o3), _DTYPE_CODE[o.dtype], N.ptr(l2), N.ptr(out),
                              _DTYPE_CODE[out_dtype], N.ptr(lse_out), n, rows, D,
                              N.i64s(o3.stride(0), o3.stride(1)), N.i64s(l2.stride(0), l2.stride(1)),
                              D, 1, N.stream_of(o))
    N.check(rc, "akt_merge_states")
    return out, lse_out


# --------------------------------------------------------------------------- decode
def decode(q, K, V, softmax_scale, return_lse=False, chunk_tokens=0):
    """Single-query GQA decode: q [B,Hq,1,D], K/V [B,Hkv,S,D] -> o [B,Hq,1,D] (, lse [B,Hq])."""
    return _hot("decode")(q, K, V, softmax_scale, return_lse=return_lse,
                          chunk_tokens=chunk_tokens)


def decode_paged(q, paged_kv_cache, kv_page_indptr, kv_page_indices, kv_last_page_len,
                 softmax_scale=None, return_lse=False, chunk_tokens=0):
    """Paged decode: q [B,Hq,1,D] (or [B,Hq,D]), pool [P,2,Hkv,page,D] -> o [B,Hq,D]."""
    return _hot("decode_paged")(q, paged_kv_cache, kv_page_indptr, kv_page_indices,
                                kv_last_page_len, softmax_scale=softmax_scale,
                                return_lse=return_lse, chunk_tokens=chunk_tokens)


def sparse_decode(q, K, V, sparse_ind, sparse_nnz, softmax_scale, return_lse=False,
                  num_splits=0):
    """Sparse-token decode over dense K/V: returns o [B,Hq,1,D] (, lse [B,Hq])."""
    return _hot("sparse_decode")(q, K, V, sparse_ind, sparse_nnz, softmax_scale,
                                 return_lse=return_lse, num_splits=num_splits)


def sparse_decode_paged(q, paged_kv_cache, kv_page_indptr, kv_page_indices, sparse_ind,
                        sparse_nnz, softmax_scale=None, return_lse=False, num_splits=0,
                        lsh_k=None, lsh_l=None):
    """Sparse-token paged decode (plain, or MagicPIG when lsh_k/lsh_l are given)."""
    return _hot("sparse_decode_paged")(q, paged_kv_cache, kv_page_indptr, kv_page_indices,
                                       sparse_ind, sparse_nnz, softmax_scale=softmax_scale,
                                       return_lse=return_lse, num_splits=num_splits,
                                       lsh_k=lsh_k, lsh_l=lsh_l)


# --------------------------------------------------------------------------- CSR kept indices
def _csr_meta(inds, ptr, dev, rows):
    inds = _int32("inds", inds, dev).contiguous()
    _need_gpu("ptr", ptr)
    if ptr.device != dev:
        raise ValueError(f"ptr is on {ptr.device}, expected {dev}")
    if ptr.dtype != torch.int64:
        raise TypeError(f"ptr must be int64, got {ptr.dtype}")
    if ptr.dim() != 1 or ptr.numel() != rows + 1:
        raise ValueError(f"ptr must be [B*Hq + 1] = [{rows + 1}], got {tuple(ptr.shape)}")
    if inds.dim() != 1:
        raise ValueError("inds must be 1-D")
    if inds.numel() == 0:
        # Every row is empty; the C ABI still takes a valid pointer (never read).
        inds = torch.full((1,), -1, dtype=torch.int32, device=dev)
    return inds, ptr.contiguous()


def _max_nnz_hint(max_nnz, inds):
    # Without a device read the longest row is only bounded by the total.
    return int(max_nnz) if max_nnz is not None else int(inds.numel())


def sparse_decode_csr(q, K, V, inds, ptr, softmax_scale: float, return_lse: bool = False,
                      num_splits: int = 0, max_nnz=None):
    """Sparse-token decode over dense K/V with CSR kept indices (inds, ptr)."""
    q = _half_rows("q", q)
    K = _half_rows("K", K)
    V = _half_rows("V", V)
    dev = q.device
    _same_device(dev, K=K, V=V)
    B, Hq, _, D = q.shape
    Hkv, S = K.shape[1], K.shape[2]
    inds, ptr = _csr_meta(inds, ptr, dev, B * Hq)
    hint = _max_nnz_hint(max_nnz, inds)
    o = torch.empty((B, Hq, 1, D), dtype=q.dtype, device=dev)
    lse = torch.empty((B, Hq), dtype=torch.float32, device=dev) if return_lse else None
    lib = N.load()
    ws_n = lib.akt_sparse_decode_workspace_size(B, Hq, D, hint, num_splits)
    st = N.stream_of(q)
    ws = N.workspace(ws_n, dev, st)
    rc = lib.akt_sparse_decode_csr_fwd(N.ptr(q), N.ptr(K), N.ptr(V), N.ptr(inds), N.ptr(ptr),
                                       N.ptr(o), N.ptr(lse), B, Hq, Hkv, S, D, hint, N.strides(q),
                                       N.strides(K), N.strides(V), float(softmax_scale),
                                       num_splits, N.ptr(ws), ws_n, st)
    N.check(rc, "akt_sparse_decode_csr_fwd")
    return (o, lse) if return_lse else o


def sparse_decode_paged_csr(q, paged_kv_cache, kv_page_indptr, kv_page_indices, inds, ptr,
                            return_lse: bool = False, num_splits: int = 0, max_nnz=None,
                            lsh_k=None, lsh_l=None):
    """Sparse-token paged decode (MagicPIG when lsh_k/lsh_l given) with CSR kept indices."""
    q = _half_rows("q", q)
    pool = _half_rows("paged_kv_cache", paged_kv_cache)
    dev = q.device
    _same_device(dev, paged_kv_cache=pool)
    indptr = _int32("kv_page_indptr", kv_page_indptr, dev).contiguous()
    indices = _int32("kv_page_indices", kv_page_indices, dev).contiguous()
    B, Hq, D = q.shape[0], q.shape[1], q.shape[-1]
    q4 = q if q.dim() == 4 else q.unsqueeze(2)
    P, _, Hkv, page, Dc = pool.shape
    if Dc != D:
        raise ValueError(f"head_dim mismatch: q has {D}, cache has {Dc}")
    if indptr.numel() != B + 1:
        raise ValueError("kv_page_indptr must have B+1 entries")
    inds, ptr = _csr_meta(inds, ptr, dev, B * Hq)
    hint = _max_nnz_hint(max_nnz, inds)
    lk = ll = None
    if lsh_k is not None or lsh_l is not None:
        for name, t in (("K", lsh_k), ("L", lsh_l)):
            _need_gpu(name, t)
            if t.dtype != torch.float32 or tuple(t.shape) != (B, Hq):
                raise ValueError(f"MagicPIG {name} must be float32 [{B}, {Hq}]")
        lk, ll = lsh_k.contiguous(), lsh_l.contiguous()
    o = torch.empty((B, Hq, D), dtype=q.dtype, device=dev)
    lse = torch.empty((B, Hq), dtype=torch.float32, device=dev) if return_lse else None
    lib = N.load()
    ws_n = lib.akt_sparse_decode_workspace_size(B, Hq, D, hint, num_splits)
    st = N.stream_of(q)
    ws = N.workspace(ws_n, dev, st)
    rc = lib.akt_sparse_decode_paged_csr_fwd(N.ptr(q4), N.ptr(pool), N.ptr(indptr),
                                             N.ptr(indices), N.ptr(inds), N.ptr(ptr), N.ptr(lk),
                                             N.ptr(ll), N.ptr(o), N.ptr(lse), B, Hq, Hkv, D, page,
                                             P, hint, N.strides(q4), N.strides(pool), num_splits,
                                             N.ptr(ws), ws_n, st)
    N.check(rc, "akt_sparse_decode_paged_csr_fwd")
    return (o, lse) if return_lse else o


def padded_to_csr(sparse_ind, sparse_nnz, l_max: int | None = None):
    """(-1-padded [B, Hq, L] indices, counts [B, Hq(, 1)]) -> CSR (inds int32, ptr int64).

    Row u = b * Hq + h keeps sparse_ind[b, h, :nnz[b, h]] (counts clamped to
    [0, L], as the decode kernels do).  Device tensor ops; no host sync.
    """
    ind = sparse_ind
    B, Hq, L = ind.shape
    cnt = sparse_nnz.reshape(B * Hq).to(torch.int64).clamp(0, L if l_max is None else l_max)
    pos = torch.arange(L, device=ind.device).unsqueeze(0)
    keep = pos < cnt.unsqueeze(1)
    inds = ind.reshape(B * Hq, L)[keep].to(torch.int32)
    ptr = torch.zeros(B * Hq + 1, dtype=torch.int64, device=ind.device)
    ptr[1:] = torch.cumsum(cnt, 0)
    return inds, ptr


# --------------------------------------------------------------------------- kept-index
def kept_indices(l_max: int, mask=None, uniform=None, kept_ratio: float | None = None,
                 row_len=None, ensure_nonempty: bool = True):
    """Sorted kept-token index lists from a keep mask or uniform draws.

    mask: bool/uint8 [..., N]; or uniform: float32 [..., N] with kept_ratio
    (keep where uniform < kept_ratio).  row_len (int32 [...]) limits each row.
    Returns (sparse_ind int32 [..., l_max] padded with -1, sparse_nnz int32 [..., 1]).
    """
    # Runs in the compiled host layer (csrc/torch_ops.cpp): a few microseconds of
    # host time, less than the kernel's, so back-to-back calls keep the GPU busy.
    return N.torch_ext().kept_indices(int(l_max), mask=mask, uniform=uniform,
                                      kept_ratio=None if kept_ratio is None else float(kept_ratio),
                                      row_len=row_len, ensure_nonempty=bool(ensure_nonempty))
