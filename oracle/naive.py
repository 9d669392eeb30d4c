"""CPU restatement of the reference's naive attention paths (test infrastructure).

Each function follows one naive PyTorch implementation of the reference
repository, cited by file:line, operation for operation, but evaluated on the
CPU in ``dtype`` (float64 by default, float32 for the reference's own
precision) from the fp16 inputs, with no intermediate fp16 rounding.  Every
function also returns the natural-log softmax normaliser (LSE) of the scaled
scores, which the reference does not compute.

Pinning (tests/test_oracle_naive.py): scalar brute force on tiny shapes,
causal row 0 equals V row 0, identical keys give the mean of V, decode equals
one row of non-causal prefill, paged decode with an identity page table equals
dense decode, sparse decode with every token kept equals dense decode, index
order invariance, nnz=1 gives the V row, the reference's loop-vs-mask
cross-check, MagicPIG with L=1 reduces to plain sparse attention and with
K=1, L=2 to the closed form score - 2 ln p, and LSE = logsumexp of the scores.
"""
from __future__ import annotations

import math

import torch

F64 = torch.float64


def _cpu(t: torch.Tensor, dtype) -> torch.Tensor:
    return t.detach().to(device="cpu", dtype=dtype)


# --------------------------------------------------------------------------- prefill
def prefill(Q, K, V, causal, softmax_scale, GQA_group_size=1, dtype=F64, head_chunk=16,
            return_lse=False):
    """prefill_flash_attention.py:415-425 (reference_implementation).

    repeat_interleave GQA, P = Q K^T * scale, causal tril mask to -inf,
    softmax, P V.  Evaluated per (batch, head chunk) to bound memory.
    Returns O [B, H, S, D] in ``dtype``; with return_lse also the
    logsumexp of the masked scaled scores [B, H, S] (the reference's
    commented-out m + log(l) store, prefill_flash_attention.py:331-334).
    """
    B, H, S, D = Q.shape
    out = torch.empty((B, H, S, D), dtype=dtype)
    lse = torch.empty((B, H, S), dtype=dtype)
    mask = torch.tril(torch.ones((S, S), dtype=torch.bool)) if causal else None
    for b in range(B):
        for h0 in range(0, H, head_chunk):
            h1 = min(H, h0 + head_chunk)
            q = _cpu(Q[b, h0:h1], dtype)
            kv_idx = torch.arange(h0, h1) // GQA_group_size
            k = _cpu(K[b], dtype)[kv_idx]
            v = _cpu(V[b], dtype)[kv_idx]
            p = torch.matmul(q, k.transpose(-2, -1)) * softmax_scale
            if causal:
                p.masked_fill_(~mask, float("-inf"))
            lse[b, h0:h1] = torch.logsumexp(p, dim=-1)
            p = torch.softmax(p, dim=-1)
            out[b, h0:h1] = torch.matmul(p, v)
    return (out, lse) if return_lse else out


def prefill_varlen(Q, K, V, causal, softmax_scale, GQA_group_size, varlen, dtype=F64):
    """prefill_flash_attention_var_len_padding.py:428-438 then :447-450.

    The reference checks var-len prefill against dense attention over the
    padded tensors and zeroes rows >= varlen[b] in both outputs; this does
    the same.
    """
    out = prefill(Q, K, V, causal, softmax_scale, GQA_group_size, dtype)
    for b, L in enumerate(varlen.tolist()):
        out[b, :, int(L):] = 0.0
    return out


# --------------------------------------------------------------------------- decode
def _attend(q, k, v, scale):
    """q [.., D], k/v [.., n, D] -> (out [.., D], lse [..])."""
    s = torch.matmul(k, q.unsqueeze(-1)).squeeze(-1) * scale
    lse = torch.logsumexp(s, dim=-1)
    w = torch.softmax(s, dim=-1)
    return torch.matmul(w.unsqueeze(-2), v).squeeze(-2), lse


def decode(q, K, V, softmax_scale, GQA_group_size=1, dtype=F64):
    """decode_flash_attention_redundant.py:306-312.

    q [B, Hq, 1, D], K/V [B, Hkv, S, D] -> (O [B, Hq, 1, D], lse [B, Hq]).
    """
    q = _cpu(q, dtype)
    K = _cpu(K, dtype).repeat_interleave(GQA_group_size, dim=1)
    V = _cpu(V, dtype).repeat_interleave(GQA_group_size, dim=1)
    o, lse = _attend(q[:, :, 0], K, V, softmax_scale)
    return o.unsqueeze(2), lse


def naive_paged_attention(q, paged_kv_cache, kv_page_indptr, kv_page_indices, kv_last_page_len,
                          dtype=F64, softmax_scale=None):
    """decode_flash_attention_redundant_var_len_paged.py:278-329.

    For each sequence: concatenate its pages (the last one truncated to
    kv_last_page_len[b]), repeat kv heads for GQA, attend with scale 1/sqrt(D).
    A sequence without pages gives zeros and lse = -inf.
    Returns (O [B, Hq, D], lse [B, Hq]).
    """
    B, Hq, D = q.shape[0], q.shape[1], q.shape[-1]
    pool = _cpu(paged_kv_cache, dtype)
    Hkv, page = pool.shape[2], pool.shape[3]
    G = Hq // Hkv
    scale = 1.0 / math.sqrt(D) if softmax_scale is None else softmax_scale
    indptr = kv_page_indptr.cpu().tolist()
    indices = kv_page_indices.cpu().to(torch.int64)
    last = kv_last_page_len.cpu().tolist()
    qv = _cpu(q, dtype).reshape(B, Hq, D)
    out = torch.zeros((B, Hq, D), dtype=dtype)
    lse = torch.full((B, Hq), float("-inf"), dtype=dtype)
    for b in range(B):
        s, e = indptr[b], indptr[b + 1]
        if s == e:
            continue
        pages = indices[s:e]
        k = pool[pages, 0]  # [n, Hkv, page, D]
        v = pool[pages, 1]
        ll = min(max(int(last[b]), 0), page)
        n = e - s
        k = torch.cat([k[:-1].permute(1, 0, 2, 3).reshape(Hkv, (n - 1) * page, D),
                       k[-1, :, :ll]], dim=1)
        v = torch.cat([v[:-1].permute(1, 0, 2, 3).reshape(Hkv, (n - 1) * page, D),
                       v[-1, :, :ll]], dim=1)
        if k.shape[1] == 0:
            continue
        k = k.repeat_interleave(G, dim=0)
        v = v.repeat_interleave(G, dim=0)
        out[b], lse[b] = _attend(qv[b], k, v, scale)
    return out, lse


# --------------------------------------------------------------------------- sparse
def sparsetoken_naive_decode(q, K, V, sparse_ind, sparse_nnz, softmax_scale, GQA_group_size,
                             dtype=F64):
    """sparsetoken_decode_flash_attention_redundant.py:173-202.

    Per (b, h): gather the kept rows K[b, h // G, ind[:nnz]] and attend.  As
    in the reference, nnz == 0 is treated as nnz = 1 (so index ind[b, h, 0] is
    used, which is -1 padding -> the last token under torch indexing).
    Returns (O [B, Hq, 1, D], lse [B, Hq]).
    """
    B, Hq, _, D = q.shape
    Kc, Vc, qc = _cpu(K, dtype), _cpu(V, dtype), _cpu(q, dtype)
    ind = sparse_ind.cpu().to(torch.int64)
    nnz = sparse_nnz.cpu().reshape(B, Hq)
    out = torch.zeros((B, Hq, 1, D), dtype=dtype)
    lse = torch.zeros((B, Hq), dtype=dtype)
    for b in range(B):
        for h in range(Hq):
            n = int(nnz[b, h])
            if n == 0:
                n = 1
            idx = ind[b, h, :n]
            kh = h // GQA_group_size
            out[b, h, 0], lse[b, h] = _attend(qc[b, h, 0], Kc[b, kh, idx], Vc[b, kh, idx],
                                              softmax_scale)
    return out, lse


def sparsetoken_naive_decode_by_mask(q, K, V, mask, softmax_scale, GQA_group_size, dtype=F64):
    """sparsetoken_decode_flash_attention_redundant.py:204-230 (dense attention, masked).

    mask: bool [B, Hq, S] of kept positions.  Returns (O [B, Hq, 1, D], lse [B, Hq]).
    """
    qc = _cpu(q, dtype)
    Kc = _cpu(K, dtype).repeat_interleave(GQA_group_size, dim=1)
    Vc = _cpu(V, dtype).repeat_interleave(GQA_group_size, dim=1)
    s = torch.matmul(qc, Kc.transpose(-2, -1)) * softmax_scale
    s = s.masked_fill(~mask.cpu().unsqueeze(2), float("-inf"))
    lse = torch.logsumexp(s, dim=-1).squeeze(-1)
    return torch.matmul(torch.softmax(s, dim=-1), Vc), lse


def _paged_rows(pool, indptr_b, indices, token_idx, page, kvh, which):
    page_idx = token_idx // page
    slot = token_idx % page
    page_id = indices[indptr_b + page_idx]
    return pool[page_id, which, kvh, slot]


def sparsetoken_naive_paged_attention(q, paged_kv_cache, kv_page_indptr, kv_page_indices,
                                      sparse_ind, sparse_nnz, dtype=F64, softmax_scale=None):
    """sparsetoken_decode_flash_attention_redundant_var_len_paged.py:234-288.

    Per (b, h): kept token t lives in page indices[indptr[b] + t // page],
    slot t % page; nnz == 0 gives zeros (lse = -inf).  Scale 1/sqrt(D).
    Returns (O [B, Hq, D], lse [B, Hq]).
    """
    B, Hq, D = q.shape[0], q.shape[1], q.shape[-1]
    pool = paged_kv_cache.detach().cpu()  # rows are converted to `dtype` once gathered
    Hkv, page = pool.shape[2], pool.shape[3]
    G = Hq // Hkv
    scale = 1.0 / math.sqrt(D) if softmax_scale is None else softmax_scale
    qc = _cpu(q, dtype).reshape(B, Hq, D)
    indptr = kv_page_indptr.cpu().to(torch.int64)
    indices = kv_page_indices.cpu().to(torch.int64)
    ind = sparse_ind.cpu().to(torch.int64)
    nnz = sparse_nnz.cpu().reshape(B, Hq)
    out = torch.zeros((B, Hq, D), dtype=dtype)
    lse = torch.full((B, Hq), float("-inf"), dtype=dtype)
    for b in range(B):
        for h in range(Hq):
            n = int(nnz[b, h])
            if n == 0:
                continue
            t = ind[b, h, :n]
            k = _paged_rows(pool, indptr[b], indices, t, page, h // G, 0).to(dtype)
            v = _paged_rows(pool, indptr[b], indices, t, page, h // G, 1).to(dtype)
            out[b, h], lse[b, h] = _attend(qc[b, h], k, v, scale)
    return out, lse


def magicpig_scores(q, k, K_val, L_val, head_dim, dtype=F64):
    """MagicPIG score of each kept row (magicpig_..._with_norm.py:252-283).

    q [D], k [n, D] (already in ``dtype``) -> score [n] = q.k/sqrt(D) - ln(u),
    u = clamp(1 - (1-x)^L - L x (1-x)^(L-1), min=1e-10), x = p^K,
    p = clamp(1 - acos(clamp(q.k / (|q||k| + 1e-8), -1+1e-7, 1-1e-7)) / pi, 0, 1).
    """
    s = torch.matmul(k, q)
    qn = torch.linalg.vector_norm(q)
    kn = torch.linalg.vector_norm(k, dim=-1)
    c = torch.clamp(s / (qn * kn + 1e-8), -1.0 + 1e-7, 1.0 - 1e-7)
    p = torch.clamp(1.0 - (1.0 / math.pi) * torch.acos(c), 0.0, 1.0)
    x = torch.pow(p, K_val)
    om = torch.clamp(1.0 - x, 0.0, 1.0)
    u = 1.0 - torch.pow(om, L_val) - L_val * x * torch.pow(om, L_val - 1.0)
    u = torch.clamp(u, min=1e-10)
    return s / math.sqrt(head_dim) - torch.log(u)


def magicpig_sparsetoken_naive_paged_attention(q, paged_kv_cache, kv_page_indptr,
                                               kv_page_indices, sparse_ind, sparse_nnz, K, L,
                                               dtype=F64):
    """magicpig_..._with_norm.py:212-291, with the normaliser added.

    ``dtype=torch.float32`` evaluates in the reference's precision;
    float64 gives the exactly-rounded answer used for parity.
    Returns (O [B, Hq, D], lse [B, Hq]) with lse = ln sum_i exp(score_i).
    """
    B, Hq, D = q.shape[0], q.shape[1], q.shape[-1]
    pool = paged_kv_cache.detach().cpu()  # rows are converted to `dtype` once gathered
    Hkv, page = pool.shape[2], pool.shape[3]
    G = Hq // Hkv
    qc = _cpu(q, dtype).reshape(B, Hq, D)
    indptr = kv_page_indptr.cpu().to(torch.int64)
    indices = kv_page_indices.cpu().to(torch.int64)
    ind = sparse_ind.cpu().to(torch.int64)
    nnz = sparse_nnz.cpu().reshape(B, Hq)
    Kc, Lc = K.cpu().to(dtype), L.cpu().to(dtype)
    out = torch.zeros((B, Hq, D), dtype=dtype)
    lse = torch.full((B, Hq), float("-inf"), dtype=dtype)
    for b in range(B):
        for h in range(Hq):
            n = int(nnz[b, h])
            if n == 0:
                continue
            t = ind[b, h, :n]
            k = _paged_rows(pool, indptr[b], indices, t, page, h // G, 0).to(dtype)
            v = _paged_rows(pool, indptr[b], indices, t, page, h // G, 1).to(dtype)
            sc = magicpig_scores(qc[b, h], k, Kc[b, h], Lc[b, h], D, dtype)
            lse[b, h] = torch.logsumexp(sc, dim=0)
            out[b, h] = torch.matmul(torch.softmax(sc, dim=0), v)
    return out, lse


# --------------------------------------------------------------------------- merge
def merge_states(o, lse, dtype=F64):
    """Log-sum-exp merge of N partial states (no reference counterpart; the
    combine implied by the stubbed LSE stores, prefill_flash_attention.py:331-334).

    o: [N, ..., D], lse: [N, ...].  Returns (sum_i w_i o_i, ln sum_i exp(lse_i))
    with w_i = exp(lse_i - LSE); rows with every lse_i = -inf give (0, -inf).
    """
    o = _cpu(o, dtype)
    lse = _cpu(lse, dtype)
    total = torch.logsumexp(lse, dim=0)
    w = torch.exp(lse - total.unsqueeze(0))
    w = torch.where(torch.isfinite(total).unsqueeze(0), w, torch.zeros_like(w))
    out = (w.unsqueeze(-1) * o).sum(dim=0)
    return out, total
