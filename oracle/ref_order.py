"""The reference's naive paths in their own operation order and dtypes (CPU baseline).

TEST INFRASTRUCTURE: only bench.py's ``cpu_baseline`` legs call these, to time
the reference's naive PyTorch implementations on the host CPU beside the GPU
kernels.  The parity oracle is ``oracle.naive`` (fp64, no intermediate fp16
rounding); the functions here keep the reference's fp16 tensors, its fp16
matmuls, its ``softmax(P.float()).half()`` (dense paths) or fp16 softmax
(paged paths), its Python loops and its per-token ``.item()`` gathers, so what
is timed is the reference's algorithm as written, on the CPU.

Pinning: tests/test_oracle_ref_order.py checks each function against
``oracle.naive`` (fp64) on small seeded inputs within fp16 rounding, and the
per-token gather loops against the vectorised gathers of ``oracle.naive``.
"""
from __future__ import annotations

import math

import torch


def prefill(Q, K, V, causal, softmax_scale, GQA_group_size=1):
    """prefill_flash_attention.py:415-425 (reference_implementation), fp16 on the CPU.

    The var-len reference (prefill_flash_attention_var_len_padding.py:427-437)
    is the same function; its harness zeroes rows >= length afterwards
    (:447-450), which ``prefill_varlen`` adds."""
    S = Q.shape[2]
    mask = torch.tril(torch.ones((S, S))) if causal else None
    if GQA_group_size > 1:
        K = K.repeat_interleave(GQA_group_size, dim=1)
        V = V.repeat_interleave(GQA_group_size, dim=1)
    P = torch.matmul(Q, K.transpose(-2, -1)) * softmax_scale
    if causal:
        P[:, :, mask == 0] = float("-inf")
    P = torch.softmax(P.float(), dim=-1).half()
    return torch.matmul(P, V)


def prefill_varlen(Q, K, V, causal, softmax_scale, GQA_group_size, varlen):
    """The var-len harness: the dense reference, then rows >= length set to zero
    (prefill_flash_attention_var_len_padding.py:427-450)."""
    O = prefill(Q, K, V, causal, softmax_scale, GQA_group_size)
    for i, L in enumerate(varlen.tolist()):
        O[i, :, int(L):, :] = 0.0
    return O


def decode(q, K, V, softmax_scale, GQA_group_size=1):
    """decode_flash_attention_redundant.py:306-312 (reference_implementation)."""
    if GQA_group_size > 1:
        K = K.repeat_interleave(GQA_group_size, dim=1)
        V = V.repeat_interleave(GQA_group_size, dim=1)
    P = torch.matmul(q, K.transpose(-2, -1)) * softmax_scale
    P = torch.softmax(P.float(), dim=-1).half()
    return torch.matmul(P, V)


def naive_paged_attention(q, paged_kv_cache, kv_page_indptr, kv_page_indices, kv_last_page_len):
    """decode_flash_attention_redundant_var_len_paged.py:278-329: per sequence, the
    pages are concatenated (the last one cut to its length), GQA by
    repeat_interleave, then fp16 scores / sqrt(D), fp16 softmax, fp16 P.V."""
    B, Hq, D = q.shape[0], q.shape[1], q.shape[3]
    Hkv = paged_kv_cache.shape[2]
    k_cache, v_cache = paged_kv_cache[:, 0], paged_kv_cache[:, 1]
    outputs = []
    for b in range(B):
        start, end = kv_page_indptr[b].item(), kv_page_indptr[b + 1].item()
        if start == end:
            outputs.append(torch.zeros_like(q[b:b + 1]).squeeze(2))
            continue
        pages = kv_page_indices[start:end]
        ks, vs = [], []
        for i, pid in enumerate(pages):
            kp, vp = k_cache[pid], v_cache[pid]
            if i == len(pages) - 1:
                last = kv_last_page_len[b].item()
                kp, vp = kp[:, :last, :], vp[:, :last, :]
            ks.append(kp)
            vs.append(vp)
        k = torch.cat(ks, dim=1)
        v = torch.cat(vs, dim=1)
        if Hq != Hkv:
            k = k.repeat_interleave(Hq // Hkv, dim=0)
            v = v.repeat_interleave(Hq // Hkv, dim=0)
        scores = torch.matmul(q[b], k.permute(0, 2, 1)) / math.sqrt(D)
        w = torch.softmax(scores, dim=-1)
        outputs.append(torch.matmul(w, v).squeeze(1).unsqueeze(0))
    return torch.cat(outputs, dim=0)


def sparsetoken_naive_decode(q, K, V, sparse_ind, sparse_nnz, softmax_scale, GQA_group_size):
    """sparsetoken_decode_flash_attention_redundant.py:173-202: a loop over (b, h)
    with an .item() count, an index gather of K and V rows, fp16 scores and
    softmax, fp16 P.V."""
    B, Hq, _, D = q.shape
    out = torch.zeros((B, Hq, 1, D), dtype=q.dtype)
    for b in range(B):
        for h in range(Hq):
            kh = h // GQA_group_size
            n = sparse_nnz[b, h].item()
            if n == 0:
                n = 1
            idx = sparse_ind[b, h, :n]
            kv, vv = K[b, kh, idx], V[b, kh, idx]
            s = torch.matmul(kv, q[b, h, 0]) * softmax_scale
            p = torch.softmax(s, dim=0)
            out[b, h, 0] = torch.matmul(p.unsqueeze(0), vv)
    return out


def _token_rows(k_cache, v_cache, kv_page_indptr, kv_page_indices, indices, b, kvh, page):
    """The reference's per-token gather (…_var_len_paged.py:270-276): one .item()
    token index, its page id through the CSR table, one [1, D] slice of K and V
    per kept token, concatenated."""
    ks, vs = [], []
    for i in range(indices.shape[0]):
        t = indices[i].item()
        pid = kv_page_indices[kv_page_indptr[b].item() + t // page]
        off = t % page
        ks.append(k_cache[pid, kvh, off:off + 1, :])
        vs.append(v_cache[pid, kvh, off:off + 1, :])
    return torch.cat(ks, dim=0).unsqueeze(0), torch.cat(vs, dim=0).unsqueeze(0)


def sparsetoken_naive_paged_attention(q, paged_kv_cache, kv_page_indptr, kv_page_indices,
                                      sparse_ind, sparse_nnz):
    """sparsetoken_decode_flash_attention_redundant_var_len_paged.py:234-288."""
    B, Hq, D = q.shape[0], q.shape[1], q.shape[3]
    Hkv, page = paged_kv_cache.shape[2], paged_kv_cache.shape[3]
    G = Hq // Hkv
    k_cache, v_cache = paged_kv_cache[:, 0], paged_kv_cache[:, 1]
    outputs = []
    for b in range(B):
        rows = []
        for h in range(Hq):
            n = sparse_nnz[b, h].item()
            if n == 0:
                rows.append(torch.zeros((1, D), dtype=q.dtype))
                continue
            k, v = _token_rows(k_cache, v_cache, kv_page_indptr, kv_page_indices,
                               sparse_ind[b, h, :n], b, h // G, page)
            scores = torch.matmul(q[b, h:h + 1], k.permute(0, 2, 1)) / math.sqrt(D)
            w = torch.softmax(scores, dim=-1)
            rows.append(torch.matmul(w, v).squeeze(1))
        outputs.append(torch.cat(rows, dim=0).unsqueeze(0))
    return torch.cat(outputs, dim=0)


def magicpig_sparsetoken_naive_paged_attention(q, paged_kv_cache, kv_page_indptr,
                                               kv_page_indices, sparse_ind, sparse_nnz, K, L):
    """magicpig_..._with_norm.py:212-291: the per-token gather, then the MagicPIG
    correction in fp32 (cosine, acos, p^K, eq. 11's u clamped at 1e-10, ln u),
    fp32 softmax and P.V, the output cast back to fp16."""
    B, Hq, D = q.shape[0], q.shape[1], q.shape[3]
    Hkv, page = paged_kv_cache.shape[2], paged_kv_cache.shape[3]
    G = Hq // Hkv
    k_cache, v_cache = paged_kv_cache[:, 0], paged_kv_cache[:, 1]
    outputs = []
    for b in range(B):
        rows = []
        for h in range(Hq):
            n = sparse_nnz[b, h].item()
            if n == 0:
                rows.append(torch.zeros((1, D), dtype=q.dtype))
                continue
            k, v = _token_rows(k_cache, v_cache, kv_page_indptr, kv_page_indices,
                               sparse_ind[b, h, :n], b, h // G, page)
            kval, lval = K[b, h].item(), L[b, h].item()
            qf = q[b, h:h + 1].float()
            kf = k.float()
            scores = torch.matmul(qf, kf.permute(0, 2, 1))
            qn = torch.norm(qf, dim=-1, keepdim=True)
            kn = torch.norm(kf, dim=-1, keepdim=True)
            c = torch.clamp(scores / (qn * kn.permute(0, 2, 1) + 1e-8), -1.0 + 1e-7, 1.0 - 1e-7)
            p = torch.clamp(1.0 - (1.0 / math.pi) * torch.acos(c), 0.0, 1.0)
            x = torch.pow(p, kval)
            om = torch.clamp(1.0 - x, 0.0, 1.0)
            u = torch.clamp(1.0 - torch.pow(om, lval) - lval * x * torch.pow(om, lval - 1.0),
                            min=1e-10)
            scores = scores / math.sqrt(D) - torch.log(u)
            w = torch.softmax(scores, dim=-1)
            rows.append(torch.matmul(w, v.float()).squeeze(1).to(q.dtype))
        outputs.append(torch.cat(rows, dim=0).unsqueeze(0))
    return torch.cat(outputs, dim=0)
