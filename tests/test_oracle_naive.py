"""Pins the CPU oracle (oracle/naive.py) against facts independent of its formulas.

Each check is chosen so that a plausible slip in the restatement (a dropped
scale, a wrong GQA head map, a transposed operand, an off-by-one in paging or
the causal mask) fails at least one of them.
"""
import math
import random

import numpy as np
import pytest
import torch

from oracle import naive
from oracle.kept import paged_seq_len

F64 = torch.float64


def _rand(g, *shape):
    return torch.randn(shape, generator=g, dtype=torch.float32).half()


def _scalar_attention(q, keys, vals, scale):
    """Textbook softmax attention with Python floats (brute force)."""
    s = [scale * sum(a * b for a, b in zip(q, k)) for k in keys]
    m = max(s)
    w = [math.exp(x - m) for x in s]
    z = sum(w)
    out = [sum(w[j] * vals[j][d] for j in range(len(vals))) / z for d in range(len(vals[0]))]
    return out, m + math.log(z)


@pytest.mark.parametrize("causal", [True, False])
def test_prefill_matches_scalar_brute_force(causal):
    g = torch.Generator().manual_seed(1)
    B, Hkv, G, S, D = 2, 2, 2, 5, 4
    Q, K, V = _rand(g, B, Hkv * G, S, D), _rand(g, B, Hkv, S, D), _rand(g, B, Hkv, S, D)
    out = naive.prefill(Q, K, V, causal, 0.37, G)
    for b in range(B):
        for h in range(Hkv * G):
            kh = h // G  # reference GQA map: q head h reads kv head h // G
            for i in range(S):
                n = i + 1 if causal else S
                keys = [[float(x) for x in K[b, kh, j]] for j in range(n)]
                vals = [[float(x) for x in V[b, kh, j]] for j in range(n)]
                ref, _ = _scalar_attention([float(x) for x in Q[b, h, i]], keys, vals, 0.37)
                assert torch.allclose(out[b, h, i], torch.tensor(ref, dtype=F64), atol=1e-12)


def test_prefill_causal_first_row_is_first_value_row():
    g = torch.Generator().manual_seed(2)
    Q, K, V = _rand(g, 1, 4, 9, 8), _rand(g, 1, 2, 9, 8), _rand(g, 1, 2, 9, 8)
    out = naive.prefill(Q, K, V, True, 0.5, 2)
    for h in range(4):
        assert torch.equal(out[0, h, 0], V[0, h // 2, 0].to(F64))


def test_prefill_identical_keys_give_running_mean():
    g = torch.Generator().manual_seed(3)
    S, D = 7, 8
    Q, V = _rand(g, 1, 1, S, D), _rand(g, 1, 1, S, D)
    K = _rand(g, 1, 1, 1, D).expand(1, 1, S, D).contiguous()
    out = naive.prefill(Q, K, V, True, 0.125, 1)
    vv = V.to(F64)[0, 0]
    for i in range(S):
        assert torch.allclose(out[0, 0, i], vv[: i + 1].mean(0), atol=1e-12)


def test_prefill_varlen_zeroes_padding_and_keeps_valid_rows():
    g = torch.Generator().manual_seed(4)
    Q, K, V = _rand(g, 2, 2, 12, 8), _rand(g, 2, 1, 12, 8), _rand(g, 2, 1, 12, 8)
    lens = torch.tensor([12, 5])
    out = naive.prefill_varlen(Q, K, V, True, 0.3, 2, lens)
    dense = naive.prefill(Q, K, V, True, 0.3, 2)
    assert torch.equal(out[1, :, 5:], torch.zeros_like(out[1, :, 5:]))
    assert torch.equal(out[1, :, :5], dense[1, :, :5])
    # Valid causal rows cannot see padding: changing it leaves them unchanged.
    K2, V2 = K.clone(), V.clone()
    K2[1, :, 5:] = 100.0
    V2[1, :, 5:] = -100.0
    out2 = naive.prefill_varlen(Q, K2, V2, True, 0.3, 2, lens)
    assert torch.equal(out, out2)


def test_decode_equals_noncausal_prefill_row_and_lse():
    g = torch.Generator().manual_seed(5)
    B, Hkv, G, S, D = 2, 2, 4, 33, 16
    q, K, V = _rand(g, B, Hkv * G, 1, D), _rand(g, B, Hkv, S, D), _rand(g, B, Hkv, S, D)
    o, lse = naive.decode(q, K, V, 0.25, G)
    Q = torch.zeros((B, Hkv * G, S, D), dtype=torch.float16)
    Q[:, :, 3] = q[:, :, 0]
    ref = naive.prefill(Q, K, V, False, 0.25, G)[:, :, 3]
    assert torch.allclose(o[:, :, 0], ref, atol=1e-12)
    s = torch.einsum("bhd,bhsd->bhs", q[:, :, 0].to(F64),
                     K.to(F64).repeat_interleave(G, 1)) * 0.25
    assert torch.allclose(lse, torch.logsumexp(s, -1), atol=1e-12)
    # The normaliser integrates to one: sum exp(s - lse) == 1.
    assert torch.allclose(torch.exp(s - lse[..., None]).sum(-1), torch.ones_like(lse), atol=1e-12)


def _dense_from_pages(pool, indptr, indices, last, b, page):
    n = int(indptr[b + 1] - indptr[b])
    toks = []
    for i in range(n):
        pid = int(indices[int(indptr[b]) + i])
        cnt = page if i < n - 1 else int(last[b])
        for slot in range(cnt):
            toks.append((pid, slot))
    k = torch.stack([pool[p, 0, :, s] for p, s in toks], dim=1)  # [Hkv, n_tok, D]
    v = torch.stack([pool[p, 1, :, s] for p, s in toks], dim=1)
    return k, v


def test_paged_reference_fixture_matches_explicit_gather():
    """Page table of decode_flash_attention_redundant_var_len_paged.py:349-353."""
    g = torch.Generator().manual_seed(6)
    Hkv, G, D, page = 2, 2, 64, 64
    pool = _rand(g, 16, 2, Hkv, page, D)
    indptr = torch.tensor([0, 4, 5, 8], dtype=torch.int32)
    indices = torch.tensor([0, 1, 3, 5, 2, 6, 7, 4], dtype=torch.int32)
    last = torch.tensor([2, 22, 3], dtype=torch.int32)
    q = _rand(g, 3, Hkv * G, 1, D)
    o, lse = naive.naive_paged_attention(q, pool, indptr, indices, last)
    for b in range(3):
        k, v = _dense_from_pages(pool, indptr, indices, last, b, page)
        assert k.shape[1] == paged_seq_len(indptr.numpy(), last.numpy(), b, page)
        ob, lb = naive.decode(q[b:b + 1], k[None], v[None], 1 / math.sqrt(D), G)
        assert torch.allclose(o[b], ob[0, :, 0], atol=1e-12)
        assert torch.allclose(lse[b], lb[0], atol=1e-12)
    assert tuple(o.shape) == (3, Hkv * G, D)


def test_paged_identity_table_equals_dense_decode():
    g = torch.Generator().manual_seed(7)
    B, Hkv, G, D, page, S = 2, 2, 2, 16, 8, 29
    K, V = _rand(g, B, Hkv, S, D), _rand(g, B, Hkv, S, D)
    q = _rand(g, B, Hkv * G, 1, D)
    npg = -(-S // page)
    pool = torch.zeros((B * npg, 2, Hkv, page, D), dtype=torch.float16)
    for b in range(B):
        for i in range(npg):
            n = min(page, S - i * page)
            pool[b * npg + i, 0, :, :n] = K[b, :, i * page:i * page + n]
            pool[b * npg + i, 1, :, :n] = V[b, :, i * page:i * page + n]
    indptr = torch.arange(0, B * npg + 1, npg, dtype=torch.int32)
    indices = torch.arange(B * npg, dtype=torch.int32)
    last = torch.full((B,), S - (npg - 1) * page, dtype=torch.int32)
    o, lse = naive.naive_paged_attention(q, pool, indptr, indices, last)
    od, ld = naive.decode(q, K, V, 1 / math.sqrt(D), G)
    assert torch.allclose(o, od[:, :, 0], atol=1e-12)
    assert torch.allclose(lse, ld, atol=1e-12)


def test_paged_empty_sequence_is_zero():
    g = torch.Generator().manual_seed(8)
    pool = _rand(g, 4, 2, 1, 8, 8)
    q = _rand(g, 2, 2, 1, 8)
    o, lse = naive.naive_paged_attention(q, pool, torch.tensor([0, 2, 2], dtype=torch.int32),
                                         torch.tensor([1, 3], dtype=torch.int32),
                                         torch.tensor([8, 4], dtype=torch.int32))
    assert torch.equal(o[1], torch.zeros_like(o[1])) and torch.isinf(lse[1]).all()


def _sparse_case(seed, B=2, Hkv=2, G=2, S=40, D=16, p=0.3):
    g = torch.Generator().manual_seed(seed)
    q, K, V = _rand(g, B, Hkv * G, 1, D), _rand(g, B, Hkv, S, D), _rand(g, B, Hkv, S, D)
    keep = torch.rand((B, Hkv * G, S), generator=g) < p
    keep[..., 0] = True
    L = S
    ind = torch.full((B, Hkv * G, L), -1, dtype=torch.int32)
    nnz = torch.zeros((B, Hkv * G, 1), dtype=torch.int32)
    for b in range(B):
        for h in range(Hkv * G):
            idx = torch.nonzero(keep[b, h]).squeeze(-1)
            ind[b, h, :idx.numel()] = idx.to(torch.int32)
            nnz[b, h, 0] = idx.numel()
    return q, K, V, keep, ind, nnz, G


def test_sparse_all_kept_equals_dense_decode():
    q, K, V, _, _, _, G = _sparse_case(9)
    B, H, S = q.shape[0], q.shape[1], K.shape[2]
    ind = torch.arange(S, dtype=torch.int32).expand(B, H, S).contiguous()
    nnz = torch.full((B, H, 1), S, dtype=torch.int32)
    o, lse = naive.sparsetoken_naive_decode(q, K, V, ind, nnz, 0.2, G)
    od, ld = naive.decode(q, K, V, 0.2, G)
    assert torch.allclose(o, od, atol=1e-12) and torch.allclose(lse, ld, atol=1e-12)


def test_sparse_loop_matches_mask_and_order_invariance():
    """The reference's own cross-check (sparse:315-328) plus index-order invariance."""
    q, K, V, keep, ind, nnz, G = _sparse_case(10)
    o, lse = naive.sparsetoken_naive_decode(q, K, V, ind, nnz, 0.2, G)
    om, lm = naive.sparsetoken_naive_decode_by_mask(q, K, V, keep, 0.2, G)
    assert torch.allclose(o, om, atol=1e-12) and torch.allclose(lse, lm, atol=1e-12)
    rnd = random.Random(0)
    ind2 = ind.clone()
    for b in range(ind.shape[0]):
        for h in range(ind.shape[1]):
            n = int(nnz[b, h])
            perm = list(range(n))
            rnd.shuffle(perm)
            ind2[b, h, :n] = ind[b, h, perm]
    o2, l2 = naive.sparsetoken_naive_decode(q, K, V, ind2, nnz, 0.2, G)
    assert torch.allclose(o, o2, atol=1e-12) and torch.allclose(lse, l2, atol=1e-12)


def test_sparse_single_token_returns_value_row():
    q, K, V, _, ind, nnz, G = _sparse_case(11)
    nnz1 = torch.ones_like(nnz)
    ind1 = ind.clone()
    ind1[..., 0] = 7
    o, lse = naive.sparsetoken_naive_decode(q, K, V, ind1, nnz1, 0.2, G)
    for b in range(q.shape[0]):
        for h in range(q.shape[1]):
            assert torch.equal(o[b, h, 0], V[b, h // G, 7].to(F64))
            s = 0.2 * (q[b, h, 0].to(F64) @ K[b, h // G, 7].to(F64))
            assert abs(float(lse[b, h] - s)) < 1e-12


def _paged_from_dense(K, V, page, g):
    """Scatter a dense cache into a randomly permuted paged pool."""
    B, Hkv, S, D = K.shape
    npg = -(-S // page)
    total = B * npg
    perm = torch.randperm(total, generator=g)
    pool = torch.zeros((total, 2, Hkv, page, D), dtype=torch.float16)
    indices = torch.empty(total, dtype=torch.int32)
    for b in range(B):
        for i in range(npg):
            pid = int(perm[b * npg + i])
            indices[b * npg + i] = pid
            n = min(page, S - i * page)
            pool[pid, 0, :, :n] = K[b, :, i * page:i * page + n]
            pool[pid, 1, :, :n] = V[b, :, i * page:i * page + n]
    indptr = torch.arange(0, total + 1, npg, dtype=torch.int32)
    return pool, indptr, indices


def test_sparse_paged_equals_sparse_dense_on_same_tokens():
    q, K, V, _, ind, nnz, G = _sparse_case(12, D=16)
    g = torch.Generator().manual_seed(13)
    pool, indptr, indices = _paged_from_dense(K, V, 8, g)
    o, lse = naive.sparsetoken_naive_paged_attention(q, pool, indptr, indices, ind, nnz)
    od, ld = naive.sparsetoken_naive_decode(q, K, V, ind, nnz, 1 / 4.0, G)
    assert torch.allclose(o, od[:, :, 0], atol=1e-12) and torch.allclose(lse, ld, atol=1e-12)


def _magic_case(seed):
    q, K, V, _, ind, nnz, G = _sparse_case(seed, D=16)
    g = torch.Generator().manual_seed(seed + 100)
    pool, indptr, indices = _paged_from_dense(K, V, 8, g)
    return q, pool, indptr, indices, ind, nnz


def test_magicpig_L1_reduces_to_plain_sparse_attention():
    """L = 1 makes u = 0 for every token, clamped to 1e-10: a constant shift."""
    q, pool, indptr, indices, ind, nnz = _magic_case(14)
    B, H = q.shape[0], q.shape[1]
    Kp = torch.full((B, H), 2.5)
    Lp = torch.ones((B, H))
    o, lse = naive.magicpig_sparsetoken_naive_paged_attention(q, pool, indptr, indices, ind, nnz,
                                                               Kp, Lp)
    op, lp = naive.sparsetoken_naive_paged_attention(q, pool, indptr, indices, ind, nnz)
    assert torch.allclose(o, op, atol=1e-12)
    assert torch.allclose(lse, lp - math.log(1e-10), atol=1e-9)


def test_magicpig_K1_L2_closed_form():
    """K = 1, L = 2: u = p^2 exactly, so score = q.k/sqrt(D) - 2 ln p (paper eq. 11)."""
    q, pool, indptr, indices, ind, nnz = _magic_case(15)
    B, H, D = q.shape[0], q.shape[1], q.shape[-1]
    o, lse = naive.magicpig_sparsetoken_naive_paged_attention(
        q, pool, indptr, indices, ind, nnz, torch.ones((B, H)), torch.full((B, H), 2.0))
    page = pool.shape[3]
    for b in range(B):
        for h in range(H):
            n = int(nnz[b, h])
            qv = [float(x) for x in q[b, h, 0]]
            qn = math.sqrt(sum(x * x for x in qv))
            scores, vals = [], []
            for i in range(n):
                t = int(ind[b, h, i])
                pid = int(indices[int(indptr[b]) + t // page])
                kv = [float(x) for x in pool[pid, 0, h // 2, t % page]]
                vals.append([float(x) for x in pool[pid, 1, h // 2, t % page]])
                dot = sum(a * c for a, c in zip(qv, kv))
                kn = math.sqrt(sum(x * x for x in kv))
                cosv = min(max(dot / (qn * kn + 1e-8), -1 + 1e-7), 1 - 1e-7)
                p = 1 - math.acos(cosv) / math.pi
                scores.append(dot / math.sqrt(D) - 2 * math.log(p))
            m = max(scores)
            w = [math.exp(s - m) for s in scores]
            z = sum(w)
            ref = [sum(w[j] * vals[j][d] for j in range(n)) / z for d in range(D)]
            assert torch.allclose(o[b, h], torch.tensor(ref, dtype=F64), atol=1e-10)
            assert abs(float(lse[b, h]) - (m + math.log(z))) < 1e-10


def test_magicpig_fp32_and_fp64_agree_on_well_conditioned_heads():
    q, pool, indptr, indices, ind, nnz = _magic_case(16)
    B, H = q.shape[0], q.shape[1]
    g = torch.Generator().manual_seed(17)
    Kp = torch.rand((B, H), generator=g) * 5 + 1
    Lp = torch.rand((B, H), generator=g) * 3 + 3  # L >= 3: no cancellation trouble
    o64, _ = naive.magicpig_sparsetoken_naive_paged_attention(q, pool, indptr, indices, ind, nnz,
                                                               Kp, Lp)
    o32, _ = naive.magicpig_sparsetoken_naive_paged_attention(q, pool, indptr, indices, ind, nnz,
                                                               Kp, Lp, dtype=torch.float32)
    assert torch.allclose(o64, o32.to(F64), atol=1e-4)


@pytest.mark.parametrize("causal", [True, False])
def test_prefill_lse_matches_scalar_brute_force(causal):
    g = torch.Generator().manual_seed(11)
    B, H, Hkv, S, D = 1, 4, 2, 6, 8
    Q, K, V = _rand(g, B, H, S, D), _rand(g, B, Hkv, S, D), _rand(g, B, Hkv, S, D)
    _, lse = naive.prefill(Q, K, V, causal, 0.41, H // Hkv, return_lse=True)
    for h in range(H):
        kvh = h // (H // Hkv)
        for i in range(S):
            n = i + 1 if causal else S
            q = Q[0, h, i].double().tolist()
            keys = K[0, kvh, :n].double().tolist()
            vals = V[0, kvh, :n].double().tolist()
            _, ref = _scalar_attention(q, keys, vals, 0.41)
            assert abs(float(lse[0, h, i]) - ref) < 1e-12


def test_prefill_lse_causal_row0_is_the_single_score():
    g = torch.Generator().manual_seed(12)
    Q, K, V = _rand(g, 1, 2, 5, 16), _rand(g, 1, 2, 5, 16), _rand(g, 1, 2, 5, 16)
    _, lse = naive.prefill(Q, K, V, True, 0.25, 1, return_lse=True)
    ref = 0.25 * (Q[0, :, 0].double() * K[0, :, 0].double()).sum(-1)
    assert torch.allclose(lse[0, :, 0], ref, atol=1e-12, rtol=0)


def test_merge_of_key_splits_equals_attention_over_all_keys():
    """Attention over disjoint key sets, merged by LSE, equals attention over
    their union -- pins merge_states through the brute-force-pinned prefill."""
    g = torch.Generator().manual_seed(13)
    B, H, Sq, D = 2, 3, 5, 16
    Q = _rand(g, B, H, Sq, D)
    K = _rand(g, B, H, 17, D)
    V = _rand(g, B, H, 17, D)
    full_o, full_l = naive.prefill(Q, K, V, False, 0.3, 1, return_lse=True)
    cuts = [0, 4, 5, 13, 17]
    parts = [naive.prefill(Q, K[:, :, a:b].contiguous(), V[:, :, a:b].contiguous(), False, 0.3, 1,
                           return_lse=True) for a, b in zip(cuts[:-1], cuts[1:])]
    o = torch.stack([p[0] for p in parts])
    lse = torch.stack([p[1] for p in parts])
    mo, ml = naive.merge_states(o, lse)
    assert torch.allclose(mo, full_o, atol=1e-12, rtol=0)
    assert torch.allclose(ml, full_l, atol=1e-12, rtol=0)
    # An empty part (lse = -inf, arbitrary o) changes nothing; all-empty rows give (0, -inf).
    o2 = torch.cat([o, torch.full_like(o[:1], 123.0)])
    l2 = torch.cat([lse, torch.full_like(lse[:1], float("-inf"))])
    mo2, ml2 = naive.merge_states(o2, l2)
    assert torch.allclose(mo2, full_o, atol=1e-12, rtol=0) and torch.allclose(ml2, full_l)
    eo, el = naive.merge_states(torch.ones(2, 3, 4), torch.full((2, 3), float("-inf")))
    assert (eo == 0).all() and torch.isneginf(el).all()


def _eq11_exact(x, L):
    """eq. 11's u = 1 - (1-x)^L - L x (1-x)^(L-1) with 60-digit decimals."""
    from decimal import Decimal, getcontext
    getcontext().prec = 60
    x, L = Decimal(x), Decimal(L)
    om = 1 - x
    return float(1 - (L * om.ln()).exp() - L * x * ((L - 1) * om.ln()).exp())


def _g32(y):
    """log1p(y) - y in float32 as the kernels evaluate it (decode.hip log1p_minus_id)."""
    f = np.float32
    y = f(y)
    if abs(y) < f(0.25):
        s = y / (f(2) + y)
        s2 = s * s
        poly = f(1 / 3) + s2 * (f(1 / 5) + s2 * (f(1 / 7) + s2 * (f(1 / 9) + s2 * f(1 / 11))))
        return f(-y * s + f(2) * s * s2 * poly)
    return f(np.log1p(y) - y)


def _u32(x, L):
    """u as the kernels evaluate it in float32: -expm1((L-1) g(-x) + g((L-1) x))."""
    f = np.float32
    x, L = f(x), f(L)
    m = L - f(1)
    return f(-np.expm1(m * _g32(-x) + _g32(m * x)))


def test_magicpig_u_reformulation_matches_eq11():
    """The kernels evaluate eq. 11's u as -expm1((L-1) g(-x) + g((L-1) x)),
    g(y) = log1p(y) - y, in float32.  Checked against eq. 11 at 60 digits over
    the harness range L in [1, 6) and the MagicPIG paper's large L (up to 200),
    for x from 1e-9 to 0.999: ln u within 1e-5, the bar being the 2e-3 output
    tolerance.  The truncated series the kernels used before (x < 0.05) is
    checked to fail at L = 150, the case that went wrong."""
    rng = random.Random(5)
    worst = 0.0
    for lo, hi in ((1.0, 6.0), (6.0, 200.0)):
        for _ in range(400):
            L = rng.uniform(lo, hi)
            x = 10 ** rng.uniform(-9, math.log10(0.999))
            ref = _eq11_exact(float(np.float32(x)), float(np.float32(L)))
            got = float(_u32(x, L))
            if ref < 1e-10:  # both are clamped to 1e-10 before the log
                assert got < 1.0001e-10 or abs(math.log(got) - math.log(1e-10)) < 1e-5
                continue
            err = abs(math.log(got) - math.log(ref))
            worst = max(worst, err)
            assert err <= 1e-5, (x, L, got, ref)
    assert float(_u32(0.3, 1.0)) == 0.0  # L = 1: u = 0 exactly (then clamped)

    def old_series(x, L):  # the former x < 0.05 branch: diverges once L x is not small
        c, xp = L * (L - 1) / 2, x * x
        u = c * xp
        for k in range(3, 9):
            c *= (L - k + 1) / k
            xp *= -x
            u += (k - 1) * c * xp
        return u

    ref = _eq11_exact(0.0499, 150.0)
    assert abs(math.log(max(old_series(0.0499, 150.0), 1e-10)) - math.log(ref)) > 1.0
    assert abs(math.log(float(_u32(0.0499, 150.0))) - math.log(ref)) <= 1e-5
    print(f"worst |ln u - ln u_exact| = {worst:.2e}")
