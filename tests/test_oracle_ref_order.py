"""Pins oracle/ref_order.py (the reference's naive paths in its own fp16 op order,
timed as bench.py's CPU baseline) against the fp64 oracle (oracle/naive.py) on
small seeded inputs: the two must agree within the fp16 rounding of the
reference's arithmetic (its own self-checks use atol 1e-2).  A restatement that
dropped a scale, swapped the GQA map or read the wrong page would be off by O(1)."""
import math

import torch

from attention_kernel_triton_amd import synthetic as syn
from oracle import naive, ref_order
from oracle.kept import kept_from_uniform

TOL = 1e-2


def _err(a, b):
    if isinstance(b, tuple):  # the oracle's (O, LSE)
        b = b[0]
    return float((a.double() - b.double()).abs().max())


def test_dense_paths_match_oracle():
    c = syn.prefill_config(0, B=2, Hq=8, Hkv=2, S=96, D=64)
    for causal in (True, False):
        got = ref_order.prefill(c.Q, c.K, c.V, causal, c.scale, c.group)
        assert _err(got, naive.prefill(c.Q, c.K, c.V, causal, c.scale, c.group)) < TOL
    v = syn.prefill_config(1, B=3, Hq=4, Hkv=1, S=128, D=64)
    got = ref_order.prefill_varlen(v.Q, v.K, v.V, True, v.scale, v.group, v.varlen)
    ref = naive.prefill_varlen(v.Q, v.K, v.V, True, v.scale, v.group, v.varlen)
    for b, L in enumerate(v.varlen.tolist()):
        assert _err(got[b, :, :L], ref[b, :, :L]) < TOL
        assert not got[b, :, L:].any()
    d = syn.decode_config(B=2, Hq=8, Hkv=2, S=300, D=64)
    assert _err(ref_order.decode(d.q, d.K, d.V, d.scale, d.group),
                naive.decode(d.q, d.K, d.V, d.scale, d.group)) < TOL


def test_paged_path_matches_oracle():
    p = syn.paged_config(B=3, Hq=8, Hkv=2, D=128, page=16, min_len=20, max_len=400)
    got = ref_order.naive_paged_attention(p.q, p.pool, p.indptr, p.indices, p.last_len)
    ref, _ = naive.naive_paged_attention(p.q, p.pool, p.indptr, p.indices, p.last_len)
    assert got.shape == ref.shape and _err(got, ref) < TOL


def _lists(s):
    B, H, N = s.uniform.shape
    ind, nnz = kept_from_uniform(s.uniform.reshape(B * H, N).numpy(), s.kept_ratio, s.l_max,
                                 s.row_len.reshape(-1).numpy())
    return torch.from_numpy(ind).reshape(B, H, -1), torch.from_numpy(nnz).reshape(B, H, 1)


def test_sparse_paths_match_oracle():
    s = syn.sparse_config(B=1, Hq=8, Hkv=2, S=2000, D=128, kept_ratio=0.05)
    ind, nnz = _lists(s)
    got = ref_order.sparsetoken_naive_decode(s.q, s.K, s.V, ind, nnz, s.scale, s.group)
    ref, _ = naive.sparsetoken_naive_decode(s.q, s.K, s.V, ind, nnz, s.scale, s.group)
    assert _err(got, ref) < TOL
    t = syn.sparse_paged_config(B=2, Hq=8, Hkv=2, D=64, page=16, min_len=500, max_len=900,
                                kept_ratio=0.05)
    ind, nnz = _lists(t)
    p = t.paged
    got = ref_order.sparsetoken_naive_paged_attention(p.q, p.pool, p.indptr, p.indices, ind, nnz)
    ref, _ = naive.sparsetoken_naive_paged_attention(p.q, p.pool, p.indptr, p.indices, ind, nnz)
    assert _err(got, ref) < TOL
    got = ref_order.magicpig_sparsetoken_naive_paged_attention(p.q, p.pool, p.indptr, p.indices,
                                                               ind, nnz, t.lsh_k, t.lsh_l)
    ref, _ = naive.magicpig_sparsetoken_naive_paged_attention(p.q, p.pool, p.indptr, p.indices,
                                                              ind, nnz, t.lsh_k, t.lsh_l)
    # The fp32 evaluation of eq. 11 cancels on some heads (the reason the parity
    # oracle is fp64): compare on the heads where fp32 and fp64 agree.
    r32, _ = naive.magicpig_sparsetoken_naive_paged_attention(
        p.q, p.pool, p.indptr, p.indices, ind, nnz, t.lsh_k, t.lsh_l, dtype=torch.float32)
    well = (r32 - ref).abs().amax(-1) < 1e-3
    assert int(well.sum()) >= 8
    assert _err(got[well], ref[well]) < TOL
