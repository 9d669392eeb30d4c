"""The seeded generators are deterministic and build valid page tables."""
import torch

from attention_kernel_triton_amd import synthetic as syn


def test_prefill_config_deterministic_and_padded():
    a = syn.prefill_config(1, B=3, Hq=4, Hkv=2, S=96, D=64)
    b = syn.prefill_config(1, B=3, Hq=4, Hkv=2, S=96, D=64)
    assert torch.equal(a.Q, b.Q) and torch.equal(a.V, b.V) and torch.equal(a.varlen, b.varlen)
    assert int(a.varlen[0]) == 96 and all(64 <= int(x) <= 96 for x in a.varlen)
    assert a.flops() == 4 * 64 * 4 * sum(int(L) * (int(L) + 1) // 2 for L in a.varlen)


def test_paged_config_block_table_is_valid():
    p = syn.paged_config(B=5, Hq=4, Hkv=2, D=64, page=16, min_len=1, max_len=100)
    P = p.pool.shape[0]
    assert sorted(p.indices.tolist()) == list(range(P))
    pages = (p.indptr[1:] - p.indptr[:-1]).tolist()
    for L, n, last in zip(p.lens, pages, p.last_len.tolist()):
        assert n == -(-L // 16) and 1 <= last <= 16 and (n - 1) * 16 + last == L
    assert p.bytes() == sum(p.lens) * 2 * 64 * 4 + 2 * p.q.numel() * 2 + 4 * (P + 6 + 5)


def test_sparse_configs_shapes():
    s = syn.sparse_config(B=1, Hq=4, Hkv=2, S=500, D=64)
    assert s.uniform.shape == (1, 4, 500) and s.l_max == int(500 * 0.12)
    sp = syn.sparse_paged_config(B=2, Hq=4, Hkv=2, D=64, page=16, min_len=100, max_len=200)
    assert sp.lsh_k.shape == (2, 4) and float(sp.lsh_k.min()) >= 1 and float(sp.lsh_l.max()) < 6
    assert sp.row_len[:, 0].tolist() == sp.paged.lens
