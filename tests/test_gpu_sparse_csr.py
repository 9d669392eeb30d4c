"""GPU parity of the CSR kept-index format (inds + ptr) for sparse decodes."""
import pytest
import torch

from attention_kernel_triton_amd import _ops
from attention_kernel_triton_amd import sparse_csr as csr
from attention_kernel_triton_amd import synthetic as syn
from helpers import assert_close
from oracle import naive
from oracle.kept import kept_from_uniform

pytestmark = pytest.mark.gpu


def _lists(s):
    B, H, N = s.uniform.shape
    ind, nnz = kept_from_uniform(s.uniform.reshape(B * H, N).numpy(), s.kept_ratio, s.l_max,
                                 s.row_len.reshape(-1).numpy())
    return torch.from_numpy(ind).reshape(B, H, -1), torch.from_numpy(nnz).reshape(B, H, 1)


def _csr_from_lists(ind, nnz):
    rows = []
    ptr = [0]
    for row, n in zip(ind.reshape(-1, ind.shape[-1]), nnz.reshape(-1)):
        rows.append(row[: int(n)])
        ptr.append(ptr[-1] + int(n))
    return torch.cat(rows).to(torch.int32), torch.tensor(ptr, dtype=torch.int64)


def test_to_csr_matches_host_conversion(dev):
    s = syn.sparse_config(seed=3, B=2, Hq=8, Hkv=2, S=2000, D=128, kept_ratio=0.05)
    ind, nnz = _lists(s)
    inds, ptr = csr.to_csr(ind.to(dev), nnz.to(dev))
    rinds, rptr = _csr_from_lists(ind, nnz)
    assert torch.equal(inds.cpu(), rinds) and torch.equal(ptr.cpu(), rptr)


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("splits", [1, 3])
def test_sparse_csr_equals_padded_bitwise(dev, D, splits):
    s = syn.sparse_config(seed=D + splits, B=2, Hq=8, Hkv=2, S=3000, D=D, kept_ratio=0.05)
    ind, nnz = _lists(s)
    inds, ptr = _csr_from_lists(ind, nnz)
    q, K, V = s.q.to(dev), s.K.to(dev), s.V.to(dev)
    o1, l1 = _ops.sparse_decode(q, K, V, ind.to(dev), nnz.to(dev), s.scale, return_lse=True,
                                num_splits=splits)
    o2, l2 = _ops.sparse_decode_csr(q, K, V, inds.to(dev), ptr.to(dev), s.scale, return_lse=True,
                                    num_splits=splits)
    assert torch.equal(o1, o2) and torch.equal(l1, l2)
    ro, rl = naive.sparsetoken_naive_decode(s.q, s.K, s.V, ind, nnz, s.scale, s.group)
    assert_close(o2, ro, what=f"csr D={D}")
    assert_close(l2, rl, atol=1e-4, what="csr lse")


def test_sparse_csr_ragged_rows_and_empty_rows(dev):
    """Rows of very different lengths (no padding) and empty rows."""
    g = torch.Generator().manual_seed(9)
    B, Hq, Hkv, S, D = 2, 4, 2, 5000, 128
    q = torch.randn(B, Hq, 1, D, generator=g).half()
    K = torch.randn(B, Hkv, S, D, generator=g).half()
    V = torch.randn(B, Hkv, S, D, generator=g).half()
    lens = [0, 1, 17, 4096, 300, 0, 2500, 64]
    rows = [torch.sort(torch.randperm(S, generator=g)[:n])[0].to(torch.int32) for n in lens]
    inds = torch.cat(rows)
    ptr = torch.tensor([0] + list(torch.cumsum(torch.tensor(lens), 0)), dtype=torch.int64)
    o, lse = csr.sparsetoken_flash_attention_decode_csr(q.to(dev), K.to(dev), V.to(dev),
                                                        inds.to(dev), ptr.to(dev), 0.1, Hq // Hkv,
                                                        return_lse=True)
    L = max(lens)
    ind = torch.full((B, Hq, L), -1, dtype=torch.int32)
    for u, r in enumerate(rows):
        ind[u // Hq, u % Hq, : len(r)] = r
    nnz = torch.tensor(lens, dtype=torch.int32).reshape(B, Hq, 1)
    ro, rl = naive.sparsetoken_naive_decode(q, K, V, ind, nnz, 0.1, Hq // Hkv)
    o, lse = o.cpu(), lse.cpu()
    for u, n in enumerate(lens):
        b, h = u // Hq, u % Hq
        if n == 0:
            assert torch.equal(o[b, h], torch.zeros_like(o[b, h])) and torch.isinf(lse[b, h])
        else:
            assert_close(o[b, h], ro[b, h], what=f"row {u} (n={n})")


def test_sparse_paged_and_magicpig_csr_equal_padded(dev):
    s = syn.sparse_paged_config(seed=41, B=2, Hq=8, Hkv=2, D=256, page=16, min_len=2000,
                                max_len=6000, kept_ratio=0.03)
    ind, nnz = _lists(s)
    inds, ptr = _csr_from_lists(ind, nnz)
    p = s.paged
    args = (p.q.to(dev), p.pool.to(dev), p.indptr.to(dev), p.indices.to(dev))
    for lk, ll in ((None, None), (s.lsh_k.to(dev), s.lsh_l.to(dev))):
        o1, l1 = _ops.sparse_decode_paged(*args, ind.to(dev), nnz.to(dev), return_lse=True,
                                          num_splits=2, lsh_k=lk, lsh_l=ll)
        o2, l2 = _ops.sparse_decode_paged_csr(*args, inds.to(dev), ptr.to(dev), return_lse=True,
                                              num_splits=2, lsh_k=lk, lsh_l=ll)
        assert torch.equal(o1, o2) and torch.equal(l1, l2), f"magicpig={lk is not None}"
    o3 = csr.magicpig_sparsetoken_flash_attention_decode_paged_csr(
        *args, inds.to(dev), ptr.to(dev), s.lsh_k.to(dev), s.lsh_l.to(dev))
    r64, _ = naive.magicpig_sparsetoken_naive_paged_attention(p.q, p.pool, p.indptr, p.indices,
                                                              ind, nnz, s.lsh_k, s.lsh_l)
    assert_close(o3, r64, what="MagicPIG CSR vs fp64 oracle")


def test_sparse_csr_every_row_empty_forced_splits(dev):
    """A CSR call whose rows are all empty (inds has no entries), at one and at
    three forced splits per row: zeros and -inf."""
    B, Hq, Hkv, S, D = 1, 4, 2, 100, 128
    q = torch.randn(B, Hq, 1, D).half().to(dev)
    K = torch.randn(B, Hkv, S, D).half().to(dev)
    inds = torch.zeros(0, dtype=torch.int32, device=dev)
    ptr = torch.zeros(B * Hq + 1, dtype=torch.int64, device=dev)
    for splits in (1, 3):
        o, lse = _ops.sparse_decode_csr(q, K, K, inds, ptr, 0.1, return_lse=True,
                                        num_splits=splits)
        assert torch.equal(o.cpu(), torch.zeros_like(o.cpu())) and torch.isinf(lse.cpu()).all()


def test_sparse_csr_every_row_empty(dev):
    """A CSR call with no kept index at all (inds has no elements) returns zeros
    and LSE -inf on every row, on both caches."""
    B, Hq, Hkv, S, D = 2, 4, 2, 300, 128
    q = torch.randn(B, Hq, 1, D, device=dev).half()
    K = torch.randn(B, Hkv, S, D, device=dev).half()
    inds = torch.zeros(0, dtype=torch.int32, device=dev)
    ptr = torch.zeros(B * Hq + 1, dtype=torch.int64, device=dev)
    o, lse = csr.sparsetoken_flash_attention_decode_csr(q, K, K, inds, ptr, 0.1, Hq // Hkv,
                                                        return_lse=True)
    assert torch.equal(o, torch.zeros_like(o)) and bool(torch.isinf(lse).all())
    pool = torch.randn(8, 2, Hkv, 16, D, device=dev).half()
    indptr = torch.tensor([0, 4, 8], dtype=torch.int32, device=dev)
    pages = torch.arange(8, dtype=torch.int32, device=dev)
    o2, lse2 = csr.sparsetoken_flash_attention_decode_paged_csr(q, pool, indptr, pages, inds, ptr,
                                                                return_lse=True)
    assert torch.equal(o2, torch.zeros_like(o2)) and bool(torch.isinf(lse2).all())
