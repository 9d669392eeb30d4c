"""Pins the integer oracle (oracle/kept.py): kept-index selection and page addressing."""
import numpy as np
import torch

from oracle.kept import kept_from_uniform, kept_indices, paged_seq_len, paged_token_address


def test_kept_indices_match_torch_nonzero_and_loops():
    rng = np.random.default_rng(0)
    keep = rng.random((6, 300)) < 0.05
    keep[2] = False  # empty row -> index 0 kept
    row_len = np.array([300, 250, 300, 10, 0, 299])
    ind, nnz = kept_indices(keep, 40, row_len)
    for r in range(6):
        nr = row_len[r]
        ref = [j for j in range(nr) if keep[r, j]]  # brute force
        tref = torch.nonzero(torch.from_numpy(keep[r, :nr])).squeeze(-1).tolist()
        assert ref == tref
        if not ref:
            ref = [0]
        assert nnz[r] == len(ref)
        assert ind[r, :len(ref)].tolist() == ref[:40]
        assert (ind[r, len(ref):] == -1).all()


def test_kept_indices_without_ensure_nonempty_and_overflow():
    keep = np.zeros((2, 8), dtype=bool)
    keep[1, :] = True
    ind, nnz = kept_indices(keep, 5, ensure_nonempty=False)
    assert nnz.tolist() == [0, 8]
    assert ind[0].tolist() == [-1] * 5 and ind[1].tolist() == [0, 1, 2, 3, 4]


def test_kept_from_uniform_uses_float32_threshold():
    u = np.array([[0.02, np.nextafter(np.float32(0.02), np.float32(0)), 0.5, 0.0]], dtype=np.float32)
    ind, nnz = kept_from_uniform(u, 0.02, 4)
    # torch compares a float32 tensor against the float32-rounded ratio
    t = (torch.from_numpy(u) < 0.02).numpy()
    assert (ind[0, :nnz[0]] == np.flatnonzero(t[0])).all()
    assert ind[0].tolist() == [1, 3, -1, -1]


def test_reference_page_table_fixtures():
    """decode_..._var_len_paged.py:349-353 and sparsetoken_..._var_len_paged.py:321-330."""
    indptr = np.array([0, 4, 5, 8])
    indices = np.array([0, 1, 3, 5, 2, 6, 7, 4])
    last = np.array([2, 22, 3])
    assert [paged_seq_len(indptr, last, b, 64) for b in range(3)] == [3 * 64 + 2, 22, 2 * 64 + 3]
    pid, slot = paged_token_address(indptr, indices, 0, [0, 63, 64, 193], 64)
    assert pid.tolist() == [0, 0, 1, 5] and slot.tolist() == [0, 63, 0, 1]
    pid, slot = paged_token_address(indptr, indices, 2, [130], 64)
    assert pid.tolist() == [4] and slot.tolist() == [2]
    # spaged fixture: 270/350/321 pages of 256 over a permuted pool, last 63/22/55
    pages = np.array([270, 350, 321])
    indptr2 = np.concatenate([[0], np.cumsum(pages)])
    last2 = np.array([63, 22, 55])
    lens = [paged_seq_len(indptr2, last2, b, 256) for b in range(3)]
    assert lens == [269 * 256 + 63, 349 * 256 + 22, 320 * 256 + 55]
    perm = np.random.default_rng(1).permutation(pages.sum())
    pid, slot = paged_token_address(indptr2, perm, 1, [0, 256 * 349 + 21], 256)
    assert pid.tolist() == [perm[270], perm[270 + 349]] and slot.tolist() == [0, 21]
