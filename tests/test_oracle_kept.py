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


def test_paged_append_round_trip_on_reference_fixture():
    """Rows appended through the reference's page-table fixture
    (decode_flash_attention_redundant_var_len_paged.py:349-353) read back at
    the sequences' last logical positions; nothing else changes."""
    from oracle.kept import paged_append, paged_seq_len, paged_token_address
    page, Hkv, D = 64, 2, 8
    indptr = np.array([0, 4, 5, 8], dtype=np.int32)
    indices = np.array([0, 1, 3, 5, 2, 6, 7, 4], dtype=np.int32)
    last = np.array([2, 22, 3], dtype=np.int32)
    rng = np.random.default_rng(0)
    pool = rng.standard_normal((16, 2, Hkv, page, D)).astype(np.float16)
    counts = [3, 22, 1]                       # 3 tokens spill back across a page boundary
    ap = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    k_new = rng.standard_normal((ap[-1], Hkv, D)).astype(np.float16)
    v_new = rng.standard_normal((ap[-1], Hkv, D)).astype(np.float16)
    out = paged_append(pool, k_new, v_new, ap, indptr, indices, last)
    touched = np.zeros(pool.shape[:1] + pool.shape[3:4], dtype=bool)  # [page, slot]
    for b in range(3):
        L = paged_seq_len(indptr, last, b, page)
        for j in range(counts[b]):
            pid, slot = paged_token_address(indptr, indices, b, L - counts[b] + j, page)
            assert np.array_equal(out[pid, 0, :, slot], k_new[ap[b] + j])
            assert np.array_equal(out[pid, 1, :, slot], v_new[ap[b] + j])
            touched[pid, slot] = True
    assert (L := paged_seq_len(indptr, last, 0, page)) == 3 * 64 + 2
    untouched = ~touched[:, None, None, :, None]
    assert np.array_equal(np.where(untouched, out, 0), np.where(untouched, pool, 0))


def test_paged_append_builds_a_cache_the_paged_oracle_reads_back():
    """Appending a history token by token into random pages, then the paged
    oracle (pinned elsewhere) equals dense decode over that history."""
    import torch
    from oracle import naive
    from oracle.kept import paged_append
    page, Hkv, D, G = 4, 2, 16, 2
    rng = np.random.default_rng(1)
    hist = [7, 1, 13]
    P = 16
    perm = rng.permutation(P)
    pages_of = [list(perm[:2]), list(perm[2:3]), list(perm[3:7])]
    pool = np.zeros((P, 2, Hkv, page, D), dtype=np.float16)
    Ks = [rng.standard_normal((n, Hkv, D)).astype(np.float16) for n in hist]
    Vs = [rng.standard_normal((n, Hkv, D)).astype(np.float16) for n in hist]
    for step in range(max(hist)):
        counts = [1 if step < n else 0 for n in hist]
        lens = [min(step + 1, n) for n in hist]
        indptr, indices, last = [0], [], []
        for b, n in enumerate(lens):
            npg = -(-n // page)
            indices += pages_of[b][:npg]
            indptr.append(len(indices))
            last.append((n - 1) % page + 1)
        ap = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
        rows = [b for b in range(3) if counts[b]]
        k_new = np.stack([Ks[b][step] for b in rows])
        v_new = np.stack([Vs[b][step] for b in rows])
        pool = paged_append(pool, k_new, v_new, ap, np.array(indptr), np.array(indices),
                            np.array(last))
    q = torch.from_numpy(rng.standard_normal((3, Hkv * G, 1, D)).astype(np.float16))
    out, _ = naive.naive_paged_attention(q, torch.from_numpy(pool),
                                         torch.tensor(indptr, dtype=torch.int32),
                                         torch.tensor(indices, dtype=torch.int32),
                                         torch.tensor(last, dtype=torch.int32))
    for b in range(3):
        K = torch.from_numpy(Ks[b]).permute(1, 0, 2).unsqueeze(0)
        V = torch.from_numpy(Vs[b]).permute(1, 0, 2).unsqueeze(0)
        ref, _ = naive.decode(q[b:b + 1], K, V, 1 / D ** 0.5, G)
        assert torch.allclose(out[b], ref[0, :, 0], atol=1e-12, rtol=0)
