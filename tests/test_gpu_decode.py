"""GPU parity of dense decode (R3) and paged var-len decode (R4)."""
import math

import pytest
import torch

from attention_kernel_triton_amd import decode_flash_attention_redundant as dec
from attention_kernel_triton_amd import decode_flash_attention_redundant_var_len_paged as pg
from attention_kernel_triton_amd import _ops
from attention_kernel_triton_amd import synthetic as syn
from helpers import assert_close
from oracle import naive

pytestmark = pytest.mark.gpu


def _dec_inputs(seed, B, Hkv, G, S, D):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hkv * G, 1, D, generator=g).half()
    K = torch.randn(B, Hkv, S, D, generator=g).half()
    V = torch.randn(B, Hkv, S, D, generator=g).half()
    return q, K, V


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("G", [1, 2, 4, 8, 16])
@pytest.mark.parametrize("S", [1, 37, 1000])
def test_decode_shapes(dev, D, G, S):
    B, Hkv = 2, 2
    q, K, V = _dec_inputs(D + G + S, B, Hkv, G, S, D)
    o, lse = dec.flash_attention_decode(q.to(dev), K.to(dev), V.to(dev), 1 / math.sqrt(D), G,
                                        return_lse=True)
    ro, rl = naive.decode(q, K, V, 1 / math.sqrt(D), G)
    assert o.shape == (B, Hkv * G, 1, D)
    assert_close(o, ro, what=f"decode D={D} G={G} S={S}")
    assert_close(lse, rl, atol=1e-4, what="decode lse")


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("chunk", [128, 256, 512, 640])
def test_decode_chunking_does_not_change_results(dev, chunk, D):
    """Every chunk length; at D = 64 the 512- and 640-token chunks run the
    persistent loop with four groups in flight per wave."""
    q, K, V = _dec_inputs(3, 2, 4, 4, 777, D)
    o, lse = _ops.decode(q.to(dev), K.to(dev), V.to(dev), 0.09, return_lse=True,
                         chunk_tokens=chunk)
    ro, rl = naive.decode(q, K, V, 0.09, 4)
    assert_close(o, ro, what=f"chunk {chunk} D={D}")
    assert_close(lse, rl, atol=1e-4, what=f"chunk {chunk} D={D} lse")


def test_decode_config2_full(dev):
    c = syn.decode_config()
    o = dec.flash_attention_decode(c.q.to(dev), c.K.to(dev), c.V.to(dev), c.scale, c.group)
    ro, _ = naive.decode(c.q, c.K, c.V, c.scale, c.group)
    print(f"config 2 max abs err {assert_close(o, ro, what='config 2'):.3e}")


def test_decode_empty_cache_gives_zeros(dev):
    q, K, V = _dec_inputs(4, 1, 2, 2, 0, 64)
    o, lse = dec.flash_attention_decode(q.to(dev), K.to(dev), V.to(dev), 0.1, 2, return_lse=True)
    assert torch.equal(o.cpu(), torch.zeros_like(o.cpu())) and torch.isinf(lse).all()


# --------------------------------------------------------------------------- paged
def _paged_call(p, dev, **kw):
    return pg.flash_attention_decode_paged(p.q.to(dev), p.pool.to(dev), p.indptr.to(dev),
                                           p.indices.to(dev), p.last_len.to(dev), **kw)


def test_paged_reference_fixture(dev):
    """Page table of decode_flash_attention_redundant_var_len_paged.py:349-353."""
    g = torch.Generator().manual_seed(6)
    pool = torch.randn(16, 2, 2, 64, 64, generator=g).half()
    indptr = torch.tensor([0, 4, 5, 8], dtype=torch.int32)
    indices = torch.tensor([0, 1, 3, 5, 2, 6, 7, 4], dtype=torch.int32)
    last = torch.tensor([2, 22, 3], dtype=torch.int32)
    q = torch.randn(3, 4, 1, 64, generator=g).half()
    o, lse = pg.flash_attention_decode_paged(q.to(dev), pool.to(dev), indptr.to(dev),
                                             indices.to(dev), last.to(dev), return_lse=True)
    ro, rl = naive.naive_paged_attention(q, pool, indptr, indices, last)
    assert o.shape == (3, 4, 64)
    assert_close(o, ro, what="paged fixture")
    assert_close(lse, rl, atol=1e-4, what="paged fixture lse")


@pytest.mark.parametrize("page", [1, 8, 16, 48, 64])
@pytest.mark.parametrize("D", [64, 128, 256])
def test_paged_page_sizes(dev, page, D):
    p = syn.paged_config(seed=page * 3 + D, B=5, Hq=8, Hkv=2, D=D, page=page, min_len=1,
                         max_len=700, extra_pages=7)
    o, lse = _paged_call(p, dev, return_lse=True)
    ro, rl = naive.naive_paged_attention(p.q, p.pool, p.indptr, p.indices, p.last_len)
    assert_close(o, ro, what=f"paged page={page} D={D}")
    assert_close(lse, rl, atol=1e-4, what="paged lse")


def test_paged_empty_sequences_and_clamped_last_len(dev):
    g = torch.Generator().manual_seed(9)
    pool = torch.randn(10, 2, 2, 16, 128, generator=g).half()
    q = torch.randn(4, 8, 1, 128, generator=g).half()
    indptr = torch.tensor([0, 0, 3, 3, 5], dtype=torch.int32)  # sequences 0 and 2 are empty
    indices = torch.tensor([9, 2, 4, 0, 7], dtype=torch.int32)
    last = torch.tensor([5, 40, 3, 0], dtype=torch.int32)       # 40 clamps to 16, 0 drops a page
    o, lse = pg.flash_attention_decode_paged(q.to(dev), pool.to(dev), indptr.to(dev),
                                             indices.to(dev), last.to(dev), return_lse=True)
    ro, rl = naive.naive_paged_attention(q, pool, indptr, indices, last)
    o, lse = o.cpu(), lse.cpu()
    assert torch.equal(o[0], torch.zeros_like(o[0])) and torch.equal(o[2], torch.zeros_like(o[2]))
    assert torch.isinf(lse[0]).all() and torch.isinf(lse[2]).all()
    assert_close(o, ro, what="paged edge cases")


def test_paged_single_token_sequences_are_exact(dev):
    """A one-token sequence returns its V row bit for bit (p = 1, l = 1)."""
    g = torch.Generator().manual_seed(10)
    pool = torch.randn(40, 2, 4, 16, 128, generator=g).half()
    B = 12
    indptr = torch.arange(B + 1, dtype=torch.int32)
    indices = torch.randperm(40, generator=g)[:B].to(torch.int32)
    last = torch.ones(B, dtype=torch.int32)
    q = torch.randn(B, 16, 1, 128, generator=g).half()
    o = pg.flash_attention_decode_paged(q.to(dev), pool.to(dev), indptr.to(dev), indices.to(dev),
                                        last.to(dev)).cpu()
    for b in range(B):
        for h in range(16):
            assert torch.equal(o[b, h], pool[int(indices[b]), 1, h // 4, 0])


def test_paged_config3_full(dev):
    p = syn.paged_config()
    o, lse = _paged_call(p, dev, return_lse=True)
    ro, rl = naive.naive_paged_attention(p.q, p.pool, p.indptr, p.indices, p.last_len)
    err = assert_close(o, ro, what="config 3")
    assert_close(lse, rl, atol=1e-4, what="config 3 lse")
    print(f"config 3 max abs err {err:.3e}")


@pytest.mark.parametrize("chunk", [256, 512, 640])
def test_paged_chunk_lengths(dev, chunk):
    p = syn.paged_config(B=8, min_len=1, max_len=5000)
    d = p.to(dev)
    o, lse = _ops.decode_paged(d.q, d.pool, d.indptr, d.indices, d.last_len, return_lse=True,
                               chunk_tokens=chunk)
    ro, rl = naive.naive_paged_attention(p.q, p.pool, p.indptr, p.indices, p.last_len)
    assert_close(o, ro, what=f"paged chunk {chunk}")
    assert_close(lse, rl, atol=1e-4, what=f"paged chunk {chunk} lse")


@pytest.mark.parametrize("Hq,D", [(32, 128), (32, 64), (64, 128)])
@pytest.mark.parametrize("chunk", [0, 640])
def test_paged_lengths_at_every_boundary(dev, Hq, D, chunk):
    """Lengths on both sides of each 16-token group and 640-token chunk
    boundary, empty and one-token sequences, padded with 8192-token ones to a
    config-3-sized launch: the automatic path (chunk 0, the stream-K kernel,
    whose wave ranges then cut units at many positions) and the persistent
    chunked kernel at 640 tokens; a second call is bit-identical."""
    from attention_kernel_triton_amd import _ops
    g = torch.Generator().manual_seed(70 + D + Hq)
    Hkv = 8
    lens = [0, 1, 15, 16, 17, 255, 256, 257, 639, 640, 641, 913, 914, 915, 916, 1279, 1280,
            1281, 1828, 1829, 1919, 1920, 1921, 4096] + [8192] * 13
    B = len(lens)
    indptr, indices, last, P = syn.block_table(g, lens, 16)
    pool = torch.randn(P, 2, Hkv, 16, D, generator=g).half()
    q = torch.randn(B, Hq, 1, D, generator=g).half()
    args = (q.to(dev), pool.to(dev), indptr.to(dev), indices.to(dev), last.to(dev))
    o, lse = _ops.decode_paged(*args, chunk_tokens=chunk, return_lse=True)
    ro, rl = naive.naive_paged_attention(q, pool, indptr, indices, last)
    nonempty = torch.tensor(lens) > 0
    assert_close(o, ro, what=f"chunk {chunk} Hq={Hq} D={D}")
    assert_close(lse, rl, atol=1e-4, what=f"chunk {chunk} lse", mask=nonempty)
    assert torch.isinf(lse.cpu()[~nonempty]).all()
    again = _ops.decode_paged(*args, chunk_tokens=chunk)
    assert torch.equal(again, o)


def test_paged_config3_page_relabelling_is_bit_exact(dev):
    """Renaming physical pages (and moving their contents) must not change a single bit."""
    p = syn.paged_config(B=8, min_len=256, max_len=4096)
    P = p.pool.shape[0]
    perm = torch.randperm(P, generator=torch.Generator().manual_seed(1))
    pool2 = torch.empty_like(p.pool)
    pool2[perm] = p.pool                      # page i moves to slot perm[i]
    indices2 = perm[p.indices.long()].to(torch.int32)
    a = _paged_call(p, dev)
    b = pg.flash_attention_decode_paged(p.q.to(dev), pool2.to(dev), p.indptr.to(dev),
                                        indices2.to(dev), p.last_len.to(dev))
    assert torch.equal(a, b)


def test_paged_invalid_page_ids_are_skipped(dev):
    g = torch.Generator().manual_seed(12)
    pool = torch.randn(6, 2, 1, 16, 64, generator=g).half()
    q = torch.randn(1, 2, 1, 64, generator=g).half()
    indptr = torch.tensor([0, 3], dtype=torch.int32)
    good = torch.tensor([4, 1], dtype=torch.int32)
    o = pg.flash_attention_decode_paged(q.to(dev), pool.to(dev), indptr.to(dev),
                                        torch.tensor([4, 99, 1], dtype=torch.int32).to(dev),
                                        torch.tensor([16], dtype=torch.int32).to(dev))
    ro, _ = naive.naive_paged_attention(q, pool, torch.tensor([0, 2], dtype=torch.int32), good,
                                        torch.tensor([16], dtype=torch.int32))
    assert_close(o, ro, what="invalid page skipped")


def test_paged_repeated_calls_are_bit_identical(dev):
    """Dynamic work scheduling changes which workgroup runs a chunk, never the result;
    the scheduling counters are left at zero by every call."""
    p = syn.paged_config(B=16, min_len=256, max_len=6000).to(dev)
    outs = [pg.flash_attention_decode_paged(p.q, p.pool, p.indptr, p.indices, p.last_len)
            for _ in range(4)]
    for o in outs[1:]:
        assert torch.equal(o, outs[0])
    from attention_kernel_triton_amd import _native
    bufs = _native.workspace_buffers()
    assert bufs
    for _, _, buf in bufs:
        assert int(buf[:256].count_nonzero()) == 0


def test_paged_on_a_side_stream_matches_the_default_stream(dev):
    """Each stream gets its own workspace (its scheduling counters must not be shared
    by calls that can overlap), and the kernels launch on the caller's current stream."""
    from attention_kernel_triton_amd import _native
    p = syn.paged_config(B=8, min_len=256, max_len=3000).to(dev)
    ref = pg.flash_attention_decode_paged(p.q, p.pool, p.indptr, p.indices, p.last_len)
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        o = pg.flash_attention_decode_paged(p.q, p.pool, p.indptr, p.indices, p.last_len)
        key = (torch.device(dev).index or 0, side.cuda_stream)
    torch.cuda.synchronize(dev)
    assert torch.equal(o, ref)
    assert key in [(d, s) for d, s, _ in _native.workspace_buffers()]
    # ctypes reads the null (default) stream back as None
    assert (_native.stream_of(p.q).value or 0) == torch.cuda.current_stream(dev).cuda_stream


def test_paged_on_two_streams_at_once(dev):
    """Two launches in flight together on two streams: each stream has its own
    workspace, so their scheduling counters never mix."""
    p = syn.paged_config(B=16, min_len=256, max_len=6000).to(dev)
    q2 = p.q.flip(1).contiguous()
    ref1 = pg.flash_attention_decode_paged(p.q, p.pool, p.indptr, p.indices, p.last_len)
    ref2 = pg.flash_attention_decode_paged(q2, p.pool, p.indptr, p.indices, p.last_len)
    s1, s2 = torch.cuda.Stream(device=dev), torch.cuda.Stream(device=dev)
    s1.wait_stream(torch.cuda.current_stream(dev))
    s2.wait_stream(torch.cuda.current_stream(dev))
    outs1, outs2 = [], []
    for _ in range(4):
        with torch.cuda.stream(s1):
            outs1.append(pg.flash_attention_decode_paged(p.q, p.pool, p.indptr, p.indices,
                                                         p.last_len))
        with torch.cuda.stream(s2):
            outs2.append(pg.flash_attention_decode_paged(q2, p.pool, p.indptr, p.indices,
                                                         p.last_len))
    torch.cuda.synchronize(dev)
    for o in outs1:
        assert torch.equal(o, ref1)
    for o in outs2:
        assert torch.equal(o, ref2)


def test_paged_page_ids_past_32_bit_byte_offsets(dev):
    """Pages near the end of a 4.6 GB pool: page id x page stride overflows 32 bits, so
    the row address must be formed in 64 bits.  Only the used pages are filled; the
    oracle runs on a compact copy of them."""
    Hq, Hkv, page, D = 8, 8, 16, 128
    P = 70000  # 70000 pages x 2 x 8 x 16 x 128 x 2 B = 4.6 GB
    lens = [100, 37]
    npg = [(L + page - 1) // page for L in lens]
    used = torch.arange(P - 1, P - 1 - sum(npg), -1, dtype=torch.int32)  # highest ids first
    g = torch.Generator().manual_seed(21)
    content = torch.randn(len(used), 2, Hkv, page, D, generator=g).half()
    q = torch.randn(len(lens), Hq, 1, D, generator=g).half()
    pool = torch.empty(P, 2, Hkv, page, D, dtype=torch.float16, device=dev)
    pool[used.long().to(dev)] = content.to(dev)
    indptr = torch.tensor([0, npg[0], npg[0] + npg[1]], dtype=torch.int32)
    last = torch.tensor([L - (n - 1) * page for L, n in zip(lens, npg)], dtype=torch.int32)
    o, lse = pg.flash_attention_decode_paged(q.to(dev), pool, indptr.to(dev), used.to(dev),
                                             last.to(dev), return_lse=True)
    compact = torch.arange(len(used), dtype=torch.int32)
    ro, rl = naive.naive_paged_attention(q, content, indptr, compact, last)
    assert_close(o, ro, what="paged, page ids near 70000")
    assert_close(lse, rl, atol=1e-4, what="paged lse, page ids near 70000")
    del pool


def test_decode_long_sequence(dev):
    """One 131072-token cache (four 640-token-or-less chunk rounds per unit and more)."""
    q, K, V = _dec_inputs(22, 1, 2, 4, 131072, 128)
    o, lse = dec.flash_attention_decode(q.to(dev), K.to(dev), V.to(dev), 1 / math.sqrt(128), 4,
                                        return_lse=True)
    ro, rl = naive.decode(q, K, V, 1 / math.sqrt(128), 4)
    assert_close(o, ro, what="decode S=131072")
    assert_close(lse, rl, atol=1e-4, what="decode S=131072 lse")


@pytest.mark.parametrize("page", [16, 8])
def test_paged_batch_past_the_lds_chunk_table(dev, page):
    """Batches over 1024 sequences take the non-persistent kernel: each workgroup
    locates its chunk by scanning the page table, chunks are 256 tokens, and the
    first workgroups write the rows of empty sequences.  Both the page-aligned
    (16) and the unaligned (8) group addressing are covered, with the LSE."""
    g = torch.Generator().manual_seed(40 + page)
    B, Hq, Hkv, D = 1100, 4, 2, 128
    lens = torch.randint(1, 700, (B,), generator=g).tolist()
    for b in (0, 3, 517, B - 1):
        lens[b] = 0
    indptr, indices, last, P = syn.block_table(g, lens, page, extra_pages=5)
    pool = torch.randn(P, 2, Hkv, page, D, generator=g).half()
    q = torch.randn(B, Hq, 1, D, generator=g).half()
    o, lse = pg.flash_attention_decode_paged(q.to(dev), pool.to(dev), indptr.to(dev),
                                             indices.to(dev), last.to(dev), return_lse=True)
    ro, rl = naive.naive_paged_attention(q, pool, indptr, indices, last)
    nonempty = torch.tensor(lens) > 0
    assert_close(o, ro, what=f"paged B={B} page={page}")
    assert_close(lse, rl, atol=1e-4, what="paged lse", mask=nonempty)
    assert torch.isinf(lse.cpu()[~nonempty]).all()


@pytest.mark.parametrize("B", [1, 63, 64, 200, 1024])
def test_paged_batches_up_to_the_lds_sequence_table(dev, B):
    """The automatic path builds every workgroup's sequence table in LDS, up to
    1024 sequences: batches from one sequence to that limit, with empty
    sequences and clamped last-page lengths, match the oracle (O and LSE)."""
    g = torch.Generator().manual_seed(70 + B)
    Hq, Hkv, D, page = 8, 2, 128, 16
    lens = torch.randint(1, 300, (B,), generator=g).tolist()
    for b in {0, B // 2, B - 1} if B > 2 else set():
        lens[b] = 0
    indptr, indices, last, P = syn.block_table(g, lens, page, extra_pages=3)
    if B > 1:
        last[1] = 40  # clamps to the page size
    pool = torch.randn(P, 2, Hkv, page, D, generator=g).half()
    q = torch.randn(B, Hq, 1, D, generator=g).half()
    o, lse = pg.flash_attention_decode_paged(q.to(dev), pool.to(dev), indptr.to(dev),
                                             indices.to(dev), last.to(dev), return_lse=True)
    ro, rl = naive.naive_paged_attention(q, pool, indptr, indices, last)
    nonempty = (indptr[1:] - indptr[:-1]) > 0
    assert_close(o, ro, what=f"paged B={B}")
    assert_close(lse, rl, atol=1e-4, what=f"paged lse B={B}", mask=nonempty)
    assert torch.isinf(lse.cpu()[~nonempty]).all()


@pytest.mark.parametrize("G,D", [(1, 128), (2, 64), (3, 128), (8, 256), (16, 128), (32, 64)])
def test_paged_automatic_path_every_head_group_width(dev, G, D):
    """Every heads-per-unit instance of the automatic path (GT = 1, 2, 4, 8,
    16; G = 3 leaves a unit's last column empty, G = 32 at D = 64 takes two
    head groups of 16 per kv head) against the oracle, O and LSE."""
    g = torch.Generator().manual_seed(90 + G + D)
    Hkv, page = 2, 32
    lens = torch.randint(1, 900, (6,), generator=g).tolist()
    indptr, indices, last, P = syn.block_table(g, lens, page, extra_pages=2)
    pool = torch.randn(P, 2, Hkv, page, D, generator=g).half()
    q = torch.randn(len(lens), Hkv * G, 1, D, generator=g).half()
    o, lse = pg.flash_attention_decode_paged(q.to(dev), pool.to(dev), indptr.to(dev),
                                             indices.to(dev), last.to(dev), return_lse=True)
    ro, rl = naive.naive_paged_attention(q, pool, indptr, indices, last)
    assert_close(o, ro, what=f"paged G={G} D={D}")
    assert_close(lse, rl, atol=1e-4, what=f"paged lse G={G} D={D}")


def test_paged_merges_are_coherent_across_launches(dev):
    """The last workgroup of a unit merges partials other workgroups (on any XCD)
    stored in the same launch.  Alternating two inputs over one workspace, every
    launch must reproduce its input's first result bit for bit: a partial read
    before it was visible, or a stale one from the previous launch, would not."""
    a = syn.paged_config(B=32, min_len=256, max_len=8192).to(dev)
    b = syn.paged_config(seed=7, B=32, min_len=256, max_len=8192).to(dev)
    ra = pg.flash_attention_decode_paged(a.q, a.pool, a.indptr, a.indices, a.last_len)
    rb = pg.flash_attention_decode_paged(b.q, b.pool, b.indptr, b.indices, b.last_len)
    outs = []
    for _ in range(10):
        outs.append((pg.flash_attention_decode_paged(a.q, a.pool, a.indptr, a.indices,
                                                     a.last_len),
                     pg.flash_attention_decode_paged(b.q, b.pool, b.indptr, b.indices,
                                                     b.last_len)))
    for oa, ob in outs:
        assert torch.equal(oa, ra) and torch.equal(ob, rb)
    ref, _ = naive.naive_paged_attention(a.q.cpu(), a.pool.cpu(), a.indptr.cpu(),
                                         a.indices.cpu(), a.last_len.cpu())
    assert_close(ra, ref, what="config-3-sized merge")


def test_decode_more_units_than_the_fixed_arrival_area(dev):
    """35200 units (B = 1100, 32 kv heads, G = 1, two chunks each).  Arrival
    counters past the fixed 32768-slot area sit where the earlier, smaller calls
    stored their partials, so the call must clear them first.  Splitting the
    batch does not change what any unit computes, so the results are bit-identical."""
    g = torch.Generator().manual_seed(50)
    B, Hkv, S, D = 1100, 32, 150, 64
    q = torch.randn(B, Hkv, 1, D, generator=g).half().to(dev)
    K = torch.randn(B, Hkv, S, D, generator=g).half().to(dev)
    V = torch.randn(B, Hkv, S, D, generator=g).half().to(dev)
    parts = [_ops.decode(q[i:i + 100], K[i:i + 100], V[i:i + 100], 0.125, chunk_tokens=128)
             for i in range(0, B, 100)]
    full = _ops.decode(q, K, V, 0.125, chunk_tokens=128)
    assert torch.equal(full, torch.cat(parts))
    ro, _ = naive.decode(q[:100].cpu(), K[:100].cpu(), V[:100].cpu(), 0.125, 1)
    assert_close(parts[0], ro, what="first slice")
