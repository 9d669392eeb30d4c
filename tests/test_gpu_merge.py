"""GPU parity of the prefill LSE output and the LSE merge of partial states."""
import math

import pytest
import torch

from attention_kernel_triton_amd import decode_flash_attention_redundant as dec
from attention_kernel_triton_amd import prefill_flash_attention as pre
from attention_kernel_triton_amd import prefill_flash_attention_var_len_padding as prv
from attention_kernel_triton_amd.merge_states import merge_states
from helpers import assert_close
from oracle import naive

pytestmark = pytest.mark.gpu

# LSE tolerance: the kernel's normaliser sums the fp16-rounded probabilities
# that multiply V (relative error <= 2^-11 per term), ln of that sum.
LSE_ATOL = 2e-3


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("S", [1, 45, 200])
def test_prefill_lse(dev, D, causal, S):
    g = torch.Generator().manual_seed(D + S + causal)
    B, Hq, Hkv = 2, 8, 2
    Q = torch.randn(B, Hq, S, D, generator=g).half()
    K = torch.randn(B, Hkv, S, D, generator=g).half()
    V = torch.randn(B, Hkv, S, D, generator=g).half()
    o, lse = pre.flash_attention_prefill(Q.to(dev), K.to(dev), V.to(dev), causal, 1 / math.sqrt(D),
                                         Hq // Hkv, return_lse=True)
    ro, rl = naive.prefill(Q, K, V, causal, 1 / math.sqrt(D), Hq // Hkv, return_lse=True)
    assert_close(o, ro, what="O")
    assert_close(lse, rl, atol=LSE_ATOL, what="LSE")
    o_plain = pre.flash_attention_prefill(Q.to(dev), K.to(dev), V.to(dev), causal, 1 / math.sqrt(D),
                                          Hq // Hkv)
    assert torch.equal(o_plain, o)  # the LSE output does not change O


def test_prefill_varlen_lse_on_valid_rows(dev):
    g = torch.Generator().manual_seed(5)
    B, Hq, Hkv, S, D = 3, 4, 2, 150, 64
    Q = torch.randn(B, Hq, S, D, generator=g).half()
    K = torch.randn(B, Hkv, S, D, generator=g).half()
    V = torch.randn(B, Hkv, S, D, generator=g).half()
    lens = torch.tensor([150, 70, 3], dtype=torch.int64)
    o, lse = prv.flash_attention_prefill(Q.to(dev), K.to(dev), V.to(dev), True, 0.125, 2,
                                         varlen=lens.to(dev), return_lse=True)
    _, rl = naive.prefill(Q, K, V, True, 0.125, 2, return_lse=True)
    for b, L in enumerate(lens.tolist()):
        assert_close(lse[b, :, :L], rl[b, :, :L], atol=LSE_ATOL, what=f"LSE b={b}")


@pytest.mark.parametrize("in_dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("out_dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("n,D", [(1, 64), (3, 128), (7, 256), (16, 8)])
def test_merge_states_matches_oracle(dev, in_dtype, out_dtype, n, D):
    g = torch.Generator().manual_seed(n * 1000 + D)
    o = torch.randn(n, 5, 9, D, generator=g).to(in_dtype)
    lse = torch.randn(n, 5, 9, generator=g) * 4
    if n > 2:
        lse[1, 0, :] = float("-inf")  # an empty part for some rows
    mo, ml = merge_states(o.to(dev), lse.to(dev), out_dtype=out_dtype)
    ro, rl = naive.merge_states(o, lse)
    tol = 2e-3 if out_dtype == torch.float16 else 1e-5
    assert mo.dtype == out_dtype and mo.shape == (5, 9, D) and ml.shape == (5, 9)
    assert_close(mo, ro, atol=tol, what="O")
    assert_close(ml, rl, atol=1e-5, what="LSE")


def test_merge_states_all_empty_rows(dev):
    o = torch.randn(3, 4, 64).half().to(dev)
    lse = torch.full((3, 4), float("-inf")).to(dev)
    lse[0, 2] = 0.5
    mo, ml = merge_states(o, lse)
    assert (mo[[0, 1, 3]] == 0).all() and torch.isneginf(ml[[0, 1, 3]]).all()
    assert torch.equal(mo[2], o[0, 2]) and abs(float(ml[2]) - 0.5) < 1e-6


@pytest.mark.parametrize("cuts", [[0, 300, 1000], [0, 1, 517, 518, 1000]])
def test_decode_over_cache_chunks_merges_to_full_decode(dev, cuts):
    """Chunked decode (LSE out) + merge_states == decode over the whole cache."""
    g = torch.Generator().manual_seed(len(cuts))
    B, Hq, Hkv, S, D = 2, 8, 2, 1000, 128
    q = torch.randn(B, Hq, 1, D, generator=g).half().to(dev)
    K = torch.randn(B, Hkv, S, D, generator=g).half().to(dev)
    V = torch.randn(B, Hkv, S, D, generator=g).half().to(dev)
    parts = [dec.flash_attention_decode(q, K[:, :, a:b], V[:, :, a:b], 1 / math.sqrt(D), Hq // Hkv,
                                        return_lse=True) for a, b in zip(cuts[:-1], cuts[1:])]
    o = torch.stack([p[0][:, :, 0] for p in parts])  # [n, B, Hq, D]
    lse = torch.stack([p[1] for p in parts])         # [n, B, Hq]
    mo, ml = merge_states(o.float(), lse, out_dtype=torch.float16)
    mo = mo.unsqueeze(2)
    full_o, full_l = dec.flash_attention_decode(q, K, V, 1 / math.sqrt(D), Hq // Hkv,
                                                return_lse=True)
    ro, rl = naive.decode(q.cpu(), K.cpu(), V.cpu(), 1 / math.sqrt(D), Hq // Hkv)
    assert_close(mo, ro, what="merged O vs oracle")
    assert_close(ml, rl, atol=LSE_ATOL, what="merged LSE vs oracle")
    assert_close(mo, full_o, what="merged O vs full decode")
