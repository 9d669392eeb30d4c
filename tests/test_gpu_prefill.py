"""GPU parity of the prefill kernels (R1 dense causal / non-causal, R2 var-len)."""
import math

import pytest
import torch

from attention_kernel_triton_amd import prefill_flash_attention as pre
from attention_kernel_triton_amd import prefill_flash_attention_var_len_padding as prevar
from attention_kernel_triton_amd import synthetic as syn
from helpers import ATOL, assert_close
from oracle import naive

pytestmark = pytest.mark.gpu


def _qkv(seed, B, Hq, Hkv, S, D):
    g = torch.Generator().manual_seed(seed)
    mk = lambda *s: torch.randn(s, generator=g).half()  # noqa: E731
    return mk(B, Hq, S, D), mk(B, Hkv, S, D), mk(B, Hkv, S, D)


@pytest.mark.parametrize("D", [64, 128, 192, 256])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("S", [1, 17, 64, 130, 257])
def test_prefill_small_shapes(dev, D, causal, S):
    B, Hq, Hkv = 2, 4, 2
    Q, K, V = _qkv(S * 7 + D, B, Hq, Hkv, S, D)
    out = pre.flash_attention_prefill(Q.to(dev), K.to(dev), V.to(dev), causal, 1 / math.sqrt(D),
                                      Hq // Hkv)
    ref = naive.prefill(Q, K, V, causal, 1 / math.sqrt(D), Hq // Hkv)
    assert out.shape == Q.shape and out.dtype == torch.float16
    assert_close(out, ref, what=f"prefill D={D} causal={causal} S={S}")


# bf16 bar: the output is rounded to bf16 (8 significant bits; |O| reaches
# about 2 here, where one bf16 ulp is 2^-6) and P is rounded to bf16 for P.V.
ATOL_BF16 = 1.6e-2


@pytest.mark.parametrize("D", [64, 128, 192, 256])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("S", [17, 130])
def test_prefill_bf16_matches_oracle(dev, D, causal, S):
    B, Hq, Hkv = 2, 4, 2
    g = torch.Generator().manual_seed(S * 3 + D)
    Q, K, V = (torch.randn(*sh, generator=g).bfloat16()
               for sh in ((B, Hq, S, D), (B, Hkv, S, D), (B, Hkv, S, D)))
    scale = 1 / math.sqrt(D)
    out, lse = pre.flash_attention_prefill(Q.to(dev), K.to(dev), V.to(dev), causal, scale,
                                           Hq // Hkv, return_lse=True)
    ref, rlse = naive.prefill(Q, K, V, causal, scale, Hq // Hkv, return_lse=True)
    assert out.dtype == torch.bfloat16 and lse.dtype == torch.float32
    err = assert_close(out, ref, atol=ATOL_BF16, what=f"bf16 D={D} causal={causal} S={S}")
    # The bf16 output is the fp64 result rounded: its mean error stays far
    # below the bound (a wrong operand type or layout is off by O(1)).
    mean = (out.float().cpu().double() - ref).abs().mean().item()
    assert mean < 2e-3, f"mean abs err {mean:.2e} (max {err:.2e})"
    assert_close(lse, rlse, atol=1e-2, what=f"bf16 lse D={D}")


def test_prefill_bf16_varlen_config1_shape(dev):
    c = syn.prefill_config(1)
    Q, K, V = (t[:2].bfloat16() for t in (c.Q, c.K, c.V))
    vl = c.varlen[:2]
    out = prevar.flash_attention_prefill(Q.to(dev), K.to(dev), V.to(dev), True, c.scale, c.group,
                                         varlen=vl.to(dev))
    ref = naive.prefill_varlen(Q, K, V, True, c.scale, c.group, vl, dtype=torch.float32)
    S = Q.shape[2]
    valid = (torch.arange(S)[None, :] < vl[:, None])[:, None, :, None].expand(Q.shape)
    assert_close(out, ref, atol=ATOL_BF16, what="bf16 var-len", mask=valid)


def test_prefill_rejects_mixed_dtypes(dev):
    Q, K, V = _qkv(1, 1, 2, 2, 16, 64)
    with pytest.raises(TypeError):
        pre.flash_attention_prefill(Q.to(dev).bfloat16(), K.to(dev), V.to(dev), True, 0.1, 1)
    with pytest.raises(TypeError):
        pre.flash_attention_prefill(Q.to(dev).float(), K.to(dev).float(), V.to(dev).float(),
                                    True, 0.1, 1)


@pytest.mark.parametrize("G", [1, 8])
def test_prefill_group_sizes_and_unmapped_xcd_layout(dev, G):
    B, Hkv, S, D = 3, 1, 200, 64  # B*Hkv not a multiple of 8: linear block order
    Q, K, V = _qkv(G, B, Hkv * G, Hkv, S, D)
    out = pre.flash_attention_prefill(Q.to(dev), K.to(dev), V.to(dev), True, 0.125, G)
    assert_close(out, naive.prefill(Q, K, V, True, 0.125, G), what=f"G={G}")


def test_prefill_strided_inputs(dev):
    B, Hq, Hkv, S, D = 2, 8, 4, 192, 128
    g = torch.Generator().manual_seed(5)
    # [B, S, H, D] storage viewed as [B, H, S, D]
    Qs = torch.randn(B, S, Hq, D, generator=g).half()
    Ks = torch.randn(B, S, Hkv, D, generator=g).half()
    Vs = torch.randn(B, S, Hkv, D, generator=g).half()
    Q, K, V = (t.to(dev).transpose(1, 2) for t in (Qs, Ks, Vs))
    assert not Q.is_contiguous()
    out = pre.flash_attention_prefill(Q, K, V, True, 0.1, 2)
    ref = naive.prefill(Qs.transpose(1, 2), Ks.transpose(1, 2), Vs.transpose(1, 2), True, 0.1, 2)
    assert_close(out, ref, what="strided")


def test_prefill_config0_full(dev):
    c = syn.prefill_config(0)
    out = pre.flash_attention_prefill(c.Q.to(dev), c.K.to(dev), c.V.to(dev), True, c.scale, c.group)
    ref = naive.prefill(c.Q, c.K, c.V, True, c.scale, c.group, dtype=torch.float32)
    err = assert_close(out, ref, what="config 0")
    print(f"config 0 max abs err {err:.3e}")


def test_prefill_varlen_config1_full(dev):
    c = syn.prefill_config(1)
    out = prevar.flash_attention_prefill(c.Q.to(dev), c.K.to(dev), c.V.to(dev), True, c.scale,
                                         c.group, varlen=c.varlen.to(dev))
    ref = naive.prefill_varlen(c.Q, c.K, c.V, True, c.scale, c.group, c.varlen,
                               dtype=torch.float32)
    S = c.Q.shape[2]
    valid = (torch.arange(S)[None, :] < c.varlen[:, None])[:, None, :, None].expand(c.Q.shape)
    err = assert_close(out, ref, what="config 1 valid rows", mask=valid)
    print(f"config 1 max abs err {err:.3e}")


@pytest.mark.parametrize("bits", [32, 64])
def test_prefill_varlen_nonfinite_padding_never_leaks(dev, bits):
    B, Hq, Hkv, S, D = 4, 4, 2, 256, 64
    Q, K, V = _qkv(11, B, Hq, Hkv, S, D)
    lens = torch.tensor([256, 1, 100, 191])
    for b, L in enumerate(lens.tolist()):
        Q[b, :, L:] = float("nan")
        K[b, :, L:] = float("inf")
        V[b, :, L:] = float("nan")
    dt = torch.int32 if bits == 32 else torch.int64
    out = prevar.flash_attention_prefill(Q.to(dev), K.to(dev), V.to(dev), True, 0.125, 2,
                                         varlen=lens.to(dev, dt)).cpu()
    Qc, Kc, Vc = Q.clone(), K.clone(), V.clone()
    for b, L in enumerate(lens.tolist()):
        Qc[b, :, L:] = 0
        Kc[b, :, L:] = 0
        Vc[b, :, L:] = 0
    ref = naive.prefill_varlen(Qc, Kc, Vc, True, 0.125, 2, lens)
    valid = (torch.arange(S)[None, :] < lens[:, None])[:, None, :, None].expand(Q.shape)
    assert torch.isfinite(out[valid]).all()
    assert_close(out, ref, what="var-len padding", mask=valid)


@pytest.mark.parametrize("G", [1, 3, 4, 8])
@pytest.mark.parametrize("D", [64, 128, 256])
def test_prefill_varlen_block_edges_and_idle_workgroups(dev, G, D):
    """Lengths at and around 64-row block edges, an empty sequence and a full one:
    workgroups whose row blocks all lie past ceil(len / 64) * 64 exit at once, and
    with G != 4 one workgroup mixes active and idle waves."""
    Hkv, S = 2, 320
    lens = torch.tensor([0, 1, 63, 64, 65, 200, 320])
    B = len(lens)
    Q, K, V = _qkv(13 + G + D, B, Hkv * G, Hkv, S, D)
    out = prevar.flash_attention_prefill(Q.to(dev), K.to(dev), V.to(dev), True, 1 / math.sqrt(D),
                                         G, varlen=lens.to(dev)).cpu()
    ref = naive.prefill_varlen(Q, K, V, True, 1 / math.sqrt(D), G, lens)
    valid = (torch.arange(S)[None, :] < lens[:, None])[:, None, :, None].expand(Q.shape)
    assert torch.isfinite(out[valid]).all()
    assert_close(out, ref, what=f"var-len edges G={G} D={D}", mask=valid)


def test_prefill_varlen_noncausal_matches_reference_semantics(dev):
    """Non-causal var-len attends all S keys, padding included (reference behaviour)."""
    B, Hq, Hkv, S, D = 2, 2, 1, 130, 64
    Q, K, V = _qkv(12, B, Hq, Hkv, S, D)
    lens = torch.tensor([130, 70])
    out = prevar.flash_attention_prefill(Q.to(dev), K.to(dev), V.to(dev), False, 0.125, 2,
                                         varlen=lens.to(dev))
    ref = naive.prefill_varlen(Q, K, V, False, 0.125, 2, lens)
    valid = (torch.arange(S)[None, :] < lens[:, None])[:, None, :, None].expand(Q.shape)
    assert_close(out, ref, what="non-causal var-len", mask=valid)


def test_prefill_is_deterministic(dev):
    c = syn.prefill_config(0, B=2, Hq=8, Hkv=2, S=512)
    args = (c.Q.to(dev), c.K.to(dev), c.V.to(dev), True, c.scale, c.group)
    a = pre.flash_attention_prefill(*args)
    b = pre.flash_attention_prefill(*args)
    assert torch.equal(a, b)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("G", [2, 3, 6])
def test_prefill_group_sizes_non_power_of_two(dev, D, G):
    """Slots (head f % G, row block f / G) that straddle row blocks inside a workgroup."""
    B, Hkv, S = 2, 2, 150
    Q, K, V = _qkv(40 + G + D, B, Hkv * G, Hkv, S, D)
    out = pre.flash_attention_prefill(Q.to(dev), K.to(dev), V.to(dev), True, 1 / math.sqrt(D), G)
    assert_close(out, naive.prefill(Q, K, V, True, 1 / math.sqrt(D), G), what=f"G={G} D={D}")


@pytest.mark.parametrize("causal", [True, False])
def test_prefill_rising_logits_raise_the_running_max_often(dev, causal):
    """Scores that climb along the keys push the running max up by more than the
    rescale slack step after step, so the rare raise-and-recompute path runs on
    many steps, not only step 0; large magnitudes also exercise fp16 range."""
    B, Hq, Hkv, S, D = 2, 4, 2, 384, 64
    g = torch.Generator().manual_seed(77)
    Q = (torch.randn(B, Hq, S, D, generator=g) * 0.2 + 1.0).half()
    ramp = torch.linspace(0.0, 6.0, S)[None, None, :, None]
    K = (torch.randn(B, Hkv, S, D, generator=g) * 0.2 + ramp).half()
    V = torch.randn(B, Hkv, S, D, generator=g).half()
    out = pre.flash_attention_prefill(Q.to(dev), K.to(dev), V.to(dev), causal, 0.125, Hq // Hkv)
    ref = naive.prefill(Q, K, V, causal, 0.125, Hq // Hkv, dtype=torch.float32)
    assert torch.isfinite(out.cpu()).all()
    assert_close(out, ref, what=f"rising logits causal={causal}")


def test_prefill_nan_query_row_leaves_every_other_row_exact(dev):
    """Rows are independent, as in the reference: a NaN query row gives a NaN
    output row and no other row changes (every row's normaliser is its own)."""
    B, Hq, Hkv, S, D = 1, 2, 1, 128, 64
    Q, K, V = _qkv(91, B, Hq, Hkv, S, D)
    bad = 37
    Q[0, 1, bad] = float("nan")
    out = pre.flash_attention_prefill(Q.to(dev), K.to(dev), V.to(dev), True, 0.125, 2).cpu()
    Qc = Q.clone()
    Qc[0, 1, bad] = 0
    ref = naive.prefill(Qc, K, V, True, 0.125, 2)
    assert not torch.isfinite(out[0, 1, bad]).all()
    keep = torch.ones(B, Hq, S, D, dtype=torch.bool)
    keep[0, 1, bad] = False
    assert torch.isfinite(out[keep]).all()
    assert_close(out, ref, what="rows other than the NaN row", mask=keep)


@pytest.mark.parametrize("D", [64, 128, 256])
def test_prefill_long_sequence(dev, D):
    """An 8192-token causal sequence (128 key tiles per row block at the end)."""
    B, Hq, Hkv, S = 1, 2, 1, 8192
    Q, K, V = _qkv(31 + D, B, Hq, Hkv, S, D)
    out = pre.flash_attention_prefill(Q.to(dev), K.to(dev), V.to(dev), True, 1 / math.sqrt(D), 2)
    ref = naive.prefill(Q, K, V, True, 1 / math.sqrt(D), 2, dtype=torch.float32)
    assert_close(out, ref, what=f"prefill S=8192 D={D}")


@pytest.mark.parametrize("case", ["non-causal", "var-len", "bf16", "G=1"])
def test_prefill_d128_long_sequence_instance(dev, case):
    """From 4096 rows, D = 128 runs its long-sequence instance (two 32-row
    blocks per wave, 64-key tiles, one wave per SIMD).  S = 4100 also leaves a
    partial last row block and key tile."""
    B, Hq, Hkv, S, D = 1, 4, 2, 4100, 128
    if case == "G=1":
        Hq = Hkv = 3
    Q, K, V = _qkv(41 + len(case), B, Hq, Hkv, S, D)
    scale, G = 1 / math.sqrt(D), Hq // Hkv
    causal = case != "non-causal"
    if case == "var-len":
        B = 2
        Q, K, V = _qkv(43, B, Hq, Hkv, S, D)
        lens = torch.tensor([4100, 2345])
        out = prevar.flash_attention_prefill(Q.to(dev), K.to(dev), V.to(dev), True, scale, G,
                                             varlen=lens.to(dev)).cpu()
        ref = naive.prefill_varlen(Q, K, V, True, scale, G, lens, dtype=torch.float32)
        valid = (torch.arange(S)[None, :] < lens[:, None])[:, None, :, None].expand(Q.shape)
        assert_close(out, ref, what="D=128 long var-len", mask=valid)
        return
    if case == "bf16":
        Q, K, V = Q.bfloat16(), K.bfloat16(), V.bfloat16()
    out, lse = pre.flash_attention_prefill(Q.to(dev), K.to(dev), V.to(dev), causal, scale, G,
                                           return_lse=True)
    ref, rl = naive.prefill(Q, K, V, causal, scale, G, dtype=torch.float32, return_lse=True)
    assert_close(out, ref, atol=ATOL_BF16 if case == "bf16" else ATOL, what=f"D=128 long {case}")
    assert_close(lse, rl, atol=1e-2 if case == "bf16" else 2e-3, what=f"D=128 long {case} lse")


@pytest.mark.parametrize("D", [192, 256])
@pytest.mark.parametrize("causal", [True, False])
def test_prefill_head_dims_192_and_256(dev, causal, D):
    """D = 192 and 256 (the reference accepts any multiple of 64,
    prefill_flash_attention.py:351; its sparse harnesses use 256): 32-row slots and
    32-key tiles, with the LSE."""
    B, Hq, Hkv, S = 2, 8, 2, 1000
    Q, K, V = _qkv(D + causal, B, Hq, Hkv, S, D)
    out, lse = pre.flash_attention_prefill(Q.to(dev), K.to(dev), V.to(dev), causal,
                                           1 / math.sqrt(D), Hq // Hkv, return_lse=True)
    ref, rl = naive.prefill(Q, K, V, causal, 1 / math.sqrt(D), Hq // Hkv, return_lse=True)
    assert_close(out, ref, what=f"D={D} causal={causal}")
    assert_close(lse, rl, atol=2e-3, what=f"D={D} lse causal={causal}")


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("scale", [-0.125, 0.0, -1.5])
def test_prefill_any_finite_softmax_scale(dev, D, causal, scale):
    """The reference's naive path takes any scale (prefill_flash_attention.py:415-425).
    A negative scale runs as (-Q) K^T at |scale|; scale 0 weights every visible key
    equally, and its LSE is ln(number of visible keys)."""
    B, Hq, Hkv, S = 1, 4, 1, 300
    Q, K, V = _qkv(int(100 * abs(scale)) + D + causal, B, Hq, Hkv, S, D)
    out, lse = pre.flash_attention_prefill(Q.to(dev), K.to(dev), V.to(dev), causal, scale,
                                           Hq // Hkv, return_lse=True)
    ref, rl = naive.prefill(Q, K, V, causal, scale, Hq // Hkv, return_lse=True)
    assert_close(out, ref, what=f"scale={scale} D={D} causal={causal}")
    assert_close(lse, rl, atol=2e-3, what=f"scale={scale} lse")
    if scale == 0.0:
        visible = torch.arange(1, S + 1) if causal else torch.full((S,), S)
        assert_close(lse[0, 0], torch.log(visible.double()), atol=1e-5, what="ln n at scale 0")


def test_prefill_negative_scale_bf16(dev):
    B, Hq, Hkv, S, D = 1, 4, 2, 200, 64
    g = torch.Generator().manual_seed(77)
    Q, K, V = (torch.randn(*sh, generator=g).bfloat16()
               for sh in ((B, Hq, S, D), (B, Hkv, S, D), (B, Hkv, S, D)))
    out = pre.flash_attention_prefill(Q.to(dev), K.to(dev), V.to(dev), True, -0.125, Hq // Hkv)
    ref = naive.prefill(Q, K, V, True, -0.125, Hq // Hkv)
    assert_close(out, ref, atol=ATOL_BF16, what="bf16 negative scale")
