"""Shared comparison helpers for the test suite."""
import torch

# Parity bar of the hot path: max abs error of the fp16 output against the
# fp64 oracle computed from the same fp16 inputs.
ATOL = 2e-3


def max_abs_err(got, ref, mask=None):
    g = got.detach().cpu().to(torch.float64)
    r = ref.detach().cpu().to(torch.float64)
    d = (g - r).abs()
    if mask is not None:
        d = d[mask]
    if d.numel() == 0:
        return 0.0
    if torch.isnan(d).any():
        return float("inf")
    return float(d.max())


def assert_close(got, ref, atol=ATOL, what="", mask=None):
    err = max_abs_err(got, ref, mask)
    assert err <= atol, f"{what}: max abs err {err:.3e} > {atol:.1e}"
    return err
