"""bf16 comparison helpers shared by the tests."""

import torch

BF = torch.bfloat16


def ulps(a, b):
    """Distance in bf16 units in the last place between two bf16 tensors."""
    ia = a.view(torch.int16).to(torch.int32)
    ib = b.view(torch.int16).to(torch.int32)
    # map sign-magnitude to a monotonic integer line
    ia = torch.where(ia < 0, -32768 - ia, ia)
    ib = torch.where(ib < 0, -32768 - ib, ib)
    return (ia - ib).abs()


def rms(t):
    return float(t.float().pow(2).mean().sqrt())


def assert_bf16_close(got, want, max_ulp=1, max_frac=0.01, atol=0.0):
    """Every element within ``max_ulp`` bf16 ulps of the reference, or within
    ``atol`` absolutely (for results near zero after cancellation, where one ulp
    of an input is many ulps of the result); at most ``max_frac`` of the
    elements differ at all."""
    assert got.dtype == BF and want.dtype == BF and got.shape == want.shape
    d = ulps(got, want)
    bad = (d > max_ulp) & ((got.float() - want.float()).abs() > atol)
    assert not bool(bad.any()), (
        f"{int(bad.sum())} elements beyond {max_ulp} ulp / atol {atol:g}; max ulp diff {int(d.max())}")
    assert float((d > 0).float().mean()) <= max_frac, f"mismatch fraction {float((d > 0).float().mean())}"


def one_ulp_at(t):
    """Absolute size of one bf16 ulp at the tensor's typical magnitude."""
    return 2.0 ** -7 * rms(t)
