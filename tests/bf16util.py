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


def bf16_ulp(t):
    """One bf16 ulp at each element's own magnitude (2^(floor(log2|v|) - 7));
    the smallest normal's ulp at zero."""
    _, e = torch.frexp(t.float().abs().clamp_min(2.0 ** -126))
    return torch.ldexp(torch.ones_like(t, dtype=torch.float32), e - 8)


def assert_resid_close(got, want, y, max_frac=0.02):
    """h <- bf16(h + bf16(y)) against the oracle's: the fp32 sums y may round to
    bf16 one ulp of y apart (near a tie), which the second rounding carries into
    h as up to ulp(y) + ulp(h) (many ulps of h where h + y cancels)."""
    d = (got.float() - want.float()).abs()
    bound = bf16_ulp(y) + bf16_ulp(want)
    bad = d > bound
    assert not bool(bad.any()), f"{int(bad.sum())} elements beyond ulp(y) + ulp(h)"
    assert float((d > 0).float().mean()) <= max_frac, f"mismatch fraction {float((d > 0).float().mean())}"
