"""GPU: ko_decode_attn_noalloc, the allocation-free form of ko_decode_attn (its
partials in the library's fixed per-GPU array), against ko_decode_attn with the
caller's scratch (the same kernels: bit-equal), through the C ABI:
- two calls in a row, the second with a smaller input (B = 16 x 8192 keys, then
  3 ragged sequences of a 700-key cache), so the second reuses the array the
  first left behind;
- a call whose partials do not fit the array is refused on the host before any
  launch (KO_ERANGE), and the array still serves the next call."""

import pytest
import torch

from kernel_optim_amd import _lib
from kernel_optim_amd.kernels.fused import DecodeAttention

pytestmark = pytest.mark.gpu
NQ, NKV, D = 32, 8, 128
KO_ERANGE = -34


def _case(dev, B, cap, lens, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    q = torch.randn(B, NQ * D, device=dev, generator=g).to(torch.bfloat16)
    k = torch.randn(B, NKV, cap, D, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(B, NKV, cap, D, device=dev, generator=g).to(torch.bfloat16)
    pos = torch.tensor([l - 1 for l in lens], dtype=torch.int32, device=dev)
    return q, k, v, pos


def _noalloc(att, q, k, v, pos, out, max_units=None):
    return _lib.lib().ko_decode_attn_noalloc(
        _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(pos), 1, att.cap, k.stride(0),
        k.stride(1), att.B, 1, NKV, D, att.unit, max_units or att.max_units, att.grid_waves,
        att.scale, _lib.ptr(out), _lib.stream_ptr())


def test_noalloc_matches_the_scratch_entry_point(dev):
    for B, cap, lens, seed in ((16, 8192, [8192] * 16, 1), (3, 700, [700, 1, 333], 2)):
        q, k, v, pos = _case(dev, B, cap, lens, seed)
        att = DecodeAttention(B, 1, cap, NQ, NKV, D, dev)   # two launches, own scratch
        want = torch.empty_like(q)
        att(q, k, v, pos, want)
        got = torch.full_like(q, float("nan"))
        assert _noalloc(att, q, k, v, pos, got) == 0
        torch.cuda.synchronize()
        assert torch.equal(got, want), (B, cap)


def test_noalloc_refuses_partials_beyond_its_array(dev):
    B, cap = 2, 4096
    q, k, v, pos = _case(dev, B, cap, [4096, 100], 3)
    att = DecodeAttention(B, 1, cap, NQ, NKV, D, dev)
    out = torch.zeros_like(q)
    # 2 x 32 rows x 600 units x 130 floats > 4 Mi floats: refused, nothing launched
    assert _noalloc(att, q, k, v, pos, out, max_units=600) == KO_ERANGE
    torch.cuda.synchronize()
    assert torch.equal(out, torch.zeros_like(q))
    with pytest.raises(RuntimeError, match="size out of range"):
        _lib.call("ko_decode_attn_noalloc", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(pos),
                  1, cap, k.stride(0), k.stride(1), B, 1, NKV, D, att.unit, 600, att.grid_waves,
                  att.scale, _lib.ptr(out), _lib.stream_ptr())
    want = torch.empty_like(q)
    att(q, k, v, pos, want)
    assert _noalloc(att, q, k, v, pos, out) == 0
    torch.cuda.synchronize()
    assert torch.equal(out, want)
