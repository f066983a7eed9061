"""GPU: ko_decode_attn_noalloc, the allocation-free form of ko_decode_attn (its
partials in the library's fixed per-GPU array), against ko_decode_attn with the
caller's scratch (the same kernels: bit-equal), through the C ABI:
- two calls in a row, the second with a smaller input (B = 16 x 8192 keys, then
  3 ragged sequences of a 700-key cache), so the second reuses the array the
  first left behind;
- a call whose partials do not fit the array is refused on the host before any
  launch (KO_ERANGE), and the array still serves the next call;
- in a fresh process, the entry point's first call (the one that looks up the
  array's device address) made under torch CUDA-graph capture, before any other
  launch of the library; the graph is replayed three times with the scratch
  form run eagerly between replays, and every replay is bit-equal to it."""

import os
import subprocess
import sys

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


_CAPTURED_FIRST = r'''
import torch
from kernel_optim_amd import _lib
from kernel_optim_amd.kernels.fused import DecodeAttention

dev = torch.device("cuda:0")
NQ, NKV, D = 32, 8, 128
B, cap, lens = 3, 700, [700, 1, 333]
g = torch.Generator(device=dev).manual_seed(4)
q = torch.randn(B, NQ * D, device=dev, generator=g).to(torch.bfloat16)
k = torch.randn(B, NKV, cap, D, device=dev, generator=g).to(torch.bfloat16)
v = torch.randn(B, NKV, cap, D, device=dev, generator=g).to(torch.bfloat16)
pos = torch.tensor([l - 1 for l in lens], dtype=torch.int32, device=dev)
att = DecodeAttention(B, 1, cap, NQ, NKV, D, dev)  # no library launch yet
out = torch.full_like(q, float("nan"))
torch.cuda.synchronize()
print("capturing the first ko_decode_attn_noalloc call", flush=True)
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):
    rc = _lib.lib().ko_decode_attn_noalloc(
        _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(pos), 1, cap, k.stride(0), k.stride(1),
        B, 1, NKV, D, att.unit, att.max_units, att.grid_waves, att.scale, _lib.ptr(out),
        _lib.stream_ptr())
print("capture rc", rc, flush=True)
assert rc == 0, rc
want = torch.empty_like(q)
for i in range(3):
    out.fill_(float("nan"))
    graph.replay()
    att(q, k, v, pos, want)  # the scratch form, eagerly, between replays
    torch.cuda.synchronize()
    assert torch.equal(out, want), ("replay", i)
print("replays bit-equal", flush=True)
'''


def test_noalloc_first_call_under_graph_capture():
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, PYTHONPATH=root + os.pathsep + os.environ.get("PYTHONPATH", ""))
    proc = subprocess.run([sys.executable, "-c", _CAPTURED_FIRST], cwd=root, env=env,
                          capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0, proc.stdout[-2000:] + proc.stderr[-4000:]
    assert "replays bit-equal" in proc.stdout
