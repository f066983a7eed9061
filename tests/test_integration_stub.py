"""CPU: the ctypes stub of the repository's integration guide (its ``_geometry``
code block) sizes DecodeAttention's launch exactly as
kernel_optim_amd.kernels.fused.DecodeAttention does (kernels/fused.py, attn_geometry),
so a maintainer who binds the C ABI that way gets the same unit, partial buffers and
grid. The stub's sizing function is taken from the guide's code block itself."""

import ast
import os

import pytest

from kernel_optim_amd.kernels.fused import attn_geometry

DOC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "INTEGRATION.md")


def _stub_geometry():
    text = open(DOC).read()
    blocks = [b.split("```", 1)[0] for b in text.split("```python\n")[1:]]
    for block in blocks:
        tree = ast.parse(block)
        for node in tree.body:
            if isinstance(node, ast.FunctionDef) and node.name == "_geometry":
                ns = {}
                exec(compile(ast.Module(body=[node], type_ignores=[]), DOC, "exec"), ns)
                return ns["_geometry"]
    raise AssertionError("INTEGRATION.md has no _geometry stub")


# the attention configurations of the benchmark (B, T, cap, nkv) and the T > 1
# calls of the verify step (up to 8 query tokens)
CASES = [
    (1, 1, 512, 8),       # single decode-attention step, 512 cached keys
    (16, 1, 8192, 8),     # B = 16 x 8192 keys
    (64, 1, 16384, 8),    # ragged B = 64 over a 16384-key cache
    (1, 1, 1296, 8), (2, 1, 640, 8), (4, 1, 2064, 8), (130, 1, 700, 8), (3, 1, 700, 2),
    (1, 7, 1296, 8), (4, 3, 2048, 8), (2, 5, 600, 8), (16, 8, 8192, 8),
]


@pytest.mark.parametrize("B,T,cap,nkv", CASES)
@pytest.mark.parametrize("target_ctas", [2048, 264, 8192])
def test_stub_sizes_the_launch_as_decode_attention(B, T, cap, nkv, target_ctas):
    unit, max_units, _, grid = attn_geometry(B, T, cap, nkv, target_ctas)
    assert _stub_geometry()(B, T, cap, nkv, target_ctas) == (unit, max_units, grid)
    # the kernel's own limits on what the stub passes (attention.hip check_common)
    assert unit % 16 == 0 and max_units * unit >= cap and 1 <= grid <= target_ctas


@pytest.mark.parametrize("B,T,cap,nkv", CASES)
def test_decode_attention_object_takes_that_geometry(B, T, cap, nkv):
    """DecodeAttention's constructor (host arithmetic only: its buffers on the CPU)
    takes attn_geometry's sizing and sizes the partials, counters and sync words
    from it."""
    from kernel_optim_amd import _lib
    from kernel_optim_amd.kernels.fused import DecodeAttention
    att = DecodeAttention(B, T, cap, 4 * nkv, nkv, 128, "cpu", fused_combine=True)
    unit, max_units, wpu, grid = attn_geometry(B, T, cap, nkv)
    assert (att.unit, att.max_units, att.waves_per_unit, att.grid_waves) == (unit, max_units, wpu, grid)
    rows = B * T * 4 * nkv
    assert att.o_part.numel() == rows * max_units * 128 and att.ml.numel() == rows * max_units * 2
    assert att.counters.numel() == B * nkv and int(att.counters.abs().sum()) == 0
    assert att.sync.numel() == _lib.lib().ko_decode_attn_qkv_oproj_sync_ints()
