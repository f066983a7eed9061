"""Fused decode ops on hand-written HIP kernels (gfx950), behind libkoptim's C ABI.

Python signatures mirror engine/kernels/fused.py of the reference so the ops
drop into engine.py unchanged:

- ``DecodeAttention(B, T, cap, nq, nkv, d, device, target_ctas=...)`` and
  ``__call__(q, k_cache, v_cache, pos, out)``      (fused.py:204-234)
- ``add_rms_norm(res, delta, weight, out, eps)``    (fused.py:39-46)
- ``qk_norm_rope(qkv, q_w, k_w, cos, sin, pos, q_out, k_cache, v_cache, T, eps, nq, nkv, d)``
                                                    (fused.py:99-106)
- ``silu_mul(gu, out)``                             (fused.py:123-127)

All tensors are caller-owned; every call launches on the current stream,
allocates nothing and never synchronises, so calls are graph-capturable.
Shapes, dtypes and contiguity are validated on the host and a bad argument
raises ValueError before anything is launched.
"""

import torch

from .. import _lib

BF16 = torch.bfloat16


def _cdiv(a, b):
    return -(-a // b)


def _need(cond, msg):
    if not cond:
        raise ValueError(msg)


def _check(t, name, dtype, shape=None, contiguous=True):
    _need(isinstance(t, torch.Tensor), f"{name} must be a tensor")
    _need(t.dtype == dtype, f"{name} must be {dtype}, got {t.dtype}")
    _need(t.is_cuda, f"{name} must be on the GPU")
    if shape is not None:
        _need(tuple(t.shape) == tuple(shape), f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")
    if contiguous:
        _need(t.is_contiguous(), f"{name} must be contiguous")


def _check_cache(t, name, B, nkv, cap, d):
    _need(t.dim() == 4, f"{name} must be [B, nkv, cap, d]")
    _need(tuple(t.shape) == (B, nkv, cap, d), f"{name} must have shape {(B, nkv, cap, d)}, got {tuple(t.shape)}")
    _need(t.dtype == BF16 and t.is_cuda, f"{name} must be a bf16 GPU tensor")
    _need(t.stride(3) == 1 and t.stride(2) == d, f"{name}: sequence stride must be d and inner stride 1")


# ---------------------------------------------------------------------------
# Split-K GQA decode attention (fused.py:130-234).
# ---------------------------------------------------------------------------
class DecodeAttention:
    """Preallocated split-K attention for T query tokens per sequence, fixed (B, T, cap).

    Work is cut into units of ``unit`` keys per (sequence, KV head); the units
    of each call are enumerated on the GPU from the device-side lengths, so
    only valid keys are read and short sequences take few units. A fixed grid
    of ``grid_waves`` wavefronts strides over the units (graph-safe).
    ``target_ctas`` is the number of wavefronts to fill the GPU with
    (256 CUs x 8 by default).
    """

    MAX_T = 4

    def __init__(self, B, T, cap, nq, nkv, d, device, target_ctas=2048, unit=None):
        _need(d == 128, "head_dim must be 128")
        _need(nq == 4 * nkv, "the kernel serves GQA groups of 4 query heads per KV head")
        _need(1 <= T <= self.MAX_T, f"T must be in 1..{self.MAX_T}")
        self.B, self.T, self.cap, self.nq, self.nkv, self.d = B, T, cap, nq, nkv, d
        if unit is None:
            unit = _cdiv(_cdiv(B * nkv * cap, target_ctas), 16) * 16
            unit = max(64, min(1024, unit))
        _need(unit % 16 == 0 and unit >= 16, "unit must be a positive multiple of 16")
        self.unit = unit
        self.max_units = _cdiv(cap, unit)
        self.grid_waves = max(1, min(B * nkv * self.max_units, target_ctas))
        rows = B * T * nq
        self.o_part = torch.empty(rows * self.max_units * d, dtype=torch.float32, device=device)
        self.ml = torch.empty(rows * self.max_units * 2, dtype=torch.float32, device=device)
        self.scale = d ** -0.5

    def _run(self, q, k_cache, v_cache, lens, len_offset, out):
        B, T, nq, nkv, d, cap = self.B, self.T, self.nq, self.nkv, self.d, self.cap
        _check(q, "q", BF16, (B * T, nq * d))
        _check(out, "out", BF16, (B * T, nq * d))
        _check_cache(k_cache, "k_cache", B, nkv, cap, d)
        _check_cache(v_cache, "v_cache", B, nkv, cap, d)
        _need(k_cache.stride() == v_cache.stride(), "k_cache and v_cache must share strides")
        _check(lens, "pos/lengths", torch.int32, (B,))
        _lib.call("ko_decode_attn", _lib.ptr(q), _lib.ptr(k_cache), _lib.ptr(v_cache),
                  _lib.ptr(lens), len_offset, cap, k_cache.stride(0), k_cache.stride(1),
                  B, T, nkv, d, self.unit, self.max_units, self.grid_waves, self.scale,
                  _lib.ptr(self.o_part), _lib.ptr(self.ml), _lib.ptr(out), _lib.stream_ptr())

    def __call__(self, q, k_cache, v_cache, pos, out):
        """q: [B*T, NQ*D]; k/v_cache: [B, NKV, cap, D]; pos: [B] int32 (first query
        position; keys 0..pos+T-1 are valid); out: [B*T, NQ*D]."""
        self._run(q, k_cache, v_cache, pos, self.T, out)

    def with_lengths(self, q, k_cache, v_cache, lengths, out):
        """Ragged form: lengths[b] = number of valid keys of sequence b (int32);
        the T queries sit at positions lengths[b]-T .. lengths[b]-1."""
        self._run(q, k_cache, v_cache, lengths, 0, out)
