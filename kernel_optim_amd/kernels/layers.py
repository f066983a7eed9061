"""Every decoder layer of one decode step in one launch (one query token, 1-2 sequences).

The per-layer loop of the reference's decode step (engine/engine.py:325-335:
add_rms_norm, the qkv projection, qk_norm_rope, decode attention, the o
projection with its residual add, add_rms_norm, the gate|up projection,
silu_mul, the down projection) as one ``ko_decode_layers`` launch: five stages
of workgroups per layer, each stage's weights streaming before its input exists
and a device-coherent hand-off between the stages. The arithmetic and rounding
are those of the per-op launches with the layout-0 GEMV (8 output columns per
workgroup) and the one-token attention with the fused combine.
"""

import ctypes

import torch

from .. import _lib
from .fused import BF16, DecodeAttention, _check, _need

_FIELDS = ("w_in", "qkv", "q_norm", "k_norm", "o", "w_post", "gu", "down")


class DecodeLayers:
    """Launch state for ``ko_decode_layers``: the device table of per-layer weight
    and cache pointers, the per-layer combine counters, the stage hand-off flags
    and the wait-failure flag.

    ``layers``: per-layer dicts with the engine's weight names (w_in [H],
    qkv [(nq+2nkv)*d, H], q_norm/k_norm [d], o [H, nq*d], w_post [H],
    gu [2I, H], down [H, I]); ``k_cache``/``v_cache``: [L, B, nkv, cap, d];
    ``attn``: the step's DecodeAttention (its unit, grid and o_part/ml scratch).
    The tensors must stay alive and in place while this object is used."""

    @staticmethod
    def supported(attn, hidden, inter):
        """The launch serves 1-2 sequences of one token each, 4 wavefronts per
        attention unit, hidden and nq*d up to 4096, intermediate up to 10240."""
        return (attn.T == 1 and attn.B <= 2 and attn.waves_per_unit == 4
                and attn.nq * attn.d <= 4096 and hidden <= 4096 and hidden % 8 == 0
                and inter <= 10240 and inter % 8 == 0)

    def __init__(self, attn: DecodeAttention, layers, k_cache, v_cache, hidden, inter):
        _need(self.supported(attn, hidden, inter), "decode_layers: unsupported shape")
        B, nq, nkv, d, cap = attn.B, attn.nq, attn.nkv, attn.d, attn.cap
        L = len(layers)
        _need(L >= 1, "decode_layers needs at least one layer")
        H, I = hidden, inter
        _need(tuple(k_cache.shape) == (L, B, nkv, cap, d) and k_cache.is_contiguous()
              and k_cache.dtype == BF16, "k_cache must be a contiguous bf16 [L, B, nkv, cap, d]")
        _need(tuple(v_cache.shape) == tuple(k_cache.shape) and v_cache.is_contiguous()
              and v_cache.dtype == BF16, "v_cache must match k_cache")
        shapes = {"w_in": (H,), "qkv": ((nq + 2 * nkv) * d, H), "q_norm": (d,), "k_norm": (d,),
                  "o": (H, nq * d), "w_post": (H,), "gu": (2 * I, H), "down": (H, I)}
        rows = []
        for i, lw in enumerate(layers):
            for f in _FIELDS:
                _check(lw[f], f"layers[{i}].{f}", BF16, shapes[f])
                _need(lw[f].data_ptr() % 16 == 0, f"layers[{i}].{f} must be 16-byte aligned")
            rows.append([lw[f].data_ptr() for f in _FIELDS]
                        + [k_cache[i].data_ptr(), v_cache[i].data_ptr()])
        dev = k_cache.device
        self.table = torch.tensor(rows, dtype=torch.int64).to(dev)
        self._keep = (layers, k_cache, v_cache)
        self.attn, self.L, self.H, self.I = attn, L, H, I
        self.cache_strides = (k_cache.stride(1), k_cache.stride(2))
        self.counters = torch.zeros(L * B * nkv, dtype=torch.int32, device=dev)
        self.sync = torch.zeros(_lib.lib().ko_decode_layers_sync_ints(L), dtype=torch.int32,
                                device=dev)
        self.err = torch.zeros(1, dtype=torch.int32, device=dev)
        self.o_delay_ns = 1000
        # workgroups of the qkv, o, gate|up and down stages (0: the library default)
        self.gemv_wgs = (ctypes.c_int * 4)(0, 0, 0, 0)

    def __call__(self, h, qkv, attn_out, act, pos, cos, sin, eps):
        """One decode step's layers at positions pos[b] (the new token's KV slot):
        h [B, H] in (the embeddings) and out (the last layer's residual stream);
        qkv [B, (nq+2nkv)*d], attn_out [B, nq*d], act [B, I] are scratch."""
        at = self.attn
        B, nq, nkv, d = at.B, at.nq, at.nkv, at.d
        _check(h, "h", BF16, (B, self.H))
        _check(qkv, "qkv", BF16, (B, (nq + 2 * nkv) * d))
        _check(attn_out, "attn_out", BF16, (B, nq * d))
        _check(act, "act", BF16, (B, self.I))
        _check(pos, "pos", torch.int32, (B,))
        _check(cos, "cos", BF16)
        _check(sin, "sin", BF16)
        _need(cos.dim() == 2 and cos.shape[1] == d and tuple(sin.shape) == tuple(cos.shape),
              "cos/sin must be [rows, d]")
        _lib.call("ko_decode_layers", _lib.ptr(self.table), self.L, _lib.ptr(h), _lib.ptr(qkv),
                  _lib.ptr(attn_out), _lib.ptr(act), B, self.H, self.I, nkv, d, _lib.ptr(cos),
                  _lib.ptr(sin), cos.shape[0], _lib.ptr(pos), at.cap, *self.cache_strides,
                  at.unit, at.max_units, at.grid_waves, eps, at.scale, _lib.ptr(at.o_part),
                  _lib.ptr(at.ml), _lib.ptr(self.counters), _lib.ptr(self.sync),
                  _lib.ptr(self.err), self.gemv_wgs, self.o_delay_ns, _lib.stream_ptr())
