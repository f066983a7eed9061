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
def attn_geometry(B, T, cap, nkv, target_ctas=2048, unit=None, token_rows=False,
                  units_per_seq=0):
    """Launch geometry of DecodeAttention: (keys per unit, units per (sequence, KV
    head) that the partials are sized for, wavefronts per unit, grid in
    wavefronts). The reference sizes its split the same way, from the cache
    length over the programs it wants in flight (fused.py:209-218)."""
    wg_split = T == 1 or token_rows
    rows_k = B * T if token_rows else B  # rows the one-token kernel sizes for
    if unit is None:
        share = _cdiv(_cdiv(rows_k * nkv * cap, target_ctas), 16) * 16  # keys per wavefront
        # one-token units stop at 4096 keys (the kernel deals several rounds
        # of units out largest first, so ragged lengths still fill the
        # rounds evenly; 4096 against 2048 keys: +1-4.5 % at B = 8-64,
        # 4096-32768 keys, and ragged B = 64 6,508 against 6,277 GB/s)
        unit = 4 * max(16, min(1024, share)) if wg_split else max(64, min(1024, share))
        # ... unless one unit of 2048-4096 keys per CU covers the whole cache:
        # then a single round of equal units, with the fewest partials to merge
        per_cu = _cdiv(_cdiv(rows_k * nkv * cap, max(1, target_ctas // 8)), 64) * 64
        if wg_split and 2048 <= per_cu <= 4096:
            unit = per_cu
    max_units = _cdiv(cap, unit)
    # wavefronts per unit: the kernel's rule (attention.hip, waves_per_unit)
    wpu = (4 if unit % 64 == 0 else 2 if unit % 32 == 0 else 1) if wg_split else 1
    units = min(max_units, units_per_seq) if units_per_seq else max_units
    return unit, max_units, wpu, max(1, min(rows_k * nkv * units * wpu, target_ctas))


class DecodeAttention:
    """Preallocated split-K attention for T query tokens per sequence, fixed (B, T, cap).

    Work is cut into units of ``unit`` keys per (sequence, KV head); the units
    of each call are enumerated on the GPU from the device-side lengths, so
    only valid keys are read and short sequences take few units. A fixed grid
    of ``grid_waves`` wavefronts strides over the units (graph-safe).
    ``target_ctas`` is the number of wavefronts to fill the GPU with
    (256 CUs x 8 by default). For one query token per sequence a unit is
    shared by the 4 wavefronts of a workgroup (merged in LDS), so the unit is
    4x the per-wavefront share.

    A second launch merges the partials, as the reference does; with
    ``fused_combine`` the last unit of each (sequence, KV head) merges them in
    the same launch instead, through an arrival counter. The partials and the
    counter travel through device-coherent stores, loads and atomics (no fence,
    no L2 write-back).
    """

    MAX_T = 8

    def __init__(self, B, T, cap, nq, nkv, d, device, target_ctas=2048, unit=None,
                 fused_combine=False, token_rows=False, units_per_seq=0):
        _need(d == 128, "head_dim must be 128")
        _need(nq == 4 * nkv, "the kernel serves GQA groups of 4 query heads per KV head")
        _need(1 <= T <= self.MAX_T, f"T must be in 1..{self.MAX_T}")
        _need(not token_rows or (T >= 2 and fused_combine),
              "token_rows serves T >= 2 with the fused combine")
        self.B, self.T, self.cap, self.nq, self.nkv, self.d = B, T, cap, nq, nkv, d
        # token_rows: the T tokens of a sequence run as T rows of the one-token
        # kernel (ko_decode_attn_token_rows), each with its own causal length
        self.token_rows = bool(token_rows)
        # units_per_seq = U > 0: decode_qkv cuts each sequence's keys into at most U
        # equal units (multiples of 64 keys, at least `unit`) from its length at
        # each step, so a batch of equal lengths fills one round of the grid
        # whatever the position (ko_decode_attn_qkv)
        self.units_per_seq = int(units_per_seq)
        if self.units_per_seq:
            _need(self.units_per_seq > 0 and T == 1 and not self.token_rows and fused_combine
                  and B <= 64, "units_per_seq serves one token per sequence, B <= 64, with "
                  "the fused combine")
            unit = 64 if unit is None else unit
            _need(unit % 64 == 0, "units_per_seq needs a unit (the smallest unit) % 64 == 0")
        _need(unit is None or (unit % 16 == 0 and unit >= 16),
              "unit must be a positive multiple of 16")
        self.unit, self.max_units, self.waves_per_unit, self.grid_waves = attn_geometry(
            B, T, cap, nkv, target_ctas, unit, self.token_rows, self.units_per_seq)
        rows = B * T * nq
        self.o_part = torch.empty(rows * self.max_units * d, dtype=torch.float32, device=device)
        self.ml = torch.empty(rows * self.max_units * 2, dtype=torch.float32, device=device)
        # per-(sequence or token row, KV head) arrival counters; every launch leaves
        # them at zero
        rows_k = B * T if self.token_rows else B  # rows of the one-token kernel
        self.counters = (torch.zeros(rows_k * nkv, dtype=torch.int32, device=device)
                         if fused_combine else None)
        # decode_qkv_oproj: its counters and done flags, and its wait-failure flag
        self.sync = torch.zeros(_lib.lib().ko_decode_attn_qkv_oproj_sync_ints(), dtype=torch.int32,
                                device=device)
        self.err = torch.zeros(1, dtype=torch.int32, device=device)
        self.oproj_delay_ns = 1000
        # polls of a pair's done flag before a decode_qkv_oproj wait gives up and
        # sets err (-1: the library's bound; 0: give up at once, for tests)
        self.oproj_spin = -1
        self.scale = d ** -0.5

    def _check_kv(self, k_cache, v_cache, lens):
        B, nkv, d, cap = self.B, self.nkv, self.d, self.cap
        _check_cache(k_cache, "k_cache", B, nkv, cap, d)
        _check_cache(v_cache, "v_cache", B, nkv, cap, d)
        _need(k_cache.stride() == v_cache.stride(), "k_cache and v_cache must share strides")
        _check(lens, "pos/lengths", torch.int32, (B,))

    def _run(self, q, k_cache, v_cache, lens, len_offset, out):
        B, T, nq, nkv, d, cap = self.B, self.T, self.nq, self.nkv, self.d, self.cap
        _check(q, "q", BF16, (B * T, nq * d))
        _check(out, "out", BF16, (B * T, nq * d))
        self._check_kv(k_cache, v_cache, lens)
        _lib.call("ko_decode_attn", _lib.ptr(q), _lib.ptr(k_cache), _lib.ptr(v_cache),
                  _lib.ptr(lens), len_offset, cap, k_cache.stride(0), k_cache.stride(1),
                  B, T, nkv, d, self.unit, self.max_units, self.grid_waves, self.scale,
                  _lib.ptr(self.o_part), _lib.ptr(self.ml), _lib.ptr(self.counters),
                  _lib.ptr(out), _lib.stream_ptr())

    def __call__(self, q, k_cache, v_cache, pos, out):
        """q: [B*T, NQ*D]; k/v_cache: [B, NKV, cap, D]; pos: [B] int32 (first query
        position; keys 0..pos+T-1 are valid); out: [B*T, NQ*D]."""
        if self.token_rows:
            B, T, nq, nkv, d = self.B, self.T, self.nq, self.nkv, self.d
            _check(q, "q", BF16, (B * T, nq * d))
            _check(out, "out", BF16, (B * T, nq * d))
            self._check_kv(k_cache, v_cache, pos)
            _lib.call("ko_decode_attn_token_rows", _lib.ptr(q), _lib.ptr(k_cache),
                      _lib.ptr(v_cache), _lib.ptr(pos), self.cap, k_cache.stride(0),
                      k_cache.stride(1), B, T, nkv, d, self.unit, self.max_units,
                      self.grid_waves, self.scale, _lib.ptr(self.o_part), _lib.ptr(self.ml),
                      _lib.ptr(self.counters), _lib.ptr(out), _lib.stream_ptr())
            return
        self._run(q, k_cache, v_cache, pos, self.T, out)

    def with_lengths(self, q, k_cache, v_cache, lengths, out):
        """Ragged form: lengths[b] = number of valid keys of sequence b (int32);
        the T queries sit at positions lengths[b]-T .. lengths[b]-1."""
        _need(not self.token_rows, "with_lengths runs the T-token kernel (token_rows=False)")
        self._run(q, k_cache, v_cache, lengths, 0, out)

    def check_sync(self):
        """Raise RuntimeError if a decode_qkv_oproj launch since the last check gave
        up its wait for the attention (its results are then invalid). Reads one
        int32 from the device, so it synchronises; before raising it clears the
        sync words, the arrival counters and the flag (zeroed sync words are a
        valid start), so the next launch starts clean."""
        if int(self.err.item()) == 0:
            return
        torch.cuda.synchronize(self.err.device)
        self.sync.zero_()
        self.err.zero_()
        if self.counters is not None:
            self.counters.zero_()
        torch.cuda.synchronize(self.err.device)
        raise RuntimeError("decode attention + o projection: the projection's wait for the "
                           "attention timed out; the results of those calls are invalid")

    def oproj_fusable(self):
        """decode_qkv_oproj serves 1-2 sequences with the fused combine and 4
        wavefronts per unit (attention.hip, ko_decode_attn_qkv_oproj)."""
        return (self.T == 1 and self.B <= 2 and self.counters is not None
                and self.waves_per_unit == 4
                and self.nq * self.d <= 4096)

    def _check_rope(self, rope):
        if rope is not None:
            _check(rope, "rope", BF16, (self.B, 2, self.d))

    def decode_qkv_oproj(self, qkv, q_w, k_w, cos, sin, pos, k_cache, v_cache, out, eps, w_o, h,
                         rope=None):
        """decode_qkv and then the o projection with its residual add, in one launch:
        out as decode_qkv leaves it, and h <- bf16(h + bf16(out @ w_o^T)) (the RESID
        GEMV of engine.py:330-331). The projection's weights stream while the
        attention runs. w_o: [H, nq*d] bf16; h: [B, H] bf16; rope: as for
        decode_qkv."""
        B, nq, nkv, d = self.B, self.nq, self.nkv, self.d
        _need(self.oproj_fusable(), "decode_qkv_oproj needs B <= 2, fused_combine and a unit "
                                    "of 4 wavefronts")
        _check(qkv, "qkv", BF16, (B, (nq + 2 * nkv) * d))
        _check(out, "out", BF16, (B, nq * d))
        _check(q_w, "q_w", BF16, (d,))
        _check(k_w, "k_w", BF16, (d,))
        _check(cos, "cos", BF16)
        _check(sin, "sin", BF16)
        _need(cos.dim() == 2 and cos.shape[1] == d and tuple(sin.shape) == tuple(cos.shape),
              "cos/sin must be [rows, d]")
        _need(h.dim() == 2 and h.shape[0] == B, "h must be [B, H]")
        H = h.shape[1]
        _check(h, "h", BF16, (B, H))
        _check(w_o, "w_o", BF16, (H, nq * d))
        self._check_kv(k_cache, v_cache, pos)
        self._check_rope(rope)
        _lib.call("ko_decode_attn_qkv_oproj", _lib.ptr(qkv), _lib.ptr(q_w), _lib.ptr(k_w),
                  _lib.ptr(cos), _lib.ptr(sin), cos.shape[0], _lib.ptr(pos), _lib.ptr(k_cache),
                  _lib.ptr(v_cache), self.cap, k_cache.stride(0), k_cache.stride(1), B, nkv, d,
                  self.unit, self.max_units, self.grid_waves, eps, self.scale,
                  _lib.ptr(self.o_part), _lib.ptr(self.ml), _lib.ptr(self.counters), _lib.ptr(out),
                  _lib.ptr(w_o), _lib.ptr(h), H, _lib.ptr(self.sync), _lib.ptr(self.err),
                  self.oproj_delay_ns, self.oproj_spin, _lib.ptr(rope), _lib.stream_ptr())

    def decode_qkv(self, qkv, q_w, k_w, cos, sin, pos, k_cache, v_cache, out, eps, rope=None):
        """Decode step (T=1) straight from the bf16 QKV projection [B, (nq+2nkv)*d]:
        per-head q/k RMSNorm + RoPE at pos[b], append of k and v at slot pos[b], and
        attention over keys 0..pos[b] -- qk_norm_rope (fused.py:54-96) and this
        op's __call__ with the q/k work folded into the attention launch.
        ``rope`` ([B, 2, d] bf16, optional): the cos and sin rows at pos[b], as
        ``rope_rows`` writes them; with it the kernel needs no table lookup behind
        the position (and at B = 1 issues its first loads before reading it)."""
        B, nq, nkv, d = self.B, self.nq, self.nkv, self.d
        _need(self.T == 1, "decode_qkv serves one decode token per sequence")
        _check(qkv, "qkv", BF16, (B, (nq + 2 * nkv) * d))
        _check(out, "out", BF16, (B, nq * d))
        _check(q_w, "q_w", BF16, (d,))
        _check(k_w, "k_w", BF16, (d,))
        _check(cos, "cos", BF16)
        _check(sin, "sin", BF16)
        _need(cos.dim() == 2 and cos.shape[1] == d and tuple(sin.shape) == tuple(cos.shape),
              "cos/sin must be [rows, d]")
        self._check_kv(k_cache, v_cache, pos)
        self._check_rope(rope)
        _lib.call("ko_decode_attn_qkv", _lib.ptr(qkv), _lib.ptr(q_w), _lib.ptr(k_w),
                  _lib.ptr(cos), _lib.ptr(sin), cos.shape[0], _lib.ptr(pos), _lib.ptr(k_cache),
                  _lib.ptr(v_cache), self.cap, k_cache.stride(0), k_cache.stride(1), B, nkv, d,
                  self.unit, self.max_units, self.grid_waves, eps, self.scale,
                  _lib.ptr(self.o_part), _lib.ptr(self.ml), _lib.ptr(self.counters),
                  _lib.ptr(out), _lib.ptr(rope), self.units_per_seq, _lib.stream_ptr())


def rope_rows(pos, cos, sin, out):
    """out[b] = (cos[p], sin[p]) with p = clamp(pos[b], 0, rows - 1): the RoPE rows
    of each sequence's new position (qk_norm_rope, fused.py:71-87, reads the same
    rows), written once per decode step for DecodeAttention's ``rope`` argument.
    pos: [B] int32; cos/sin: [rows, d] bf16; out: [B, 2, d] bf16."""
    _check(pos, "pos", torch.int32)
    _need(pos.dim() == 1, "pos must be [B]")
    B = pos.shape[0]
    _check(cos, "cos", BF16)
    _check(sin, "sin", BF16)
    _need(cos.dim() == 2 and tuple(sin.shape) == tuple(cos.shape), "cos/sin must be [rows, d]")
    d = cos.shape[1]
    _check(out, "out", BF16, (B, 2, d))
    _lib.call("ko_rope_rows", _lib.ptr(pos), _lib.ptr(cos), _lib.ptr(sin), cos.shape[0], d, B,
              _lib.ptr(out), _lib.stream_ptr())


# ---------------------------------------------------------------------------
# Residual add + RMSNorm (fused.py:16-46).
# ---------------------------------------------------------------------------
def add_rms_norm(res, delta, weight, out, eps):
    """out = rmsnorm(res + delta); res <- res + delta (bf16). Rows contiguous [M, N],
    N a multiple of 8 and at most 8192."""
    n_rows, n_cols = res.shape
    _check(res, "res", BF16)
    if delta is not None:
        _check(delta, "delta", BF16, (n_rows, n_cols))
    _check(weight, "weight", BF16, (n_cols,))
    _check(out, "out", BF16, (n_rows, n_cols))
    _lib.call("ko_add_rms_norm", _lib.ptr(res), _lib.ptr(delta), _lib.ptr(weight), _lib.ptr(out),
              n_rows, n_cols, eps, _lib.stream_ptr())


# ---------------------------------------------------------------------------
# Per-head q/k RMSNorm + RoPE, writing K/V straight into the cache (fused.py:49-106).
# ---------------------------------------------------------------------------
def qk_norm_rope(qkv, q_w, k_w, cos, sin, pos, q_out, k_cache, v_cache, T, eps, nq, nkv, d):
    """qkv: [M, (nq+2nkv)*d] bf16 with M = B*T rows (row m is batch m//T at position
    pos[b] + m%T); k_cache/v_cache: one layer, [B, nkv, cap, d]."""
    M = qkv.shape[0]
    _need(M % T == 0, "rows must be B*T")
    B = M // T
    _check(qkv, "qkv", BF16, (M, (nq + 2 * nkv) * d))
    _check(q_out, "q_out", BF16, (M, nq * d))
    _check(q_w, "q_w", BF16, (d,))
    _check(k_w, "k_w", BF16, (d,))
    _check(cos, "cos", BF16)
    _check(sin, "sin", BF16)
    _check(pos, "pos", torch.int32, (B,))
    _check_cache(k_cache, "k_cache", B, nkv, k_cache.shape[2], d)
    _check_cache(v_cache, "v_cache", B, nkv, k_cache.shape[2], d)
    _need(k_cache.stride() == v_cache.stride(), "k_cache and v_cache must share strides")
    _lib.call("ko_qk_norm_rope", _lib.ptr(qkv), _lib.ptr(q_w), _lib.ptr(k_w), _lib.ptr(cos),
              _lib.ptr(sin), _lib.ptr(pos), _lib.ptr(q_out), _lib.ptr(k_cache), _lib.ptr(v_cache),
              M, T, k_cache.stride(0), k_cache.stride(1), eps, nq, nkv, d,
              min(k_cache.shape[2], cos.shape[0], sin.shape[0]), _lib.stream_ptr())


# ---------------------------------------------------------------------------
# SwiGLU: out = bf16(bf16(silu(gate)) * up), gate/up as [M, 2*I] (fused.py:109-127).
# ---------------------------------------------------------------------------
def silu_mul(gu, out):
    M, two_i = gu.shape
    I = two_i // 2
    _check(gu, "gu", BF16, (M, 2 * I))
    _check(out, "out", BF16, (M, I))
    _lib.call("ko_silu_mul", _lib.ptr(gu), _lib.ptr(out), M, I, _lib.stream_ptr())
