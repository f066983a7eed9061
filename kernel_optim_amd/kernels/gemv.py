"""Fused skinny GEMMs for the decode step on hand-written HIP kernels (gfx950).

Python surface of the reference's engine/kernels/gemv.py:
- ``EPI_F32, EPI_BF16, EPI_RESID, EPI_SWIGLU = 0, 1, 2, 3``        (gemv.py:27)
- ``Gemv(M, N, K, epi, norm, allow_split=False, eps=1e-6)``          (gemv.py:109-120)
  ``__call__(x, w, y=None, nw=None, ss=None, h=None, ss_out=None, cfg=None)``
                                                                    (gemv.py:140-150)
  ``candidates()``, ``tune(weights, deadline)``                      (gemv.py:122-195)
- ``embed_ss(ids, emb, h, ss)``                                      (gemv.py:214-216)
- ``qk_norm_rope_acc(acc, q_w, k_w, cos, sin, pos, q_out, k_cache, v_cache,
  zero_buf, eps, nq, nkv, d)``                                       (gemv.py:271-277)

Additions of this backend:
- ``EPI_ARGMAX = 4``: the LM head with greedy selection fused in; pass ``ids``
  ([M] int64) and optionally ``y`` for the bf16 logits.
- NORM with ``ss=None`` computes the row's sum of squares from x inside the
  kernel (no separate sum-of-squares buffer or zeroing discipline needed).

``cfg`` is an opaque tuple ``(layout, rows, waves)``: layout 0 gives each
256-thread workgroup ``rows`` output columns (any M); layout 1 gives each
wavefront ``rows`` columns with ``waves`` wavefronts per workgroup sharing the
normalised input through LDS (M <= 4); layouts 2, 3 and 4 put 2..16 rows on
MFMA tiles (layouts 2 and 4 with ``waves`` = 2: 32 rows, two row tiles sharing
each weight load; layout 4 with ``waves`` = 4: 64 rows) and read a tiled copy of the weights (``tile_weights``), layout 3 with
the K range of a tile cut into ``rows`` slices merged by the tile's last slice,
layout 4 with each tile cut into 16 K chunks dealt out 10 per workgroup and
merged by the tile's last workgroup (no atomics on the output in either, so the
F32 epilogue is a plain store).
``allow_split`` is accepted for signature compatibility.

Drop-in rule for the tiled layouts: the default configuration (``cfg`` before
``tune``) is always a row-major layout, ``tune(weights, deadline)`` makes the
tiled copies itself when it times a tiled candidate (and keeps them, keyed by
the row-major weight), and ``__call__`` maps a row-major weight to its copy
when the configuration needs one. A tiled configuration on a weight with no
copy, or a tiled copy under a row-major configuration, raises ValueError.
"""

import time
import weakref

import torch

from .. import _lib
from .fused import BF16, _cdiv, _check, _need

EPI_F32, EPI_BF16, EPI_RESID, EPI_SWIGLU, EPI_ARGMAX = 0, 1, 2, 3, 4


def uses_tiled(cfg):
    """Layouts 2, 3 and 4 (MFMA) read the tile_weights copy of the weights."""
    return cfg[0] in (2, 3, 4)


def is_tiled(w):
    """True for a tensor written by tile_weights (the MFMA-layout copy)."""
    return getattr(w, "_ko_tiled", False)


class Gemv:
    """One fused projection y[M, N] = x[M, K] @ W[N, K]^T with a norm prologue and
    an epilogue; its launch config is picked by GPU timing at setup."""

    def __init__(self, M, N, K, epi, norm, allow_split=False, eps=1e-6):
        _need(epi in (EPI_F32, EPI_BF16, EPI_RESID, EPI_SWIGLU, EPI_ARGMAX), f"bad epilogue {epi}")
        _need(K % 8 == 0, "K must be a multiple of 8")
        self.M, self.N, self.K, self.epi, self.norm, self.eps = M, N, K, epi, bool(norm), eps
        self.allow_split = allow_split
        self.cfg = self.candidates()[0]
        self._part = None
        self._tiles = {}   # id(row-major weight) -> (weakref to it, its tiled copy)
        self.us = float("nan")
        self.tune_log = []

    def mfma_ok(self):
        """Layout 2 (MFMA tiles, x rows padded to 16) takes K in {2560, 4096, 9728},
        SWIGLU only up to 4096 (gemv.hip, mfma_supported)."""
        return self.K in (2560, 4096) or (self.K == 9728 and self.epi != EPI_SWIGLU)

    def mfma2_ok(self):
        """Layout 2 with two row tiles (``waves`` = 2: 32 rows of x per weight
        pass) keeps both tiles of x in registers: K in {2560, 4096}, SWIGLU
        K = 2560 (gemv_launch.h, mfma_supported)."""
        return self.K == 2560 or (self.K == 4096 and self.epi != EPI_SWIGLU)

    def ks_slices(self):
        """K slices layout 3 takes for this projection (gemv.hip, ks_steps):
        K = 128 * S * slices with S in {20, 19, 8, 4}; NORM computes the row norms
        in one workgroup, so it takes one slice (K = 2560); no ARGMAX."""
        if self.epi == EPI_ARGMAX:
            return []
        out = []
        for s in (1, 2, 4, 8, 19):
            if self.K % (128 * s) == 0 and self.K // (128 * s) in (20, 19, 8, 4):
                out.append(s)
        return [s for s in out if s == 1 and self.K == 2560] if self.norm else out

    def sk_ok(self):
        """Layout 4 (MFMA tiles cut into 16 chunks of S steps, dealt out 10 per
        workgroup; gemv.hip, sk_steps): K = 512 * S with S in {19, 8, 5}, no NORM,
        F32, BF16 or RESID."""
        return (not self.norm and self.epi in (EPI_F32, EPI_BF16, EPI_RESID)
                and self.K % 512 == 0 and self.K // 512 in (19, 8, 5))

    def candidates(self):
        """Launch configurations, the default first. The default is always a
        row-major layout, so an untuned Gemv runs on the weights the caller holds.
        Layout 1 (a wavefront per row group) is the batch-1..4 path; layout 0
        serves every batch up to 16 rows per launch with VALU dot products;
        layout 2 puts 2..16 rows on MFMA (``(2, per_cu, 0)``: a persistent grid
        of at most 256 x per_cu workgroups, the fewest that keep the most tiles
        per workgroup at its minimum; ``(2, per_cu, 2)``: 32 rows per weight
        pass, offered above 16 rows), layout 3 splits its tiles' K range and
        layout 4 (``(4, 10, 0)``; ``(4, 10, 2)`` / ``(4, 10, 4)`` with 32 / 64
        rows) deals the tiles' 16 K chunks out 10 per workgroup."""
        out = []
        mfma = [(2, 2, 0), (2, 1, 0)] if self.M >= 2 and self.mfma_ok() else []
        mfma += [(2, 2, 2), (2, 1, 2)] if self.M > 16 and self.mfma2_ok() else []
        mfma += [(3, s, 0) for s in self.ks_slices()] if self.M >= 2 else []
        mfma += [(4, 10, 0)] if self.M >= 2 and self.sk_ok() else []
        mfma += [(4, 10, 2)] if self.M > 16 and self.sk_ok() else []
        mfma += [(4, 10, 4)] if self.M > 32 and self.sk_ok() else []
        if self.M <= 4 and (not self.norm or self.M * self.K * 2 <= 40960):
            per_wave = (4, 2, 1) if self.N >= 32768 else (1, 2, 4)
            for rows in per_wave:
                for waves in (2, 4):
                    out.append((1, rows, waves))
        out += [(0, 4, 0), (0, 8, 0)] if self.N < 32768 else [(0, 8, 0), (0, 4, 0)]
        if self.M <= 2 and self.N >= 32768:
            out.append((0, 16, 0))  # fewer ARGMAX partials
        return out + mfma

    def _scratch(self, device, cfg):
        """fp32 scratch of the ARGMAX partials or of layout 3's and 4's slots and
        arrival counters (allocated zeroed: the counters start at zero and every
        launch leaves them there)."""
        n = _lib.lib().ko_gemv_argmax_scratch(self.N, *cfg)
        if self._part is None or self._part.device != device or self._part.numel() < n:
            self._part = torch.zeros(max(n, 2), dtype=torch.float32, device=device)
        return self._part

    def _weight_for(self, w, cfg):
        """The weight tensor this configuration reads: ``w`` itself, or for a tiled
        layout the copy ``tune`` made of the row-major ``w``."""
        if uses_tiled(cfg):
            if is_tiled(w):
                return w
            ent = self._tiles.get(id(w))
            if ent is not None and ent[0]() is w:
                return ent[1]
            raise ValueError(f"cfg {cfg} reads MFMA-tiled weights, but this weight has no tiled "
                             "copy: pass tile_weights(w) or tune() with these weights")
        _need(not is_tiled(w), f"cfg {cfg} reads row-major weights, got a tile_weights copy")
        return w

    def _remember_tiles(self, weights, tiled):
        for w, t in zip(weights, tiled):
            if not is_tiled(w):
                self._tiles[id(w)] = (weakref.ref(w), t)

    def __call__(self, x, w, y=None, nw=None, ss=None, h=None, ss_out=None, cfg=None, ids=None,
                 pos_inc=None, next_emb=None, next_h=None, rope=None, ring=None):
        """ARGMAX extras: ``pos_inc`` ([M] int32) is advanced by one; with
        ``next_emb`` ([N, K] bf16, the embedding) the chosen ids' rows are gathered
        into ``next_h`` ([M, K] bf16), the next decode step's input. The decode
        step's tail (ko_lm_head_argmax): ``rope = (cos, sin, out)`` writes the
        RoPE rows of the advanced positions into out ([M, 2, d] bf16, what
        rope_rows writes), and ``ring = (host, ctr)`` stores the ids into row
        ctr[m] of host ([R, M] int64, pinned) and advances ctr ([M] int32 on the
        device) modulo R; ``ring = (host, ctr, err)`` stores -2 in place of the
        ids while err ([1] int32 on the device, DecodeAttention.err) is set."""
        M, N, K, epi = self.M, self.N, self.K, self.epi
        layout, rows, waves = cfg or self.cfg
        _check(x, "x", BF16, (M, K))
        w = self._weight_for(w, (layout, rows, waves))
        nrows = _cdiv(N, 16) * 16 if uses_tiled((layout,)) else N  # the tile_weights copy
        _check(w, "w", BF16, ((2 * nrows) if epi == EPI_SWIGLU else nrows, K))
        if self.norm:
            _check(nw, "nw", BF16, (K,))
            if ss is not None:
                _check(ss, "ss", torch.float32, (M,))
        if epi == EPI_F32:
            _check(y, "y", torch.float32, (M, N))
        elif epi in (EPI_BF16, EPI_SWIGLU):
            _check(y, "y", BF16, (M, N))
        elif epi == EPI_RESID:
            _check(h, "h", BF16, (M, N))
            if ss_out is not None:
                _check(ss_out, "ss_out", torch.float32, (M,))
        else:
            _check(ids, "ids", torch.int64, (M,))
            if y is not None:
                _check(y, "y", BF16, (M, N))
            if pos_inc is not None:
                _check(pos_inc, "pos_inc", torch.int32, (M,))
            _need((next_emb is None) == (next_h is None), "next_emb and next_h go together")
            if next_emb is not None:
                _check(next_emb, "next_emb", BF16, (N, K))
                _check(next_h, "next_h", BF16, (M, K))
            if rope is not None:
                cos, sin, rope_out = rope
                _need(pos_inc is not None, "rope rows need the positions (pos_inc)")
                _check(cos, "cos", BF16)
                _need(cos.dim() == 2 and tuple(sin.shape) == tuple(cos.shape),
                      "cos/sin must be [rows, d]")
                _check(sin, "sin", BF16)
                _check(rope_out, "rope", BF16, (M, 2, cos.shape[1]))
            if ring is not None:
                _need(len(ring) in (2, 3), "ring is (host, ctr) or (host, ctr, err)")
                host, ctr = ring[:2]
                _need(isinstance(host, torch.Tensor) and host.dtype == torch.int64
                      and not host.is_cuda and host.is_pinned() and host.is_contiguous()
                      and host.dim() == 2 and host.shape[1] == M,
                      "ring host must be a pinned contiguous int64 [R, M] CPU tensor")
                _check(ctr, "ring counter", torch.int32, (M,))
                if len(ring) == 3 and ring[2] is not None:
                    _check(ring[2], "ring err", torch.int32, (1,))
        part = (self._scratch(x.device, (layout, rows, waves))
                if epi == EPI_ARGMAX or (layout == 3 and rows > 1) or layout == 4 else None)
        if epi == EPI_ARGMAX and (rope is not None or ring is not None):
            cos, sin, rope_out = rope if rope is not None else (None, None, None)
            host, ctr, err = (tuple(ring) + (None,))[:3] if ring is not None else (None,) * 3
            _lib.call("ko_lm_head_argmax", _lib.ptr(x), _lib.ptr(w),
                      _lib.ptr(nw) if self.norm else None, _lib.ptr(ss) if self.norm else None,
                      _lib.ptr(y), _lib.ptr(ids), _lib.ptr(pos_inc), _lib.ptr(next_emb),
                      _lib.ptr(next_h), _lib.ptr(cos), _lib.ptr(sin),
                      0 if cos is None else cos.shape[0], 0 if cos is None else cos.shape[1],
                      _lib.ptr(rope_out),
                      None if host is None else _lib.host_device_ptr(host),
                      0 if host is None else host.shape[0],
                      _lib.ptr(ctr), _lib.ptr(err), _lib.ptr(part), part.numel(), M, N, K,
                      layout, rows, waves, self.eps, _lib.stream_ptr())
            return
        _lib.call("ko_gemv", _lib.ptr(x), _lib.ptr(w), _lib.ptr(y),
                  _lib.ptr(nw) if self.norm else None, _lib.ptr(ss) if self.norm else None,
                  _lib.ptr(h), _lib.ptr(ss_out), _lib.ptr(ids), _lib.ptr(pos_inc),
                  _lib.ptr(next_emb), _lib.ptr(next_h), _lib.ptr(part),
                  0 if part is None else part.numel(), M, N, K, epi, int(self.norm), 0, layout,
                  rows, waves, self.eps, _lib.stream_ptr())

    def tune(self, weights, deadline, tiled=None, rounds=3):
        """Pick the fastest candidate by GPU time: one call per layer weight (cold),
        captured in a graph and replayed twice (gemv.py:152-195). The candidates'
        graphs are captured first and timed in ``rounds`` interleaved rounds, each
        candidate keeping its best round, so drift and one-off noise do not decide
        the choice; a candidate replaces an earlier (default-first) one only when
        it is more than 1 % faster. Tiled (MFMA) candidates run on ``tiled`` (the
        tile_weights copies of ``weights``); without it, tune makes the copies
        itself (before the deadline) and keeps them, so a later call with a
        row-major weight of ``weights`` reads its copy. With the deadline passed
        nothing is timed and the configuration stays the row-major default."""
        dev = weights[0].device
        if any(uses_tiled(c) for c in self.candidates()):
            if tiled is None and time.monotonic() <= deadline:
                tiled = [tile_weights(w, swiglu=self.epi == EPI_SWIGLU) for w in weights]
            if tiled is not None:
                self._remember_tiles(weights, tiled)
        M, N, K = self.M, self.N, self.K
        x = torch.randn(M, K, device=dev, dtype=BF16)
        y = torch.zeros(M, N, device=dev, dtype=torch.float32 if self.epi == EPI_F32 else BF16)
        nw = torch.ones(K, device=dev, dtype=BF16)
        h = torch.zeros(M, N, device=dev, dtype=BF16)
        ids = torch.zeros(M, device=dev, dtype=torch.int64)
        kw = dict(y=y, nw=nw, h=h, ids=ids)
        # the scratch is sized for every candidate before any graph captures it:
        # the graphs are replayed after all captures
        for cfg in self.candidates():
            if ((self.epi == EPI_ARGMAX or cfg[0] in (3, 4))
                    and _lib.lib().ko_gemv_argmax_scratch(self.N, *cfg) > 0):
                self._scratch(dev, cfg)
        graphs = []
        for cfg in self.candidates():
            if time.monotonic() > deadline:
                break
            ws = tiled if uses_tiled(cfg) else weights
            if ws is None:
                continue
            try:
                self(x, ws[0], cfg=cfg, **kw)
                torch.cuda.synchronize()
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    for wt in ws:
                        self(x, wt, cfg=cfg, **kw)
                g.replay()
                torch.cuda.synchronize()
            except RuntimeError:
                torch.cuda.synchronize()
                continue
            graphs.append((cfg, g))
        cfgs = [c for c, _ in graphs]
        if not graphs:
            return self.cfg
        times = [float("inf")] * len(graphs)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        for _ in range(rounds):
            for i, (_, g) in enumerate(graphs):
                a.record()
                g.replay()
                g.replay()
                b.record()
                torch.cuda.synchronize()
                times[i] = min(times[i], a.elapsed_time(b))
        del graphs
        per_call = [t / (2 * len(weights)) * 1e3 for t in times]
        self.tune_log = [(c, round(u, 2)) for c, u in zip(cfgs, per_call)]
        best = None
        for c, u in zip(cfgs, per_call):
            if best is None or u < 0.99 * best[1]:
                best = (c, u)
        if best is not None:
            self.cfg, self.us = best
        return self.cfg


def tile_weights(w, swiglu=False):
    """The layout-2 (MFMA) copy of a row-major bf16 weight: [N, K] -> [ceil(N/16)*16, K]
    in the tiled order of ko_gemv_tile (one 1 KiB block per 16-row tile and 32-column
    step, in the MFMA B-operand lane order). For SWIGLU ([2N, K], gate | up) the gate
    and up halves are tiled separately. A one-time transform on the current stream."""
    _check(w, "w", BF16)
    _need(w.dim() == 2 and w.shape[1] % 32 == 0, "w must be [rows, K] with K % 32 == 0")
    R, K = w.shape
    halves = [w[: R // 2], w[R // 2:]] if swiglu else [w]
    if swiglu:
        _need(R % 2 == 0, "a SWIGLU weight has 2N rows")
    n = halves[0].shape[0]
    npad = _cdiv(n, 16) * 16
    out = torch.empty(npad * len(halves), K, dtype=BF16, device=w.device)
    for i, part in enumerate(halves):
        _lib.call("ko_gemv_tile", _lib.ptr(part), _lib.ptr(out[i * npad:(i + 1) * npad]), n, K,
                  _lib.stream_ptr())
    out._ko_tiled = True
    return out


def embed_ss(ids, emb, h, ss):
    """h[m] = emb[ids[m]]; ss[m] = sum(h[m]^2) (gemv.py:201-216). ss may be None."""
    M, H = h.shape
    _check(ids, "ids", torch.int64, (M,))
    _check(emb, "emb", BF16)
    _need(emb.dim() == 2 and emb.shape[1] == H, "emb must be [V, H]")
    _check(h, "h", BF16, (M, H))
    if ss is not None:
        _check(ss, "ss", torch.float32, (M,))
    _lib.call("ko_embed_ss", _lib.ptr(ids), _lib.ptr(emb), _lib.ptr(h), _lib.ptr(ss), M, H,
              emb.shape[0], _lib.stream_ptr())


def argmax_rows(x, ids):
    """ids[m] = argmax_n x[m, n] over bf16 logits [M, N], lowest index on ties:
    torch.argmax(logits, dim=-1, out=vout) of the verify step (engine.py:413-415),
    without the memset a multi-block torch reduction records in a graph."""
    _check(x, "x", BF16, contiguous=False)
    _need(x.dim() == 2 and x.stride(1) == 1, "x must be [M, N] with unit column stride")
    M, N = x.shape
    _check(ids, "ids", torch.int64, (M,))
    _lib.call("ko_argmax_rows", _lib.ptr(x), x.stride(0), M, N, _lib.ptr(ids), _lib.stream_ptr())


def qk_norm_rope_acc(acc, q_w, k_w, cos, sin, pos, q_out, k_cache, v_cache, zero_buf, eps, nq,
                     nkv, d):
    """Decode (T=1) q/k norm + RoPE from the fp32 QKV accumulator (gemv.py:219-277):
    rounds the projection to bf16, writes q and the K/V cache slot pos[b],
    re-zeroes the consumed accumulator and zeroes ``zero_buf``."""
    B = acc.shape[0]
    _check(acc, "acc", torch.float32, (B, (nq + 2 * nkv) * d))
    _check(q_out, "q_out", BF16, (B, nq * d))
    _check(pos, "pos", torch.int32, (B,))
    _check(q_w, "q_w", BF16, (d,))
    _check(k_w, "k_w", BF16, (d,))
    _check(cos, "cos", BF16)
    _check(sin, "sin", BF16)
    _need(k_cache.shape[0] == B and k_cache.stride(3) == 1 and k_cache.stride(2) == d,
          "k_cache must be [B, nkv, cap, d] with sequence stride d")
    _need(k_cache.stride() == v_cache.stride(), "k_cache and v_cache must share strides")
    if zero_buf is not None:
        _check(zero_buf, "zero_buf", torch.float32)
    _lib.call("ko_qk_norm_rope_acc", _lib.ptr(acc), _lib.ptr(q_w), _lib.ptr(k_w), _lib.ptr(cos),
              _lib.ptr(sin), _lib.ptr(pos), _lib.ptr(q_out), _lib.ptr(k_cache),
              _lib.ptr(v_cache), _lib.ptr(zero_buf),
              0 if zero_buf is None else zero_buf.numel(), B, k_cache.stride(0),
              k_cache.stride(1), eps, nq, nkv, d, min(k_cache.shape[2], cos.shape[0], sin.shape[0]),
              _lib.stream_ptr())
