"""CPU oracle for the fused decode ops (test infrastructure only).

Every function restates the cast chain of the reference kernel it cites, in
fp32 on the CPU: ``bf(x)`` is ".to(bfloat16).to(float32)", the round trip the
reference writes as ``.to(tl.bfloat16).to(tl.float32)``.
"""

import torch

F32 = torch.float32
BF16 = torch.bfloat16


def bf(x):
    """Round fp32 to bf16 (round-to-nearest-even) and widen back to fp32."""
    return x.to(BF16).to(F32)


def add_rms_norm(res, delta, weight, eps):
    """engine/kernels/fused.py:16-36. Returns (new_res bf16, out bf16).

    res <- bf16(res + delta) when delta is given (fused.py:26-30);
    out = bf16(w * bf16(x * rsqrt(mean(x^2) + eps))) (fused.py:31-35).
    """
    x = res.to(F32)
    if delta is not None:
        x = bf(x + delta.to(F32))
    var = (x * x).sum(-1, keepdim=True) / x.shape[-1]
    normed = bf(x * torch.rsqrt(var + eps))
    y = (weight.to(F32) * normed).to(BF16)
    return x.to(BF16), y


def rope_tables(n, d=128, theta=1.0e6):
    """cos/sin [n, d] bf16 as Qwen3RotaryEmbedding builds them (engine.py:164-171 ->
    modeling_qwen3.py:116-137): inv_freq = 1/theta^(2i/d), freqs = inv_freq*pos in
    fp32, emb = cat(freqs, freqs), cos/sin in fp32, rounded to bf16."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.int64).to(F32) / d))
    pos = torch.arange(n, dtype=torch.int64).to(F32)
    freqs = pos[:, None] * inv_freq[None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(BF16), emb.sin().to(BF16)


def _norm_rope_head(x, w, cos_row, sin_row, eps):
    """One head (fp32 [..., D]) of fused.py:71-87: per-head RMSNorm then RoPE."""
    D = x.shape[-1]
    half = D // 2
    rstd = torch.rsqrt((x * x).sum(-1, keepdim=True) / D + eps)
    xn = bf(w.to(F32) * bf(x * rstd))                     # fused.py:80
    rh = torch.cat((-xn[..., half:], xn[..., :half]), -1)  # fused.py:82 (rotate_half)
    a = bf(xn * cos_row.to(F32))                           # fused.py:85
    b = bf(rh * sin_row.to(F32))                           # fused.py:86
    return (a + b).to(BF16)                                # fused.py:87


def qk_norm_rope(qkv, q_w, k_w, cos, sin, pos, k_cache, v_cache, T, eps, nq, nkv, d):
    """engine/kernels/fused.py:54-96 on bf16 qkv [M, (nq+2nkv)*d], M = B*T.

    Row m is batch m//T at position pos[b] + m%T. Returns q_out [M, nq*d] bf16 and
    writes k (normed + roped) and v (raw) into k_cache/v_cache[b, h, pos] in place.
    """
    M = qkv.shape[0]
    x = qkv.to(F32).view(M, nq + 2 * nkv, d)
    q_out = torch.empty(M, nq * d, dtype=BF16)
    for m in range(M):
        b, p = m // T, int(pos[m // T]) + m % T
        q_out[m] = _norm_rope_head(x[m, :nq], q_w, cos[p], sin[p], eps).reshape(-1)
        k_cache[b, :, p] = _norm_rope_head(x[m, nq:nq + nkv], k_w, cos[p], sin[p], eps)
        v_cache[b, :, p] = qkv[m].view(nq + 2 * nkv, d)[nq + nkv:]
    return q_out


def qk_norm_rope_acc(acc, q_w, k_w, cos, sin, pos, k_cache, v_cache, eps, nq, nkv, d):
    """engine/kernels/gemv.py:219-268 (T=1): round the fp32 QKV accumulator to bf16
    (gemv.py:240-241), then the same norm/RoPE/append as fused.py. The reference also
    re-zeroes ``acc`` and the sum-of-squares buffer (gemv.py:242,266-268); callers
    check that separately."""
    return qk_norm_rope(acc.to(BF16), q_w, k_w, cos, sin, pos, k_cache, v_cache, 1, eps,
                        nq, nkv, d)


def silu_mul(gu):
    """engine/kernels/fused.py:112-120: gu [M, 2I] (gate | up) -> bf16(bf16(silu(g)) * u)."""
    I = gu.shape[1] // 2
    g = gu[:, :I].to(F32)
    u = gu[:, I:].to(F32)
    s = bf(g / (1.0 + torch.exp(-g)))
    return (s * u).to(BF16)


EPI_F32, EPI_BF16, EPI_RESID, EPI_SWIGLU = 0, 1, 2, 3


def gemv(x, w, epi, nw=None, ss=None, h=None, eps=1e-6):
    """engine/kernels/gemv.py:30-106, y = x @ W^T with fp32 accumulation.

    NORM prologue when ``nw`` is given: x <- bf16(nw * bf16(x * rsqrt(ss/K + eps)))
    with ss[m] the row's sum of squares (gemv.py:67-79).
    Epilogues (gemv.py:86-106):
      EPI_F32    -> fp32 y
      EPI_BF16   -> bf16(y)
      EPI_RESID  -> returns (h_new = bf16(h + bf16(y)), ss_out = sum(h_new^2))
      EPI_SWIGLU -> w is [2N, K] (gate | up); bf16(bf16(silu(bf16 g)) * bf16 u)
    """
    xf = x.to(F32)
    K = xf.shape[1]
    if nw is not None:
        rstd = torch.rsqrt(ss.to(F32)[:, None] / K + eps)
        xf = bf(nw.to(F32)[None, :] * bf(xf * rstd))
    wf = w.to(F32)
    if epi == EPI_SWIGLU:
        N = w.shape[0] // 2
        g = bf(xf @ wf[:N].T)
        u = bf(xf @ wf[N:].T)
        s = bf(g / (1.0 + torch.exp(-g)))
        return (s * u).to(BF16)
    y = xf @ wf.T
    if epi == EPI_F32:
        return y
    if epi == EPI_BF16:
        return y.to(BF16)
    if epi == EPI_RESID:
        hn = (h.to(F32) + bf(y)).to(BF16)
        hf = hn.to(F32)
        return hn, (hf * hf).sum(-1)
    raise ValueError(f"unknown epilogue {epi}")


def embed_ss(ids, emb):
    """engine/kernels/gemv.py:201-211: h[m] = emb[ids[m]], ss[m] = sum(h[m]^2) fp32."""
    h = emb[ids.long()]
    hf = h.to(F32)
    return h, (hf * hf).sum(-1)


def argmax_first(logits):
    """torch.argmax over the last dim with the lowest index on exact ties
    (engine.py:291; OPTIMIZATION_GUIDE.md:213)."""
    lf = logits.to(F32)
    mx = lf.max(dim=-1, keepdim=True).values
    idx = torch.arange(lf.shape[-1]).expand_as(lf)
    big = torch.full_like(idx, lf.shape[-1])
    return torch.where(lf == mx, idx, big).min(dim=-1).values
