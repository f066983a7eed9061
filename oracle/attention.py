"""CPU oracle for split-K GQA decode attention (test infrastructure only).

decode_attention: closed form softmax(q K^T / sqrt(D)) V in fp64 with the
reference's causal rule for T query tokens (engine/kernels/fused.py:149-174:
query t of sequence b sees keys 0 .. pos[b]+t) and GQA head mapping h -> h//4
(OPTIMIZATION_GUIDE.md:100).

decode_attention_splitk: the reference's two-pass algorithm restated
(fused.py:138-201, split sizing fused.py:209-215): per (b, kv head, split)
online softmax over BLOCK_N tiles with m initialised to -1e30, P rounded to
bf16 before the PV product, fp32 partials (m, l, acc), then the LSE combine.
"""

import math

import torch


def decode_attention(q, k_cache, v_cache, kv_len, T=1, scale=None, dtype=torch.float64):
    """q: [B*T, NQ*D]; k/v_cache: [B, NKV, cap, D]; kv_len: [B] ints = valid keys.

    Query t (0..T-1) of sequence b sits at position kv_len[b]-T+t and sees keys
    0 .. kv_len[b]-T+t. Returns [B*T, NQ*D] in ``dtype``.
    """
    B, nkv, cap, D = k_cache.shape
    nq = q.shape[1] // D
    grp = nq // nkv
    scale = D ** -0.5 if scale is None else scale
    out = torch.zeros(B * T, nq * D, dtype=dtype)
    qf = q.to(dtype).view(B, T, nq, D)
    for b in range(B):
        L = int(kv_len[b])
        if L <= 0:
            continue
        k = k_cache[b, :, :L].to(dtype)        # [nkv, L, D]
        v = v_cache[b, :, :L].to(dtype)
        kr = k.repeat_interleave(grp, 0)       # [nq, L, D]
        vr = v.repeat_interleave(grp, 0)
        s = torch.einsum("thd,hld->thl", qf[b], kr) * scale   # [T, nq, L]
        keys = torch.arange(L)
        for t in range(T):
            lim = L - T + t                    # last visible key
            s[t, :, keys > lim] = -math.inf
        p = torch.softmax(s, dim=-1)
        o = torch.einsum("thl,hld->thd", p, vr)
        out.view(B, T, nq, D)[b] = o
    return out


def splitk_sizing(B, cap, nkv, target_ctas, block_n=64):
    """nsplit / chunk exactly as DecodeAttention.__init__ (fused.py:209-215)."""
    cdiv = lambda a, b: -(-a // b)
    max_split = max(1, cdiv(cap, 128))
    nsplit = max(1, min(max_split, cdiv(target_ctas, B * nkv)))
    chunk = cdiv(cdiv(cap, nsplit), block_n) * block_n
    return cdiv(cap, chunk), chunk


def decode_attention_splitk(q, k_cache, v_cache, pos, T=1, nsplit=None, chunk=None,
                            target_ctas=264, block_n=64):
    """Two-pass split-K flash-decoding, fused.py:138-201, on the CPU in fp32.

    pos[b] is the first query position (valid keys = pos[b]+T). Returns
    (out_bf16 [B*T, NQ*D], o_part, ml) with the reference's partial layout.
    """
    B, nkv, cap, D = k_cache.shape
    nq = q.shape[1] // D
    grp = nq // nkv
    if nsplit is None or chunk is None:
        nsplit, chunk = splitk_sizing(B, cap, nkv, target_ctas, block_n)
    scale = D ** -0.5
    rows = B * T * nq
    o_part = torch.zeros(rows * nsplit, D, dtype=torch.float32)
    ml = torch.zeros(rows * nsplit, 2, dtype=torch.float32)
    qv = q.view(B, T, nq, D)
    for b in range(B):
        p0 = int(pos[b])
        for kh in range(nkv):
            # rows r = (t, head) of this GQA group, fused.py:153-157
            heads = [kh * grp + i for i in range(grp)]
            qs = torch.stack([qv[b, t, h] for t in range(T) for h in heads]).float()  # [T*grp, D]
            limit = torch.tensor([p0 + t for t in range(T) for _ in heads])
            row_ids = [(b * T + t) * nq + h for t in range(T) for h in heads]
            for sp in range(nsplit):
                start = sp * chunk
                end = min(start + chunk, p0 + T)                       # fused.py:150-151
                m_i = torch.full((len(row_ids),), -1.0e30)             # fused.py:164
                l_i = torch.zeros(len(row_ids))
                acc = torch.zeros(len(row_ids), D)
                for s0 in range(start, end, block_n):                  # fused.py:168
                    idx = torch.arange(s0, min(s0 + block_n, end))
                    k = k_cache[b, kh, idx].float()
                    v = v_cache[b, kh, idx].float()
                    s = (qs @ k.T) * scale                             # fused.py:173
                    s = torch.where(idx[None, :] <= limit[:, None], s, torch.tensor(-math.inf))
                    m_new = torch.maximum(m_i, s.max(dim=1).values)    # fused.py:175
                    alpha = torch.exp(m_i - m_new)
                    p = torch.exp(s - m_new[:, None])
                    l_i = l_i * alpha + p.sum(dim=1)
                    acc = acc * alpha[:, None] + p.to(torch.bfloat16).float() @ v   # fused.py:179
                    m_i = m_new
                for i, row in enumerate(row_ids):
                    o_part[row * nsplit + sp] = acc[i]
                    ml[row * nsplit + sp, 0] = m_i[i]
                    ml[row * nsplit + sp, 1] = l_i[i]
    out = combine(o_part, ml, nsplit, rows, D).view(B * T, nq * D)
    return out, o_part, ml


def combine(o_part, ml, nsplit, rows, D):
    """LSE merge of split partials, fused.py:188-201. Returns bf16 [rows, D]."""
    o = o_part.view(rows, nsplit, D)
    m = ml.view(rows, nsplit, 2)[..., 0]
    l = ml.view(rows, nsplit, 2)[..., 1]
    M = m.max(dim=1, keepdim=True).values
    w = torch.exp(m - M)
    L = (w * l).sum(dim=1, keepdim=True)
    res = (o * w[..., None]).sum(dim=1) / L
    return res.to(torch.bfloat16)


def hbm_bytes(B, nkv, kv_lens, nq, D=128, T=1):
    """Algorithmic HBM bytes of one decode-attention call: K and V of every valid
    key once, q read once, out written once (bf16)."""
    kv = sum(int(x) for x in kv_lens) * nkv * D * 2 * 2
    return kv + 2 * B * T * nq * D * 2
