"""Prompt forward (prefill) on PyTorch-ROCm ops, writing the static KV cache.

Follows the reference's prefill (engine/engine.py:343-386): the same operation
order and bf16 cast placement as Transformers' Qwen3 forward, hipBLASLt GEMMs
for the projections, causal GQA attention, the prompt's K/V written into
cache slots 0..S-1, greedy id of the last position, positions set to S.

Attention runs in fp32 from the bf16 q/k/v (one sequence at a time, contiguous
operands), then rounds to bf16; it stays off the bf16 batched-matmul path.
"""

import torch
import torch.nn.functional as F

BF16 = torch.bfloat16
F32 = torch.float32


def rmsnorm(x, w, eps):
    xf = x.to(F32)
    return w * (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype)


def rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def causal_gqa_fp32(q, k, v, scale):
    """q [nq, S, d], k/v [nkv, S, d] bf16 -> [nq, S, d] bf16, causal."""
    nq, S, d = q.shape
    grp = nq // k.shape[0]
    kf = k.to(F32).repeat_interleave(grp, 0)
    vf = v.to(F32).repeat_interleave(grp, 0)
    s = torch.matmul(q.to(F32), kf.transpose(1, 2).contiguous()) * scale
    mask = torch.ones(S, S, dtype=torch.bool, device=q.device).triu_(1)
    s.masked_fill_(mask, float("-inf"))
    return torch.matmul(torch.softmax(s, dim=-1), vf).to(BF16)


@torch.no_grad()
def prefill(cfg, w, prompt, k_cache, v_cache, cos, sin):
    """prompt [B, S] int64 on the device; caches [L, B, nkv, cap, d]. Returns the
    greedy next ids [B] (int64) and the last-position logits [B, V] (bf16)."""
    B, S = prompt.shape
    nq, nkv, d, I, eps = cfg.nq, cfg.nkv, cfg.head_dim, cfg.inter, cfg.eps
    x = F.embedding(prompt, w["embed"])
    c = cos[:S][None, None]
    s_ = sin[:S][None, None]
    for i, lw in enumerate(w["layers"]):
        res = x
        hn = rmsnorm(x, lw["w_in"], eps)
        qkv = lw["qkv"]
        q = F.linear(hn, qkv[:nq * d]).view(B, S, nq, d)
        k = F.linear(hn, qkv[nq * d:(nq + nkv) * d]).view(B, S, nkv, d)
        v = F.linear(hn, qkv[(nq + nkv) * d:]).view(B, S, nkv, d)
        q = rmsnorm(q, lw["q_norm"], eps).transpose(1, 2)
        k = rmsnorm(k, lw["k_norm"], eps).transpose(1, 2)
        v = v.transpose(1, 2)
        q = (q * c) + (rotate_half(q) * s_)
        k = (k * c) + (rotate_half(k) * s_)
        k_cache[i, :, :, :S] = k
        v_cache[i, :, :, :S] = v
        o = torch.empty(B, nq, S, d, dtype=BF16, device=x.device)
        for b in range(B):
            o[b] = causal_gqa_fp32(q[b], k[b], v[b], d ** -0.5)
        o = o.transpose(1, 2).reshape(B, S, nq * d)
        x = res + F.linear(o, lw["o"])
        res = x
        hn = rmsnorm(x, lw["w_post"], eps)
        gu = lw["gu"]
        x = res + F.linear(F.silu(F.linear(hn, gu[:I])) * F.linear(hn, gu[I:]), lw["down"])
    xl = rmsnorm(x[:, -1], w["final_norm"], eps)
    logits = F.linear(xl, w["lm_head"])
    return torch.argmax(logits, dim=-1), logits
