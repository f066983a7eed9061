"""Prompt forward (prefill) on PyTorch-ROCm ops, writing the static KV cache.

The reference's prefill (engine/engine.py:343-386) exists to produce exactly
the K/V and last-position logits of Transformers' own Qwen3 forward: a prefill
that drifts a little per layer can flip which key a sharp attention row picks
and cost whole logits downstream (engine.py:344-351). So this one is built
from the same torch operations, in the same order and with the same shapes, as
Transformers' modules (modeling_qwen3.py Qwen3RMSNorm, Qwen3Attention,
Qwen3MLP, Qwen3DecoderLayer):
- separate q / k / v and gate / up GEMMs (row slices of the engine's
  concatenated weights are the same matrices, so the same GEMM shapes);
- RMSNorm, per-head q/k RMSNorm, RoPE, SiLU-multiply and the residual adds as
  the modules write them (fp32 statistics, bf16 rounding before the gain);
- attention = torch's scaled_dot_product_attention, causal, on the modules'
  [B, heads, S, d] layouts, with ``enable_gqa`` only where a probe shows it
  bit-equal to repeated KV heads on this torch (engine.py:96-116), else on
  repeated KV heads; restricted to the fused SDPA kernels (a flash or
  memory-efficient backend), never the bf16 batched-matmul math path;
- the final RMSNorm and the LM head on the last position only (engine.py:383-385).
The prompt's K (normed + roped) and V go to cache slots 0..S-1.
"""

import torch
import torch.nn.functional as F

BF16 = torch.bfloat16
F32 = torch.float32

_GQA_EXACT = {}


def _sdpa_kernels():
    """Context restricting SDPA to its fused GPU kernels."""
    from torch.nn.attention import SDPBackend, sdpa_kernel
    return sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION])


def gqa_exact(device):
    """Whether SDPA with enable_gqa (the KV heads read in place) returns the same
    bits as SDPA on KV heads repeated 4x on causal prefill-shaped inputs, on this
    device and torch (the reference's probe, engine.py:96-116). Cached per device."""
    key = str(device)
    if key not in _GQA_EXACT:
        ok = True
        try:
            g = torch.Generator(device=device).manual_seed(0)
            with _sdpa_kernels():
                for B, S in ((1, 300), (4, 1024)):
                    q = torch.randn(B, 32, S, 128, device=device, dtype=BF16, generator=g)
                    k = torch.randn(B, 8, S, 128, device=device, dtype=BF16, generator=g) * 4
                    v = torch.randn(B, 8, S, 128, device=device, dtype=BF16, generator=g)
                    ref = F.scaled_dot_product_attention(q, k.repeat_interleave(4, 1),
                                                         v.repeat_interleave(4, 1), is_causal=True,
                                                         scale=128 ** -0.5)
                    got = F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=128 ** -0.5,
                                                         enable_gqa=True)
                    ok = ok and torch.equal(ref, got)
        except RuntimeError:
            ok = False
        _GQA_EXACT[key] = ok
    return _GQA_EXACT[key]


def rmsnorm(x, w, eps):
    """Qwen3RMSNorm.forward."""
    xf = x.to(F32)
    variance = xf.pow(2).mean(-1, keepdim=True)
    xf = xf * torch.rsqrt(variance + eps)
    return w * xf.to(x.dtype)


def rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def causal_attention(q, k, v, scale, exact_gqa):
    """q [B, nq, S, d], k/v [B, nkv, S, d] bf16 -> [B, nq, S, d] bf16, causal, by
    torch SDPA on its fused kernels."""
    rep = q.shape[1] // k.shape[1]
    with _sdpa_kernels():
        if exact_gqa:
            return F.scaled_dot_product_attention(q, k, v, attn_mask=None, dropout_p=0.0,
                                                  scale=scale, is_causal=True, enable_gqa=True)
        kr = k[:, :, None].expand(-1, -1, rep, -1, -1).reshape(k.shape[0], -1, *k.shape[2:])
        vr = v[:, :, None].expand(-1, -1, rep, -1, -1).reshape(v.shape[0], -1, *v.shape[2:])
        return F.scaled_dot_product_attention(q, kr, vr, attn_mask=None, dropout_p=0.0,
                                              scale=scale, is_causal=True)


@torch.no_grad()
def prefill(cfg, w, prompt, k_cache, v_cache, cos, sin):
    """prompt [B, S] int64 on the device; caches [L, B, nkv, cap, d]; cos/sin
    [>= S, d] bf16 (Qwen3RotaryEmbedding's rows for positions 0..S-1). Returns
    the greedy next ids [B] (int64) and the last-position logits [B, V] (bf16)."""
    B, S = prompt.shape
    nq, nkv, d, I, eps = cfg.nq, cfg.nkv, cfg.head_dim, cfg.inter, cfg.eps
    exact_gqa = gqa_exact(prompt.device)
    x = F.embedding(prompt, w["embed"])
    c = cos[:S][None, None]          # apply_rotary_pos_emb's unsqueeze(1)
    s_ = sin[:S][None, None]
    shape = (B, S, -1, d)
    for i, lw in enumerate(w["layers"]):
        residual = x
        h = rmsnorm(x, lw["w_in"], eps)
        qkv = lw["qkv"]
        q = rmsnorm(F.linear(h, qkv[:nq * d]).view(shape), lw["q_norm"], eps).transpose(1, 2)
        k = rmsnorm(F.linear(h, qkv[nq * d:(nq + nkv) * d]).view(shape), lw["k_norm"],
                    eps).transpose(1, 2)
        v = F.linear(h, qkv[(nq + nkv) * d:]).view(shape).transpose(1, 2)
        q = (q * c) + (rotate_half(q) * s_)
        k = (k * c) + (rotate_half(k) * s_)
        k_cache[i, :, :, :S] = k
        v_cache[i, :, :, :S] = v
        o = causal_attention(q, k, v, d ** -0.5, exact_gqa)
        o = o.transpose(1, 2).reshape(B, S, -1).contiguous()
        x = residual + F.linear(o, lw["o"])
        residual = x
        h = rmsnorm(x, lw["w_post"], eps)
        gu = lw["gu"]
        x = residual + F.linear(F.silu(F.linear(h, gu[:I])) * F.linear(h, gu[I:]), lw["down"])
    xl = rmsnorm(x[:, -1:], w["final_norm"], eps)
    logits = F.linear(xl, w["lm_head"])[:, -1]
    return torch.argmax(logits, dim=-1), logits
