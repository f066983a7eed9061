"""Qwen3 eager forward restated in PyTorch (test infrastructure only).

This is the "reference eager path" of the decode engine: the operation order
and bf16 cast placement of Transformers' Qwen3 (modeling_qwen3.py
Qwen3RMSNorm / Qwen3Attention / Qwen3MLP / Qwen3DecoderLayer, the semantics
the reference engine keeps: engine/engine.py:274-292 and OPTIMIZATION_GUIDE.md
:395-410), over a static KV cache [L, B, nkv, cap, d]. Linear layers are bf16
F.linear; RMSNorm reduces in fp32 and rounds before the gain; attention is
computed in fp32 from the bf16 q/k/v and rounded to bf16.

Weights use the decode layout of kernel_optim_amd.model (qkv and gate|up
concatenated). Runs on any device (fp32 attention keeps it off the bf16
batched-matmul path).
"""

import torch
import torch.nn.functional as F

from .ops import rope_tables

BF16 = torch.bfloat16
F32 = torch.float32


def rmsnorm(x, w, eps):
    """Qwen3RMSNorm.forward: w * bf16(x * rsqrt(mean(x^2) + eps))."""
    xf = x.to(F32)
    var = xf.pow(2).mean(-1, keepdim=True)
    return w * (xf * torch.rsqrt(var + eps)).to(x.dtype)


def rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def attention_fp32(q, k, v, start, scale):
    """q [B, nq, T, d] at positions start..start+T-1; k/v [B, nkv, start+T, d].
    Causal: query t sees keys 0..start+t. Returns bf16 [B, nq, T, d]."""
    B, nq, T, d = q.shape
    nkv = k.shape[1]
    grp = nq // nkv
    kf = k.to(F32).repeat_interleave(grp, 1)
    vf = v.to(F32).repeat_interleave(grp, 1)
    s = torch.matmul(q.to(F32), kf.transpose(-1, -2).contiguous()) * scale    # [B, nq, T, L]
    L = k.shape[2]
    keys = torch.arange(L, device=q.device)
    lim = start + torch.arange(T, device=q.device)
    s = s.masked_fill(keys[None, :] > lim[:, None], float("-inf"))
    p = torch.softmax(s, dim=-1)
    return torch.matmul(p, vf).to(BF16)


class Qwen3Oracle:
    """Eager Qwen3 with a static cache. ``forward(ids, start)`` consumes T tokens per
    sequence at positions start..start+T-1 and returns bf16 logits [B, T, V]."""

    def __init__(self, cfg, weights, B, cap, device="cpu"):
        self.cfg, self.w, self.device = cfg, weights, torch.device(device)
        L, d = cfg.layers, cfg.head_dim
        self.k = torch.zeros(L, B, cfg.nkv, cap, d, dtype=BF16, device=device)
        self.v = torch.zeros_like(self.k)
        self.cos, self.sin = (t.to(device) for t in rope_tables(cap, d, cfg.theta))

    @torch.no_grad()
    def forward(self, ids, start, hidden=False):
        """bf16 logits [B, T, V]; with ``hidden`` the residual stream after the last
        layer instead (before the final norm), [B, T, H]."""
        cfg, w = self.cfg, self.w
        B, T = ids.shape
        nq, nkv, d, I = cfg.nq, cfg.nkv, cfg.head_dim, cfg.inter
        x = F.embedding(ids.to(self.device), w["embed"])
        cos = self.cos[start:start + T][None, None]
        sin = self.sin[start:start + T][None, None]
        for i, lw in enumerate(w["layers"]):
            res = x
            hn = rmsnorm(x, lw["w_in"], cfg.eps)
            qkv = lw["qkv"]
            q = F.linear(hn, qkv[:nq * d]).view(B, T, nq, d)
            k = F.linear(hn, qkv[nq * d:(nq + nkv) * d]).view(B, T, nkv, d)
            v = F.linear(hn, qkv[(nq + nkv) * d:]).view(B, T, nkv, d)
            q = rmsnorm(q, lw["q_norm"], cfg.eps).transpose(1, 2)
            k = rmsnorm(k, lw["k_norm"], cfg.eps).transpose(1, 2)
            v = v.transpose(1, 2)
            q = (q * cos) + (rotate_half(q) * sin)
            k = (k * cos) + (rotate_half(k) * sin)
            self.k[i, :, :, start:start + T] = k
            self.v[i, :, :, start:start + T] = v
            o = attention_fp32(q, self.k[i, :, :, :start + T], self.v[i, :, :, :start + T], start,
                               d ** -0.5)
            o = o.transpose(1, 2).reshape(B, T, nq * d)
            x = res + F.linear(o, lw["o"])
            res = x
            hn = rmsnorm(x, lw["w_post"], cfg.eps)
            gu = lw["gu"]
            mlp = F.linear(F.silu(F.linear(hn, gu[:I])) * F.linear(hn, gu[I:]), lw["down"])
            x = res + mlp
        if hidden:
            return x
        x = rmsnorm(x, w["final_norm"], cfg.eps)
        return F.linear(x, w["lm_head"])

    def greedy(self, prompt, n_new):
        """Greedy decode: returns (tokens [B, n_new], per-step logits list of [B, V])."""
        S = prompt.shape[1]
        logits = self.forward(prompt, 0)[:, -1]
        toks, steps = [], [logits]
        tok = logits.float().argmax(-1)
        toks.append(tok)
        for j in range(1, n_new):
            logits = self.forward(tok[:, None], S + j - 1)[:, -1]
            steps.append(logits)
            tok = logits.float().argmax(-1)
            toks.append(tok)
        return torch.stack(toks, 1), steps

    def teacher_forced_decode(self, prompt, tokens):
        """Decode-shaped replay of a given token sequence: the prompt in one forward,
        then each of tokens[:, :-1] at its own position, one forward per token (the
        shapes of Transformers' generate with a KV cache). Returns the logits at the
        n generated positions, [B, n, V], on the CPU."""
        S = prompt.shape[1]
        out = [self.forward(prompt, 0)[:, -1].cpu()]
        for j in range(1, tokens.shape[1]):
            out.append(self.forward(tokens[:, j - 1:j], S + j - 1)[:, -1].cpu())
        return torch.stack(out, 1)

    def teacher_forced(self, prompt, tokens):
        """Logits after the prompt and after each of tokens[:, :-1] (one forward
        over the whole sequence): [B, n, V] for the n generated positions."""
        seq = torch.cat([prompt, tokens[:, :-1]], 1)
        out = self.forward(seq, 0)
        return out[:, prompt.shape[1] - 1:]
