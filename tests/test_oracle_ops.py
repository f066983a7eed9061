"""Pins the fused-op oracle (CPU) against the Transformers Qwen3 modules and torch
library routines that the reference's kernels reproduce
(engine/kernels/fused.py, engine/kernels/gemv.py)."""

import pytest
import torch
import torch.nn.functional as F
from transformers import Qwen3Config
from transformers.models.qwen3 import modeling_qwen3 as MQ

from oracle import ops as O
from tests.bf16util import assert_bf16_close

BF = torch.bfloat16


def cfg(theta=1.0e6):
    return Qwen3Config(hidden_size=2560, intermediate_size=9728, num_hidden_layers=1,
                       num_attention_heads=32, num_key_value_heads=8, head_dim=128,
                       rms_norm_eps=1e-6, rope_theta=theta, vocab_size=151936,
                       max_position_embeddings=40960)


def test_rmsnorm_matches_qwen3_module():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(4, 2560, generator=g).to(BF)
    w = (1 + 0.1 * torch.randn(2560, generator=g)).to(BF)
    mod = MQ.Qwen3RMSNorm(2560, eps=1e-6)
    mod.weight.data = w.clone()
    mod = mod.to(BF)
    want = mod(x)
    _, got = O.add_rms_norm(x, None, w, 1e-6)
    assert_bf16_close(got, want)


def test_residual_add_then_norm_matches_decoder_layer_math():
    g = torch.Generator().manual_seed(1)
    res = torch.randn(3, 2560, generator=g).to(BF)
    delta = torch.randn(3, 2560, generator=g).to(BF)
    w = torch.randn(2560, generator=g).to(BF)
    new_res, out = O.add_rms_norm(res, delta, w, 1e-6)
    assert torch.equal(new_res, res + delta)           # residual + hidden in bf16
    mod = MQ.Qwen3RMSNorm(2560, eps=1e-6)
    mod.weight.data = w.clone()
    assert_bf16_close(out, mod.to(BF)(res + delta))


@pytest.mark.parametrize("theta", [1.0e6, 5.0e6])
def test_rope_tables_match_rotary_module(theta):
    rot = MQ.Qwen3RotaryEmbedding(cfg(theta))
    n = 3000
    x = torch.empty(1, dtype=BF)
    cos, sin = rot(x, torch.arange(n).unsqueeze(0))
    c, s = O.rope_tables(n, 128, theta)
    assert torch.equal(c, cos[0]) and torch.equal(s, sin[0])


@pytest.mark.parametrize("theta", [1.0e6, 5.0e6])
def test_engine_rope_tables_match_rotary_module(theta):
    """The engine's tables (computed with the module's recipe, here on the CPU)
    equal Qwen3RotaryEmbedding's forward bit for bit."""
    from kernel_optim_amd.engine import _rope_tables
    rot = MQ.Qwen3RotaryEmbedding(cfg(theta))
    n = 3000
    cos, sin = rot(torch.empty(1, dtype=BF), torch.arange(n).unsqueeze(0))
    c, s = _rope_tables(n, 128, theta, "cpu")
    assert torch.equal(c, cos[0]) and torch.equal(s, sin[0])


@pytest.mark.parametrize("T", [1, 3])
def test_qk_norm_rope_matches_hf_attention_prologue(T):
    B, nq, nkv, d, cap = 2, 32, 8, 128, 64
    g = torch.Generator().manual_seed(2 + T)
    qkv = torch.randn(B * T, (nq + 2 * nkv) * d, generator=g).to(BF)
    qw = (1 + 0.2 * torch.randn(d, generator=g)).to(BF)
    kw = (1 + 0.2 * torch.randn(d, generator=g)).to(BF)
    pos = torch.tensor([5, 60 - T], dtype=torch.int32)
    cos, sin = O.rope_tables(cap, d, 1.0e6)
    kc = torch.zeros(B, nkv, cap, d, dtype=BF)
    vc = torch.zeros(B, nkv, cap, d, dtype=BF)
    q_out = O.qk_norm_rope(qkv, qw, kw, cos, sin, pos, kc, vc, T, 1e-6, nq, nkv, d)

    qn = MQ.Qwen3RMSNorm(d, eps=1e-6)
    qn.weight.data = qw.clone()
    kn = MQ.Qwen3RMSNorm(d, eps=1e-6)
    kn.weight.data = kw.clone()
    qn, kn = qn.to(BF), kn.to(BF)
    x = qkv.view(B, T, nq + 2 * nkv, d)
    for b in range(B):
        p = torch.arange(int(pos[b]), int(pos[b]) + T)
        qh = qn(x[b, :, :nq]).transpose(0, 1)[None]          # [1, nq, T, d]
        kh = kn(x[b, :, nq:nq + nkv]).transpose(0, 1)[None]  # [1, nkv, T, d]
        qe, ke = MQ.apply_rotary_pos_emb(qh, kh, cos[p][None], sin[p][None])
        assert_bf16_close(q_out.view(B, T, nq, d)[b], qe[0].transpose(0, 1))
        assert_bf16_close(kc[b, :, p], ke[0])
        assert torch.equal(vc[b, :, p], x[b, :, nq + nkv:].transpose(0, 1))
    # every other slot untouched
    mask = torch.ones(B, cap, dtype=torch.bool)
    for b in range(B):
        mask[b, int(pos[b]):int(pos[b]) + T] = False
    assert torch.all(kc.permute(0, 2, 1, 3)[mask] == 0)


def test_qk_norm_rope_acc_rounds_accumulator_first():
    B, nq, nkv, d, cap = 2, 32, 8, 128, 16
    g = torch.Generator().manual_seed(9)
    acc = torch.randn(B, (nq + 2 * nkv) * d, generator=g)
    qw = torch.ones(d, dtype=BF)
    kw = torch.ones(d, dtype=BF)
    cos, sin = O.rope_tables(cap)
    pos = torch.tensor([3, 7], dtype=torch.int32)
    k1, v1 = torch.zeros(B, nkv, cap, d, dtype=BF), torch.zeros(B, nkv, cap, d, dtype=BF)
    k2, v2 = k1.clone(), v1.clone()
    a = O.qk_norm_rope_acc(acc, qw, kw, cos, sin, pos, k1, v1, 1e-6, nq, nkv, d)
    b = O.qk_norm_rope(acc.to(BF), qw, kw, cos, sin, pos, k2, v2, 1, 1e-6, nq, nkv, d)
    assert torch.equal(a, b) and torch.equal(k1, k2) and torch.equal(v1, v2)


def test_silu_mul_matches_mlp_activation():
    g = torch.Generator().manual_seed(3)
    gu = (3 * torch.randn(5, 2 * 9728, generator=g)).to(BF)
    got = O.silu_mul(gu)
    want = F.silu(gu[:, :9728]) * gu[:, 9728:]
    assert_bf16_close(got, want)


def test_gemv_norm_prologue_and_epilogues_match_torch():
    g = torch.Generator().manual_seed(4)
    M, K, N = 3, 2560, 512
    x = torch.randn(M, K, generator=g).to(BF)
    nw = (1 + 0.1 * torch.randn(K, generator=g)).to(BF)
    W = (0.02 * torch.randn(2 * N, K, generator=g)).to(BF)
    ss = x.float().pow(2).sum(-1)
    mod = MQ.Qwen3RMSNorm(K, eps=1e-6)
    mod.weight.data = nw.clone()
    xn = mod.to(BF)(x)                                     # the reference's input_layernorm
    # F32 / BF16: a bf16 nn.Linear on the normed input
    y32 = O.gemv(x, W[:N], O.EPI_F32, nw=nw, ss=ss)
    torch.testing.assert_close(y32, xn.float() @ W[:N].float().T, rtol=1e-5, atol=1e-4)
    assert_bf16_close(O.gemv(x, W[:N], O.EPI_BF16, nw=nw, ss=ss), F.linear(xn, W[:N]), max_frac=0.02)
    # SWIGLU: Qwen3MLP's act(gate(x)) * up(x)
    want = F.silu(F.linear(xn, W[:N])) * F.linear(xn, W[N:])
    assert_bf16_close(O.gemv(x, W, O.EPI_SWIGLU, nw=nw, ss=ss), want, max_ulp=2, max_frac=0.03)
    # RESID: residual + o_proj(attn)
    h = torch.randn(M, N, generator=g).to(BF)
    a = torch.randn(M, K, generator=g).to(BF)
    hn, ss_out = O.gemv(a, W[:N], O.EPI_RESID, h=h)
    assert_bf16_close(hn, h + F.linear(a, W[:N]), max_frac=0.02)
    torch.testing.assert_close(ss_out, hn.float().pow(2).sum(-1))


def test_embed_ss_and_argmax():
    g = torch.Generator().manual_seed(5)
    emb = torch.randn(1000, 64, generator=g).to(BF)
    ids = torch.tensor([3, 999, 0])
    h, ss = O.embed_ss(ids, emb)
    assert torch.equal(h, F.embedding(ids, emb))
    torch.testing.assert_close(ss, h.float().pow(2).sum(-1))
    logits = torch.randn(4, 5000, generator=g).to(BF)
    logits[1, 17] = logits[1, 4000] = 100.0                # exact tie: lowest index wins
    logits[2, :] = 0.0
    got = O.argmax_first(logits)
    assert torch.equal(got, torch.argmax(logits, dim=-1))
    assert int(got[1]) == 17 and int(got[2]) == 0
