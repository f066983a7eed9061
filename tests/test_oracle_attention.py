"""Pins the attention oracle (CPU): library routine, brute force, closed forms,
and split-K invariants of the reference algorithm (engine/kernels/fused.py:138-234)."""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import attention as A


def _rand(B, nq, nkv, cap, D, T, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B * T, nq * D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, nkv, cap, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, nkv, cap, D, generator=g).to(torch.bfloat16)
    return q, k, v


@pytest.mark.parametrize("T", [1, 2, 4])
def test_closed_form_matches_sdpa(T):
    B, nq, nkv, cap, D = 3, 8, 2, 70, 16
    q, k, v = _rand(B, nq, nkv, cap, D, T)
    lens = [70, 33, T]
    got = A.decode_attention(q, k, v, lens, T=T)
    for b in range(B):
        L = lens[b]
        qq = q.view(B, T, nq, D)[b].transpose(0, 1).double()[None]        # [1, nq, T, D]
        kk = k[b, :, :L].double().repeat_interleave(nq // nkv, 0)[None]   # [1, nq, L, D]
        vv = v[b, :, :L].double().repeat_interleave(nq // nkv, 0)[None]
        mask = torch.ones(T, L, dtype=torch.bool)
        for t in range(T):
            mask[t, L - T + t + 1:] = False
        ref = F.scaled_dot_product_attention(qq, kk, vv, attn_mask=mask, scale=D ** -0.5)
        ref = ref[0].transpose(0, 1).reshape(T, nq * D)
        torch.testing.assert_close(got.view(B, T, -1)[b], ref, rtol=1e-12, atol=1e-12)


def test_brute_force_tiny():
    B, nq, nkv, cap, D, T = 1, 4, 2, 5, 3, 2
    q, k, v = _rand(B, nq, nkv, cap, D, T, seed=3)
    got = A.decode_attention(q, k, v, [4], T=T)
    qf, kf, vf = q.double().view(T, nq, D), k.double(), v.double()
    for t in range(T):
        for h in range(nq):
            kh = h // (nq // nkv)
            keys = range(0, 4 - T + t + 1)
            sc = [sum(qf[t, h, i] * kf[0, kh, j, i] for i in range(D)) / math.sqrt(D) for j in keys]
            mx = max(sc)
            w = [math.exp(s - mx) for s in sc]
            z = sum(w)
            for i in range(D):
                want = sum(w[n] * vf[0, kh, j, i] for n, j in enumerate(keys)) / z
                assert abs(float(got[t, h * D + i]) - float(want)) < 1e-12


def test_uniform_scores_give_mean_of_v():
    B, nq, nkv, cap, D = 2, 8, 2, 40, 16
    _, k, v = _rand(B, nq, nkv, cap, D, 1, seed=5)
    q = torch.zeros(B, nq * D, dtype=torch.bfloat16)
    lens = [40, 17]
    got = A.decode_attention(q, k, v, lens)
    for b in range(B):
        mean = v[b, :, :lens[b]].double().mean(dim=1)                    # [nkv, D]
        want = mean.repeat_interleave(nq // nkv, 0).reshape(-1)
        torch.testing.assert_close(got[b], want, rtol=1e-12, atol=1e-12)


def test_dominant_key_selects_its_value():
    B, nq, nkv, cap, D = 1, 4, 1, 30, 8
    _, k, v = _rand(B, nq, nkv, cap, D, 1, seed=6)
    q = torch.ones(1, nq * D, dtype=torch.bfloat16) * 8
    k = torch.zeros_like(k)
    k[0, 0, 11] = 8.0          # score 64*8/sqrt(8) >> 0 for key 11 only
    got = A.decode_attention(q, k, v, [30])
    want = v[0, 0, 11].double().repeat(nq)
    torch.testing.assert_close(got[0], want, rtol=0, atol=1e-30)


@pytest.mark.parametrize("T", [1, 3])
@pytest.mark.parametrize("nsplit", [1, 2, 3, 7])
def test_splitk_equals_closed_form(T, nsplit):
    B, nq, nkv, cap, D = 2, 8, 2, 200, 32
    q, k, v = _rand(B, nq, nkv, cap, D, T, seed=nsplit)
    pos = torch.tensor([200 - T, 57], dtype=torch.int32)
    chunk = -(-(-(-cap // nsplit)) // 16) * 16
    ns = -(-cap // chunk)
    out, _, _ = A.decode_attention_splitk(q, k, v, pos, T=T, nsplit=ns, chunk=chunk, block_n=16)
    want = A.decode_attention(q, k, v, [int(p) + T for p in pos], T=T)
    torch.testing.assert_close(out.double(), want, rtol=2e-2, atol=2e-2)


def test_empty_split_contributes_nothing():
    B, nq, nkv, cap, D = 1, 4, 1, 256, 16
    q, k, v = _rand(B, nq, nkv, cap, D, 1, seed=11)
    pos = torch.tensor([40], dtype=torch.int32)   # only split 0 of 4 has keys
    out, o_part, ml = A.decode_attention_splitk(q, k, v, pos, nsplit=4, chunk=64, block_n=16)
    l = ml.view(-1, 4, 2)[..., 1]
    assert torch.all(l[:, 1:] == 0) and torch.all(l[:, 0] > 0)
    assert torch.all(o_part.view(-1, 4, D)[:, 1:] == 0)
    out1, _, _ = A.decode_attention_splitk(q, k, v, pos, nsplit=1, chunk=256, block_n=16)
    torch.testing.assert_close(out.float(), out1.float(), rtol=0, atol=1e-2)


def test_reference_split_sizing_at_config2():
    # The reference's formula (fused.py:209-215) at B=16, cap=8192 with 264 CTAs.
    assert A.splitk_sizing(16, 8192, 8, 264) == (3, 2752)


def test_config1_cpu_path_matches_fp32():
    """Config 1: B1, 32q/8kv, d128, ctx 512, bf16 N(0,1) seeds q=0 k=1 v=2, the
    reference's CPU eager/SDPA path against the fp32 closed form."""
    gq, gk, gv = (torch.Generator().manual_seed(s) for s in (0, 1, 2))
    q = torch.randn(1, 32, 128, generator=gq).to(torch.bfloat16)
    k = torch.randn(1, 8, 512, 128, generator=gk).to(torch.bfloat16)
    v = torch.randn(1, 8, 512, 128, generator=gv).to(torch.bfloat16)
    sdpa = F.scaled_dot_product_attention(q[:, :, None], k, v, scale=128 ** -0.5, enable_gqa=True)
    ref = A.decode_attention(q.reshape(1, -1), k, v, [512], dtype=torch.float32)
    torch.testing.assert_close(sdpa.reshape(1, -1).float(), ref, rtol=2e-2, atol=2e-2)


def test_hbm_bytes_config2():
    assert A.hbm_bytes(16, 8, [8192] * 16, 32) == 537_133_056
