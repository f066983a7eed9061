"""Pins the Qwen3 eager oracle (CPU) against Transformers' Qwen3ForCausalLM at
random init: prefill logits, cached decode steps, greedy tokens, and the
one-forward teacher-forced replay (the reference's correctness judge,
QWEN_ENGINE_CONTRACT.md:105-121)."""

import pytest
import torch

from kernel_optim_amd.model import Qwen3Config, random_weights, to_hf_state_dict
from oracle.qwen3 import Qwen3Oracle

SMALL = Qwen3Config(hidden=512, inter=1024, layers=2, nq=8, nkv=2, head_dim=128, vocab=1000)


def hf_model(cfg, weights, attn="eager"):
    from transformers import Qwen3Config as HC, Qwen3ForCausalLM
    hc = HC(hidden_size=cfg.hidden, intermediate_size=cfg.inter,
            num_hidden_layers=cfg.layers, num_attention_heads=cfg.nq,
            num_key_value_heads=cfg.nkv, head_dim=cfg.head_dim, vocab_size=cfg.vocab,
            rms_norm_eps=cfg.eps, rope_theta=cfg.theta, tie_word_embeddings=cfg.tied,
            max_position_embeddings=4096, attn_implementation=attn)
    m = Qwen3ForCausalLM(hc).to(torch.bfloat16).eval()
    missing, unexpected = m.load_state_dict(to_hf_state_dict(cfg, weights), strict=False)
    assert not unexpected and all(k == "lm_head.weight" for k in missing)
    return m


def perturbed_weights(cfg, seed):
    w = random_weights(cfg, seed=seed)
    g = torch.Generator().manual_seed(seed + 100)
    for l in w["layers"]:
        for k in ("w_in", "w_post", "q_norm", "k_norm"):
            l[k] = (1 + 0.2 * torch.randn(l[k].shape, generator=g)).to(torch.bfloat16)
    w["final_norm"] = (1 + 0.2 * torch.randn(cfg.hidden, generator=g)).to(torch.bfloat16)
    return w


@torch.no_grad()
def hf_greedy(m, prompt, n_new):
    from transformers import DynamicCache
    cache = DynamicCache()
    out = m(input_ids=prompt, past_key_values=cache, use_cache=True)
    logits = [out.logits[:, -1]]
    tok = logits[-1].float().argmax(-1)
    toks = [tok]
    for _ in range(1, n_new):
        out = m(input_ids=tok[:, None], past_key_values=cache, use_cache=True)
        logits.append(out.logits[:, -1])
        tok = logits[-1].float().argmax(-1)
        toks.append(tok)
    return torch.stack(toks, 1), logits


@pytest.mark.parametrize("attn", ["eager", "sdpa"])
def test_oracle_matches_transformers_greedy(attn):
    cfg = SMALL
    w = perturbed_weights(cfg, seed=1)
    g = torch.Generator().manual_seed(2)
    prompt = torch.randint(0, cfg.vocab, (2, 24), generator=g)
    n_new = 12
    ref_toks, ref_logits = hf_greedy(hf_model(cfg, w, attn), prompt, n_new)
    orc = Qwen3Oracle(cfg, w, B=2, cap=64)
    toks, logits = orc.greedy(prompt, n_new)
    assert torch.equal(toks, ref_toks)
    for a, b in zip(logits, ref_logits):
        torch.testing.assert_close(a.float(), b.float(), rtol=0, atol=0.05)


def test_teacher_forced_replay_matches_cached_decode():
    cfg = SMALL
    w = perturbed_weights(cfg, seed=3)
    prompt = torch.randint(0, cfg.vocab, (2, 16), generator=torch.Generator().manual_seed(4))
    orc = Qwen3Oracle(cfg, w, B=2, cap=64)
    toks, logits = orc.greedy(prompt, 8)
    replay = Qwen3Oracle(cfg, w, B=2, cap=64).teacher_forced(prompt, toks)
    for j, step in enumerate(logits):
        torch.testing.assert_close(replay[:, j].float(), step.float(), rtol=0, atol=0.05)
    assert torch.equal(replay.float().argmax(-1), toks)


def test_weight_byte_counts_match_the_qwen3_4b_layout():
    cfg = Qwen3Config()
    assert cfg.layer_bytes() == 201_861_632
    assert cfg.weight_bytes_per_step() == 8_044_936_192


def test_bench_transformers_builder_matches_a_plain_build():
    """bench.py's CPU baseline builds Transformers' Qwen3ForCausalLM on the meta
    device and hands it the weights in place (no random init of 4B parameters);
    it must compute what a plain construction + load_state_dict computes, with
    the rotary inv_freq buffer in fp32 as from_pretrained(torch_dtype=bf16)
    leaves it (hf_model's blanket .to(bf16) rounds that buffer too)."""
    import bench
    cfg = SMALL
    w = perturbed_weights(cfg, seed=3)
    prompt = torch.randint(0, cfg.vocab, (2, 20), generator=torch.Generator().manual_seed(4))
    plain = hf_model(cfg, w, "sdpa")
    plain.model.rotary_emb.__init__(plain.config)
    assert plain.model.rotary_emb.inv_freq.dtype == torch.float32
    with torch.no_grad():
        want = plain(input_ids=prompt).logits
        got = bench.hf_qwen3_cpu(cfg, w)(input_ids=prompt).logits
    assert torch.equal(got, want)
