"""GPU: the prefill (kernel_optim_amd.prefill) against Transformers, not against
the oracle it once restated:
- bit for bit against a live Transformers Qwen3ForCausalLM (sdpa attention, bf16,
  the same weights) forward on the GPU: the prompt's K/V in every layer and the
  last-position logits, where the enable_gqa probe holds (else within 1 bf16 ulp);
- against the frozen Transformers greedy decodes of tests/golden/qwen3_greedy.json
  (first-step top-5 logits within 0.05, the first token the fixture's or a
  near-tie);
- the RoPE tables the engine builds on the GPU equal Qwen3RotaryEmbedding's
  forward on the GPU bit for bit.
Both forwards run with SDPA restricted to its fused kernels (no bf16 math path)."""

import json
import os

import pytest
import torch

from kernel_optim_amd.engine import _rope_tables
from kernel_optim_amd.model import Qwen3Config, random_weights, weights_to
from kernel_optim_amd.prefill import _sdpa_kernels, gqa_exact, prefill
from tests.bf16util import assert_bf16_close
from tests.golden.make_golden import CASES, build

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "qwen3_greedy.json")


def _caches(cfg, B, cap, dev):
    k = torch.zeros(cfg.layers, B, cfg.nkv, cap, cfg.head_dim, dtype=torch.bfloat16, device=dev)
    return k, torch.zeros_like(k)


@pytest.mark.parametrize("theta", [1.0e6, 5.0e6])
def test_rope_tables_equal_the_rotary_module_on_the_gpu(dev, theta):
    from transformers import Qwen3Config as HC
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RotaryEmbedding
    rot = Qwen3RotaryEmbedding(HC(head_dim=128, rope_theta=theta)).to(dev)
    n = 5000
    cos, sin = rot(torch.empty(1, dtype=torch.bfloat16, device=dev),
                   torch.arange(n, device=dev).unsqueeze(0))
    c, s = _rope_tables(n, 128, theta, dev)
    assert torch.equal(c, cos[0]) and torch.equal(s, sin[0])


@pytest.mark.parametrize("B,S", [(1, 77), (2, 300)])
def test_prefill_matches_transformers_sdpa(dev, B, S):
    import bench
    from transformers import DynamicCache
    cfg = Qwen3Config(layers=2)
    w = random_weights(cfg, seed=80 + B)
    m = bench.hf_qwen3_cpu(cfg, w).to(dev)
    prompt = torch.randint(0, cfg.vocab, (B, S), generator=torch.Generator().manual_seed(S)).to(dev)
    with torch.no_grad(), _sdpa_kernels():
        cache = DynamicCache()
        # the LM head on the last position only, as generate() runs it
        # (logits_to_keep=1) and as the reference's prefill does (engine.py:385)
        want = m(input_ids=prompt, past_key_values=cache, use_cache=True,
                 logits_to_keep=1).logits[:, -1]
    wd = weights_to(w, dev)
    kc, vc = _caches(cfg, B, S + 8, dev)
    cos, sin = _rope_tables(S + 8, cfg.head_dim, cfg.theta, dev)
    ids, logits = prefill(cfg, wd, prompt, kc, vc, cos, sin)
    exact = gqa_exact(dev)
    for i in range(cfg.layers):
        hk, hv = cache.layers[i].keys, cache.layers[i].values
        assert torch.equal(kc[i, :, :, :S], hk) and torch.equal(vc[i, :, :, :S], hv), i
    if exact:
        assert torch.equal(logits, want)
    else:
        assert_bf16_close(logits.cpu(), want.cpu(), max_frac=0.05)
    assert torch.equal(ids, logits.float().argmax(-1))
    print(f"prefill B={B} S={S}: enable_gqa bit-exact {exact}, max |dlogit| "
          f"{float((logits.float() - want.float()).abs().max()):.3e}")


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_prefill_matches_frozen_transformers(dev, case):
    with open(GOLDEN) as f:
        gold = json.load(f)["cases"][case[0]]
    cfg, w, prompt, n = build(case)
    B, S = prompt.shape
    kc, vc = _caches(cfg, B, S + 8, dev)
    cos, sin = _rope_tables(S + 8, cfg.head_dim, cfg.theta, dev)
    ids, logits = prefill(cfg, weights_to(w, dev), prompt.to(dev), kc, vc, cos, sin)
    lg = logits.float().cpu()
    top_ids = torch.tensor(gold["top5_ids"])[:, 0]          # first step
    want = torch.tensor(gold["top5_values"])[:, 0]
    assert float((lg.gather(1, top_ids) - want).abs().max()) < 0.05
    first = torch.tensor(gold["tokens"])[:, 0]
    chosen = lg.gather(1, first[:, None])[:, 0]
    assert torch.all(lg.max(-1).values - chosen <= 0.1)
