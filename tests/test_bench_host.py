"""CPU: the benchmark's quality check, the reference contract's teacher-forced replay
(QWEN_ENGINE_CONTRACT.md, "The quality rule"), on a small Qwen3 model: the model's own
cached greedy tokens pass with full agreement, and a token planted off the argmax by
more than the tie margin is counted and fails the check."""

import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

transformers = pytest.importorskip("transformers")


def _greedy(m, prompt, n):
    from transformers import DynamicCache
    with torch.inference_mode():
        out = m(input_ids=torch.tensor(prompt), past_key_values=DynamicCache(), use_cache=True)
        tok = out.logits[:, -1].float().argmax(-1)
        steps, pkv = [tok.tolist()], out.past_key_values
        for _ in range(n - 1):
            out = m(input_ids=tok[:, None], past_key_values=pkv, use_cache=True)
            tok = out.logits[:, -1].float().argmax(-1)
            steps.append(tok.tolist())
    return steps


def test_teacher_forced_quality_check():
    import bench
    from kernel_optim_amd.model import Qwen3Config, random_weights
    cfg = Qwen3Config(hidden=512, inter=1024, layers=2, nq=8, nkv=2, head_dim=128, vocab=1000)
    m = bench.hf_qwen3_cpu(cfg, random_weights(cfg, seed=1))
    prompt = torch.randint(0, cfg.vocab, (3, 30), generator=torch.Generator().manual_seed(2)).tolist()
    steps = _greedy(m, prompt, 8)
    q = bench.hf_teacher_forced_quality(m, prompt, steps, [0, 1, 2])
    assert q["positions"] == 24 and q["greedy_agreement"] == 1.0
    assert q["max_gap_to_argmax_logits"] == 0.0 and q["pass"]
    # plant the token least likely at step 3 of sequence 1: far outside the margin
    with torch.inference_mode():
        ids = torch.tensor([prompt[1] + [s[1] for s in steps[:3]]])
        worst = int(m(input_ids=ids).logits[0, -1].float().argmin())
    bad = [list(s) for s in steps]
    bad[3][1] = worst
    q = bench.hf_teacher_forced_quality(m, prompt, bad, [1])
    assert not q["pass"] and q["positions_over_margin"] >= 1
    assert q["max_gap_to_argmax_logits"] > q["tie_margin_logits"]
