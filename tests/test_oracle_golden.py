"""The Qwen3 oracle against frozen Transformers outputs (tests/golden/qwen3_greedy.json,
written by tests/golden/make_golden.py with the installed Transformers): greedy
decodes at random init of a small config and of the Qwen3-4B width with 2
layers. The oracle replays the frozen tokens decode-shaped (prompt, then one
token per forward); its logits at the fixture's top-5 ids must be within 0.05 of
Transformers' (the bound of the live comparison in test_oracle_qwen3.py), and
every frozen token must be the oracle's argmax or within twice that bound of
its maximum (random-init logits are nearly flat, so near-ties occur)."""

import json
import os

import pytest
import torch

from oracle.qwen3 import Qwen3Oracle
from tests.golden.make_golden import CASES, build

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "qwen3_greedy.json")
TOL = 0.05


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_oracle_matches_frozen_transformers_greedy(case):
    with open(GOLDEN) as f:
        gold = json.load(f)["cases"][case[0]]
    cfg, w, prompt, n = build(case)
    toks = torch.tensor(gold["tokens"])
    B, S = prompt.shape
    with torch.no_grad():
        logits = Qwen3Oracle(cfg, w, B=B, cap=S + n).teacher_forced_decode(prompt, toks).float()
    ids = torch.tensor(gold["top5_ids"])
    want = torch.tensor(gold["top5_values"])
    assert float((logits.gather(2, ids) - want).abs().max()) < TOL
    best = logits.max(-1).values
    chosen = logits.gather(2, toks[..., None])[..., 0]
    assert torch.all(best - chosen <= 2 * TOL)
