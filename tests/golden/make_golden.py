"""Writes qwen3_greedy.json: greedy decodes of Transformers' Qwen3ForCausalLM
(the library the reference's model semantics come from, installed here) at
random init, frozen as fixtures: the generated ids and the top-5 logits of
every step. Inputs are not stored; they are rebuilt from the seeds below with
kernel_optim_amd.model.random_weights and torch.Generator on the CPU.

Run from the repository root: python tests/golden/make_golden.py
"""

import json
import os
import sys

import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from kernel_optim_amd.model import Qwen3Config, random_weights  # noqa: E402
from tests.test_oracle_qwen3 import SMALL, hf_greedy, hf_model, perturbed_weights  # noqa: E402

CASES = [
    # name, config kwargs, weights ("perturbed" norms or plain random), weight seed,
    # prompt seed, batch, prompt length, new tokens
    ("small_b2", dict(hidden=512, inter=1024, layers=2, nq=8, nkv=2, head_dim=128, vocab=1000),
     "perturbed", 21, 22, 2, 24, 10),
    ("qwen3_4b_width_2_layers_b1", dict(layers=2), "random", 23, 24, 1, 16, 4),
]


def build(case):
    name, kw, kind, wseed, pseed, B, S, n = case
    cfg = Qwen3Config(**kw)
    w = perturbed_weights(cfg, seed=wseed) if kind == "perturbed" else random_weights(cfg, seed=wseed)
    prompt = torch.randint(0, cfg.vocab, (B, S), generator=torch.Generator().manual_seed(pseed))
    return cfg, w, prompt, n


def main():
    assert SMALL.vocab == 1000
    out = {"library": "transformers", "version": __import__("transformers").__version__,
           "attention": "eager", "cases": {}}
    for case in CASES:
        cfg, w, prompt, n = build(case)
        toks, logits = hf_greedy(hf_model(cfg, w, "eager"), prompt, n)
        lg = torch.stack([l.float() for l in logits], 1)   # [B, n, V]
        top = lg.topk(5, dim=-1)
        out["cases"][case[0]] = {
            "tokens": toks.tolist(),
            "top5_values": [[[round(v, 4) for v in s] for s in b] for b in top.values.tolist()],
            "top5_ids": top.indices.tolist(),
        }
        print(case[0], toks.tolist(), flush=True)
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "qwen3_greedy.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    print("wrote", path)


if __name__ == "__main__":
    main()
