"""Checkpoint ingest (the reference's weight loading and concatenated qkv / gate-up
layout, engine/engine.py:124-154), on the CPU: save/load round trips, bit-exact,
with tied and untied LM heads, and a directory written by Transformers' own
save_pretrained of Qwen3ForCausalLM loads into the decode layout with every
tensor bit-equal and the same config."""

import dataclasses

import torch

from kernel_optim_amd.model import Qwen3Config, load_checkpoint, random_weights, save_checkpoint
from tests.test_oracle_qwen3 import SMALL, hf_model, perturbed_weights


def _assert_same(cfg_a, w_a, cfg_b, w_b):
    assert dataclasses.asdict(cfg_a) == dataclasses.asdict(cfg_b)
    for key in ("embed", "final_norm", "lm_head"):
        assert torch.equal(w_a[key], w_b[key]), key
    assert len(w_a["layers"]) == len(w_b["layers"])
    for la, lb in zip(w_a["layers"], w_b["layers"]):
        assert la.keys() == lb.keys()
        for k in la:
            assert torch.equal(la[k], lb[k]), k
    assert (w_b["lm_head"] is w_b["embed"]) == cfg_b.tied


def test_save_load_round_trip_tied(tmp_path):
    w = perturbed_weights(SMALL, seed=31)
    save_checkpoint(str(tmp_path), SMALL, w)
    cfg, w2 = load_checkpoint(str(tmp_path))
    _assert_same(SMALL, w, cfg, w2)


def test_save_load_round_trip_untied(tmp_path):
    cfg0 = dataclasses.replace(SMALL, tied=False)
    w = random_weights(cfg0, seed=32)
    assert w["lm_head"] is not w["embed"]
    save_checkpoint(str(tmp_path), cfg0, w)
    cfg, w2 = load_checkpoint(str(tmp_path))
    _assert_same(cfg0, w, cfg, w2)


def test_loads_a_transformers_save_pretrained_directory(tmp_path):
    w = perturbed_weights(SMALL, seed=33)
    hf_model(SMALL, w, "eager").save_pretrained(str(tmp_path), safe_serialization=True)
    cfg, w2 = load_checkpoint(str(tmp_path))
    assert isinstance(cfg, Qwen3Config)
    _assert_same(SMALL, w, cfg, w2)
