"""GPU: speculative decoding by prompt lookup (engine/engine.py:48-93, 403-508).

The verify step runs B*(K+1) rows through the decode layers with attention
causal within each sequence's block; its logits must match the oracle's
teacher-forced logits at the same positions, and its ids must be the first
maximum of its own logits. Speculative generate() must emit the oracle's greedy
tokens except where the oracle's own top-1 and the chosen token are within the
logit tolerance of each other (a near-tie), on the fused-GEMV verify path
(B*(K+1) <= 16 rows), on the hipBLASLt path above it, while speculating
throughout and after handing over to the one-token graph."""

import pytest
import torch

from kernel_optim_amd.model import Qwen3Config, random_weights
from oracle.ops import argmax_first
from oracle.qwen3 import Qwen3Oracle
from tests.test_oracle_qwen3 import SMALL, perturbed_weights

pytestmark = pytest.mark.gpu
LOGIT_ATOL = 0.25


def _engine(cfg, w, **kw):
    from kernel_optim_amd.engine import Engine
    return Engine.from_weights(cfg, w, spec=True, **kw)


def _case(which, seed):
    if which == "small":
        return SMALL, perturbed_weights(SMALL, seed=seed)
    cfg = Qwen3Config(layers=2)   # Qwen3-4B width: the MFMA GEMV verify path at B = 1
    return cfg, random_weights(cfg, seed=seed)


@pytest.mark.parametrize("which,B", [("small", 1), ("small", 3), ("small", 16), ("small", 32),
                                     ("4b", 1), ("4b", 4)])
def test_verify_step_matches_teacher_forced_oracle(dev, which, B):
    """B = 16 and 32 draft 4 and 2 tokens: 80 and 96 verify rows, on hipBLASLt,
    with the attention's token rows past one wavefront's 64 lengths."""
    cfg, w = _case(which, 11)
    S, n = 40, 12
    prompt = torch.randint(0, cfg.vocab, (B, S), generator=torch.Generator().manual_seed(12))
    eng = _engine(cfg, w, keep_logits=True)
    toks, _ = eng.trace(prompt.tolist(), n)
    K = eng.K
    T = K + 1
    assert K == (6 if B <= 4 else 4 if B <= 16 else 2) and eng.verify_fused == (B * T <= 16)
    x = torch.cat([prompt, toks], 1)
    j = 2                      # verify rows x[p0 .. p0+K], p0 the position of x[p0]
    p0 = S - 1 + j
    print(f"{which} B={B}: verify rows {B * T} on the "
          f"{'fused GEMV' if eng.verify_fused else 'hipBLASLt'} path", flush=True)
    vout, logits = eng.verify_step(x[:, p0:p0 + T], torch.full((B,), p0, dtype=torch.int32))
    replay = Qwen3Oracle(cfg, w, B=B, cap=S + n).teacher_forced(prompt, toks)   # [B, n, V]
    ref = replay[:, j:j + T].float()
    got = logits.view(B, T, -1).float()
    err = float((got - ref).abs().max())
    print(f"  max |dlogit| {err:.4f}", flush=True)
    assert err < LOGIT_ATOL
    assert torch.equal(vout, argmax_first(logits).view(B, T))
    best = ref.max(-1).values
    chosen = ref.gather(2, vout[..., None])[..., 0]
    assert torch.all(best - chosen <= 2 * err + 1e-6)


@pytest.mark.parametrize("B,min_advance,graph", [(1, 0.0, "auto"), (2, 0.0, "auto"),
                                                 (3, 0.0, "auto"), (2, 1e9, "auto"),
                                                 (2, 1e9, "hipblaslt")])
def test_spec_generate_emits_oracle_greedy_tokens(dev, B, min_advance, graph):
    """min_advance 0: every step is a verify step; 1e9: the first acceptance check
    (after 8 verify steps) hands decoding to the one-token graph (graph: which
    decode graph that is)."""
    cfg = SMALL
    w = perturbed_weights(cfg, seed=13)
    g = torch.Generator().manual_seed(14)
    prompt = torch.randint(0, cfg.vocab, (B, 8), generator=g).repeat(1, 5)  # lookup finds matches
    S, n = prompt.shape[1], 40
    eng = _engine(cfg, w, decode_graph=graph)
    eng.min_advance = min_advance
    out = torch.tensor(list(eng.generate(prompt.tolist(), n))).T
    assert tuple(out.shape) == (B, n)
    steps = eng.spec_steps
    assert steps >= 1
    assert steps <= (n - 1 if min_advance == 0.0 else 8)
    print(f"B={B}: {steps} verify steps for {n - 1} tokens after the first", flush=True)
    again = torch.tensor(list(eng.generate(prompt.tolist(), n))).T
    assert torch.equal(again, out)   # deterministic; nothing left over from the first call
    replay = Qwen3Oracle(cfg, w, B=B, cap=S + n).teacher_forced(prompt, out).float()
    best = replay.max(-1).values
    chosen = replay.gather(2, out[..., None])[..., 0]
    assert torch.all(best - chosen <= 2 * LOGIT_ATOL)
    agree = float((argmax_first(replay) == out).float().mean())
    print(f"  oracle greedy agreement {agree:.3f}", flush=True)
