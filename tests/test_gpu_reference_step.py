"""GPU: the reference engine's own fused decode step, run verbatim through this
package's ops (the "drops into engine.py" claim).

The sequence is engine/engine.py:245-292 (_setup_fused + _step1_fused):
- Gemv objects at their defaults, ``tune(weights, deadline)`` with the row-major
  weights only (no tiled copies passed), once with a live deadline and once with
  one that has passed (the reference's 150 s budget spent, engine.py:45,265);
- qkv GEMV with EPI_F32 and allow_split into an fp32 accumulator, its NORM
  prologue reading ss[0];
- qk_norm_rope_acc re-zeroing the accumulator and both ss rows;
- the two-launch DecodeAttention;
- o GEMV with RESID and ss_out=ss[1], gate/up with SWIGLU and ss=ss[1], down with
  RESID and ss_out=ss[0];
- the BF16 LM head with ss=ss[0], torch.argmax, pos += 1.

The prompt's K/V come from the oracle's prefill; each step's logits are checked
against the oracle's forward of the same token at the same position, and the
K/V the step appended against the oracle's cache slot.
"""

import time

import pytest
import torch

from kernel_optim_amd.kernels.fused import DecodeAttention
from kernel_optim_amd.kernels.gemv import (EPI_BF16, EPI_F32, EPI_RESID, EPI_SWIGLU, Gemv,
                                           embed_ss, qk_norm_rope_acc, uses_tiled)
from kernel_optim_amd.model import Qwen3Config, random_weights
from oracle.ops import rope_tables
from oracle.qwen3 import Qwen3Oracle
from tests.test_gpu_engine import LOGIT_ATOL, check_against_replay

pytestmark = pytest.mark.gpu


class ReferenceStep:
    """The reference's _setup_fused / _step1_fused state and call order, with this
    package's ops in place of its Triton kernels."""

    def __init__(self, cfg, w, B, cap, cos, sin, deadline, dev):
        self.cfg, self.w, self.B = cfg, w, B
        self.nq, self.nkv, self.d, self.eps = cfg.nq, cfg.nkv, cfg.head_dim, cfg.eps
        H, I, V = cfg.hidden, cfg.inter, cfg.vocab
        nqkv = (self.nq + 2 * self.nkv) * self.d
        bf = torch.bfloat16
        self.h = torch.zeros(B, H, dtype=bf, device=dev)
        self.ss = torch.zeros(2, B, dtype=torch.float32, device=dev)
        self.acc_qkv = torch.zeros(B, nqkv, dtype=torch.float32, device=dev)
        self.q1 = torch.zeros(B, self.nq * self.d, dtype=bf, device=dev)
        self.attn_out = torch.zeros(B, self.nq * self.d, dtype=bf, device=dev)
        self.act = torch.zeros(B, I, dtype=bf, device=dev)
        self.logits = torch.zeros(B, V, dtype=bf, device=dev)
        eps = self.eps
        L = w["layers"]
        self.gv = dict(
            qkv=(Gemv(B, nqkv, H, EPI_F32, norm=True, allow_split=True, eps=eps),
                 [l["qkv"] for l in L]),
            o=(Gemv(B, H, self.nq * self.d, EPI_RESID, norm=False, eps=eps), [l["o"] for l in L]),
            gu=(Gemv(B, I, H, EPI_SWIGLU, norm=True, eps=eps), [l["gu"] for l in L]),
            down=(Gemv(B, H, I, EPI_RESID, norm=False, eps=eps), [l["down"] for l in L]),
            lm=(Gemv(B, V, H, EPI_BF16, norm=True, eps=eps), [w["lm_head"]]),
        )
        for name, (g, ws) in self.gv.items():
            g.tune(ws, deadline)
        self.acc_qkv.zero_()
        self.ss.zero_()
        self.attn1 = DecodeAttention(B, 1, cap, self.nq, self.nkv, self.d, dev)
        self.cos, self.sin = cos, sin

    def step(self, ids, pos, k_cache, v_cache):
        g = {k: v[0] for k, v in self.gv.items()}
        h, ss, w = self.h, self.ss, self.w
        embed_ss(ids, w["embed"], h, ss[0])
        for i, lw in enumerate(w["layers"]):
            g["qkv"](h, lw["qkv"], y=self.acc_qkv, nw=lw["w_in"], ss=ss[0])
            qk_norm_rope_acc(self.acc_qkv, lw["q_norm"], lw["k_norm"], self.cos, self.sin, pos,
                             self.q1, k_cache[i], v_cache[i], ss, self.eps, self.nq, self.nkv,
                             self.d)
            self.attn1(self.q1, k_cache[i], v_cache[i], pos, self.attn_out)
            g["o"](self.attn_out, lw["o"], h=h, ss_out=ss[1])
            g["gu"](h, lw["gu"], y=self.act, nw=lw["w_post"], ss=ss[1])
            g["down"](self.act, lw["down"], h=h, ss_out=ss[0])
        g["lm"](h, w["lm_head"], y=self.logits, nw=w["final_norm"], ss=ss[0])
        torch.argmax(self.logits, dim=-1, out=ids)
        pos.add_(1)


@pytest.mark.parametrize("deadline", ["live", "expired"])
@pytest.mark.parametrize("B", [1, 5, 16])
def test_reference_fused_decode_step(dev, B, deadline):
    cfg = Qwen3Config(layers=2)
    w = random_weights(cfg, seed=40 + B, device=dev)
    S, steps = 40, 4
    cap = S + steps + 12
    prompt = torch.randint(0, cfg.vocab, (B, S), generator=torch.Generator().manual_seed(B))
    orc = Qwen3Oracle(cfg, w, B=B, cap=cap, device=dev)
    first = orc.forward(prompt.to(dev), 0)[:, -1]
    k_cache, v_cache = orc.k.clone(), orc.v.clone()   # the prompt's K/V (slots 0..S-1)
    cos, sin = (t.to(dev) for t in rope_tables(cap, cfg.head_dim, cfg.theta))
    t_end = time.monotonic() + (150.0 if deadline == "live" else -1.0)
    ref = ReferenceStep(cfg, w, B, cap, cos, sin, t_end, dev)
    cfgs = {k: g.cfg for k, (g, _) in ref.gv.items()}
    if deadline == "expired":
        assert not any(uses_tiled(c) for c in cfgs.values()), cfgs
    ids = first.float().argmax(-1)
    pos = torch.full((B,), S, dtype=torch.int32, device=dev)
    toks, got, want = [], [], []
    for j in range(steps):
        tok = ids.clone()
        ref.step(ids, pos, k_cache, v_cache)
        torch.cuda.synchronize()
        want.append(orc.forward(tok[:, None], S + j)[:, -1].cpu())
        got.append(ref.logits.cpu())
        toks.append(ids.cpu().clone())
        # the appended slot, against the oracle's cache: layer 0 projects the same
        # input in both (a bf16 ulp apart at most); later layers project a residual
        # stream that already differs by bf16 roundings, so their bar is 2e-2 of
        # the slot's largest magnitude
        for i in range(cfg.layers):
            for mine, theirs in ((k_cache, orc.k), (v_cache, orc.v)):
                a, b = mine[i, :, :, S + j].float(), theirs[i, :, :, S + j].float()
                if i == 0:
                    torch.testing.assert_close(a, b, atol=2e-2, rtol=2e-2)
                else:
                    assert float((a - b).abs().max()) <= 2e-2 * float(b.abs().max())
        assert torch.all(pos == S + j + 1)
    agree, err = check_against_replay(torch.stack(toks, 1), got, torch.stack(want, 1))
    print(f"reference decode step B={B} ({deadline} deadline, cfgs {cfgs}): agreement "
          f"{agree:.3f}, max |dlogit| {err:.4f}")
    assert err < LOGIT_ATOL
