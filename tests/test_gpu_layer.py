"""GPU: one Qwen3-4B decoder layer decode step at 2048 cached keys (batch 1, 4
and 16), through the engine's own layer body (kernel_optim_amd.engine.decode_layer
with its tuned GEMVs and attention launch), against the oracle.

- The cache holds 2048 seeded N(0, 1) keys and values per sequence; the step
  runs RoPE and the KV append at position 2048 and attends over 2049 keys.
- Weights are random N(0, 0.02) bf16 (norm gains 1), the input token's
  embedding is the layer input.
- Checks: the appended K/V slot is bit-exact to oracle.ops.qk_norm_rope applied
  to the step's own bf16 qkv projection; the attention output matches the fp64
  oracle on those q/k/v within atol = rtol = 2e-2; the layer output (the
  residual stream) matches the oracle's eager layer within 2e-2 of its largest
  magnitude;
  every slot except 2048 is untouched.
"""

import time

import pytest
import torch

from kernel_optim_amd.engine import OPROJ_DELAY_NS, build_decode_gemvs, decode_layer
from kernel_optim_amd.kernels.fused import DecodeAttention, rope_rows
from kernel_optim_amd.model import Qwen3Config, random_weights
from oracle import attention as A
from oracle import ops as O
from oracle.qwen3 import Qwen3Oracle

pytestmark = pytest.mark.gpu
CTX = 2048


@pytest.mark.parametrize("B", [1, 4, 16])
def test_decoder_layer_2048_cached_keys(dev, B):
    cfg = Qwen3Config(layers=1)
    nq, nkv, d = cfg.nq, cfg.nkv, cfg.head_dim
    w = random_weights(cfg, seed=60 + B, device=dev)
    cap = CTX + 16
    orc = Qwen3Oracle(cfg, w, B=B, cap=cap, device=dev)
    g = torch.Generator(device=dev).manual_seed(B)
    orc.k[0, :, :, :CTX] = torch.randn(B, nkv, CTX, d, device=dev, generator=g).to(torch.bfloat16)
    orc.v[0, :, :, :CTX] = torch.randn(B, nkv, CTX, d, device=dev, generator=g).to(torch.bfloat16)
    k_cache, v_cache = orc.k[0].clone(), orc.v[0].clone()
    k_before = k_cache.clone()
    ids = torch.randint(0, cfg.vocab, (B,), generator=torch.Generator().manual_seed(70 + B))
    want_h = orc.forward(ids[:, None].to(dev), CTX, hidden=True)[:, 0].float().cpu()

    lw = w["layers"][0]
    raw = {name: [lw[name]] for name in ("qkv", "o", "gu", "down")}
    gv, W = build_decode_gemvs(cfg, B, raw, time.monotonic() + 30)
    attn = DecodeAttention(B, 1, cap, nq, nkv, d, dev, fused_combine=True)
    attn.oproj_delay_ns = OPROJ_DELAY_NS
    cos, sin = orc.cos, orc.sin
    pos = torch.full((B,), CTX, dtype=torch.int32, device=dev)
    rope = torch.empty(B, 2, d, dtype=torch.bfloat16, device=dev)
    rope_rows(pos, cos, sin, rope)
    h = w["embed"][ids.to(dev)].contiguous()
    qkv = torch.zeros(B, cfg.nqkv, dtype=torch.bfloat16, device=dev)
    attn_out = torch.zeros(B, nq * d, dtype=torch.bfloat16, device=dev)
    act = torch.zeros(B, cfg.inter, dtype=torch.bfloat16, device=dev)
    fuse_o = attn.oproj_fusable()
    decode_layer(gv, W, 0, lw, attn, h, qkv, attn_out, act, k_cache, v_cache, cos, sin, pos,
                 rope, cfg.eps, fuse_o)
    torch.cuda.synchronize()
    attn.check_sync()

    # the appended slot: bit-exact to the oracle's norm + RoPE + append of this qkv
    kc = torch.zeros(B, nkv, CTX + 1, d, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    q_ref = O.qk_norm_rope(qkv.cpu(), lw["q_norm"].cpu(), lw["k_norm"].cpu(), cos.cpu(),
                           sin.cpu(), pos.cpu(), kc, vc, 1, cfg.eps, nq, nkv, d)
    assert torch.equal(k_cache[:, :, CTX].cpu(), kc[:, :, CTX])
    assert torch.equal(v_cache[:, :, CTX].cpu(), vc[:, :, CTX])
    assert torch.equal(k_cache[:, :, :CTX], k_before[:, :, :CTX])
    assert torch.equal(k_cache[:, :, CTX + 1:], k_before[:, :, CTX + 1:])

    # the attention output on those q/k/v
    kf = k_cache[:, :, :CTX + 1].cpu()
    vf = v_cache[:, :, :CTX + 1].cpu()
    att_ref = A.decode_attention(q_ref, kf, vf, [CTX + 1] * B)
    torch.testing.assert_close(attn_out.cpu().double(), att_ref, atol=2e-2, rtol=2e-2)

    # the layer output
    got_h = h.float().cpu()
    err = float((got_h - want_h).abs().max())
    print(f"layer B={B} at {CTX} cached keys (o projection "
          f"{'in the attention launch' if fuse_o else 'own launch'}, cfgs "
          f"{ {k: gv[k].cfg for k in W} }): max |dh| {err:.3e}, max |h| "
          f"{float(want_h.abs().max()):.3f}")
    # the residual stream is rounded to bf16 at the scale of its largest elements
    # (|h| reaches ~4 here: one bf16 ulp is 0.016 there), so the 2e-2 bar is taken
    # relative to the tensor's magnitude
    scale = float(want_h.abs().max())
    assert err <= 2e-2 * scale, f"layer output differs by {err} (bar {2e-2 * scale})"
