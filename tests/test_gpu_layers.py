"""GPU parity of the one-launch decode layers (ko_decode_layers) against the
per-op launches it replaces (engine/engine.py:325-335 for one query token):
the qkv GEMV with the input RMSNorm, the one-token attention with the q/k norm,
RoPE, KV append and fused combine, the o GEMV with its residual add, the
gate|up GEMV with the post-attention RMSNorm and SwiGLU, and the down GEMV with
its residual add. The one-launch kernel runs the same per-workgroup code with
the same reduction order, so the comparison is bit for bit: the residual
stream, the appended KV slots and every scratch activation, over several graph
replays whose positions advance (the launch re-arms its counters and flags)."""

import pytest
import torch

pytestmark = pytest.mark.gpu

BF = torch.bfloat16
NQ, NKV, D, H, I = 32, 8, 128, 2560, 9728
EPS = 1e-6


def _model(L, B, cap, dev, seed):
    g = torch.Generator(device=dev).manual_seed(seed)

    def w(*shape):
        return (0.02 * torch.randn(*shape, device=dev, generator=g)).to(BF)

    def gain(n):
        return (1 + 0.2 * torch.randn(n, device=dev, generator=g)).to(BF)

    nqkv = (NQ + 2 * NKV) * D
    layers = [dict(w_in=gain(H), qkv=w(nqkv, H), q_norm=gain(D), k_norm=gain(D), o=w(H, NQ * D),
                   w_post=gain(H), gu=w(2 * I, H), down=w(H, I)) for _ in range(L)]
    k = torch.randn(L, B, NKV, cap, D, device=dev, generator=g).to(BF)
    v = torch.randn(L, B, NKV, cap, D, device=dev, generator=g).to(BF)
    h = torch.randn(B, H, device=dev, generator=g).to(BF)
    return layers, k, v, h


@pytest.mark.parametrize("B,cap,pos0,L", [(1, 1296, 1024, 3), (1, 1296, 0, 2), (2, 640, 517, 3)])
def test_decode_layers_equals_per_op_launches(dev, B, cap, pos0, L):
    from oracle import ops as O
    from kernel_optim_amd.kernels import gemv as GV
    from kernel_optim_amd.kernels.fused import DecodeAttention
    from kernel_optim_amd.kernels.layers import DecodeLayers

    layers, k0, v0, h0 = _model(L, B, cap, dev, 80 + B + pos0)
    cos, sin = (t.to(dev) for t in O.rope_tables(cap, D, 1.0e6))
    pos_start = torch.tensor([pos0, max(pos0 - 300, 0)][:B], dtype=torch.int32, device=dev)
    nqkv = (NQ + 2 * NKV) * D

    def run(one_launch, steps):
        k, v, h = k0.clone(), v0.clone(), h0.clone()
        pos = pos_start.clone()
        att = DecodeAttention(B, 1, cap, NQ, NKV, D, dev, fused_combine=True)
        qkv = torch.zeros(B, nqkv, device=dev, dtype=BF)
        out = torch.zeros(B, NQ * D, device=dev, dtype=BF)
        act = torch.zeros(B, I, device=dev, dtype=BF)
        if one_launch:
            assert DecodeLayers.supported(att, H, I)
            dl = DecodeLayers(att, layers, k, v, H, I)
        else:
            gq = GV.Gemv(B, nqkv, H, GV.EPI_BF16, norm=True, eps=EPS)
            go = GV.Gemv(B, H, NQ * D, GV.EPI_RESID, norm=False, eps=EPS)
            ggu = GV.Gemv(B, I, H, GV.EPI_SWIGLU, norm=True, eps=EPS)
            gd = GV.Gemv(B, H, I, GV.EPI_RESID, norm=False, eps=EPS)

        def step():
            if one_launch:
                dl(h, qkv, out, act, pos, cos, sin, EPS)
            else:
                for i, lw in enumerate(layers):
                    gq(h, lw["qkv"], y=qkv, nw=lw["w_in"], cfg=(0, 8, 0))
                    att.decode_qkv(qkv, lw["q_norm"], lw["k_norm"], cos, sin, pos, k[i], v[i],
                                   out, EPS)
                    go(out, lw["o"], h=h, cfg=(0, 8, 0))
                    ggu(h, lw["gu"], y=act, nw=lw["w_post"], cfg=(0, 8, 0))
                    gd(act, lw["down"], h=h, cfg=(0, 8, 0))
            pos.add_(1)

        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            step()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        for _ in range(steps - 1):
            graph.replay()
        torch.cuda.synchronize()
        if one_launch:
            assert int(dl.err.item()) == 0, "a stage wait gave up"
            assert torch.all(dl.counters == 0) and torch.all(dl.sync == 0)
        return dict(h=h.cpu(), k=k.cpu(), v=v.cpu(), qkv=qkv.cpu(), attn=out.cpu(),
                    act=act.cpu())

    want = run(False, 4)
    got = run(True, 4)
    assert torch.isfinite(want["h"].float()).all()
    for name in want:
        assert torch.equal(got[name], want[name]), name


def test_decode_layers_rejects_unsupported(dev):
    from kernel_optim_amd.kernels.fused import DecodeAttention
    from kernel_optim_amd.kernels.layers import DecodeLayers
    att3 = DecodeAttention(3, 1, 256, NQ, NKV, D, dev, fused_combine=True)
    assert not DecodeLayers.supported(att3, H, I)
    att = DecodeAttention(1, 1, 256, NQ, NKV, D, dev, fused_combine=True)
    assert DecodeLayers.supported(att, H, I)
    assert not DecodeLayers.supported(att, H, 10248)
    layers, k, v, _ = _model(1, 1, 256, dev, 5)
    with pytest.raises(ValueError):
        DecodeLayers(att, layers, k[:, :, :, :128], v, H, I)  # cache capacity mismatch
