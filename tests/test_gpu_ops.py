"""GPU parity of the fused decode ops and the GEMV family against the CPU oracle
(engine/kernels/fused.py and gemv.py semantics). bf16 outputs are compared in
bf16 units in the last place (ulp): the kernels follow the reference's cast
chain, so only fp32 reduction order (and rsqrt/exp last-bit differences) may
move a result by one bf16 ulp."""

import pytest
import torch

from oracle import ops as O
from tests.bf16util import assert_bf16_close, assert_resid_close, one_ulp_at

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def K():
    from kernel_optim_amd.kernels import fused, gemv
    return fused, gemv


def _g(dev, seed):
    return torch.Generator(device=dev).manual_seed(seed)


@pytest.mark.parametrize("with_delta", [False, True])
def test_add_rms_norm(dev, with_delta):
    fused, _ = K()
    g = _g(dev, 1)
    res = torch.randn(5, 2560, device=dev, generator=g).to(BF)
    delta = torch.randn(5, 2560, device=dev, generator=g).to(BF) if with_delta else None
    w = (1 + 0.1 * torch.randn(2560, device=dev, generator=g)).to(BF)
    want_res, want = O.add_rms_norm(res.cpu(), None if delta is None else delta.cpu(), w.cpu(), 1e-6)
    out = torch.empty_like(res)
    fused.add_rms_norm(res, delta, w, out, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(res.cpu(), want_res)
    assert_bf16_close(out.cpu(), want)


@pytest.mark.parametrize("T", [1, 3])
def test_qk_norm_rope_append(dev, T):
    fused, _ = K()
    B, nq, nkv, d, cap = 3, 32, 8, 128, 96
    g = _g(dev, 2)
    qkv = torch.randn(B * T, (nq + 2 * nkv) * d, device=dev, generator=g).to(BF)
    qw = (1 + 0.2 * torch.randn(d, device=dev, generator=g)).to(BF)
    kw = (1 + 0.2 * torch.randn(d, device=dev, generator=g)).to(BF)
    cos, sin = (t.to(dev) for t in O.rope_tables(cap, d, 1.0e6))
    pos = torch.tensor([0, 41, cap - T], dtype=torch.int32, device=dev)
    kc = torch.randn(B, nkv, cap, d, device=dev, generator=g).to(BF)
    vc = torch.randn(B, nkv, cap, d, device=dev, generator=g).to(BF)
    kc0, vc0 = kc.cpu(), vc.cpu()
    q_out = torch.empty(B * T, nq * d, device=dev, dtype=BF)
    fused.qk_norm_rope(qkv, qw, kw, cos, sin, pos, q_out, kc, vc, T, 1e-6, nq, nkv, d)
    torch.cuda.synchronize()
    kref, vref = kc0.clone(), vc0.clone()
    qref = O.qk_norm_rope(qkv.cpu(), qw.cpu(), kw.cpu(), cos.cpu(), sin.cpu(), pos.cpu(), kref,
                          vref, T, 1e-6, nq, nkv, d)
    assert_bf16_close(q_out.cpu(), qref)
    assert_bf16_close(kc.cpu(), kref, max_frac=1e-3)
    assert torch.equal(vc.cpu(), vref)


def test_qk_norm_rope_acc_rezeroes(dev):
    _, gemv = K()
    B, nq, nkv, d, cap = 2, 32, 8, 128, 40
    g = _g(dev, 3)
    acc = torch.randn(B, (nq + 2 * nkv) * d, device=dev, generator=g)
    acc_cpu = acc.cpu()
    qw = torch.ones(d, device=dev, dtype=BF)
    kw = torch.ones(d, device=dev, dtype=BF)
    cos, sin = (t.to(dev) for t in O.rope_tables(cap))
    pos = torch.tensor([7, 39], dtype=torch.int32, device=dev)
    kc = torch.zeros(B, nkv, cap, d, device=dev, dtype=BF)
    vc = torch.zeros_like(kc)
    q_out = torch.empty(B, nq * d, device=dev, dtype=BF)
    zb = torch.ones(2, B, device=dev)
    gemv.qk_norm_rope_acc(acc, qw, kw, cos, sin, pos, q_out, kc, vc, zb, 1e-6, nq, nkv, d)
    torch.cuda.synchronize()
    assert torch.all(acc == 0) and torch.all(zb == 0)
    kref, vref = torch.zeros(B, nkv, cap, d, dtype=BF), torch.zeros(B, nkv, cap, d, dtype=BF)
    qref = O.qk_norm_rope_acc(acc_cpu, qw.cpu(), kw.cpu(), cos.cpu(), sin.cpu(), pos.cpu(), kref,
                              vref, 1e-6, nq, nkv, d)
    assert_bf16_close(q_out.cpu(), qref)
    assert_bf16_close(kc.cpu(), kref, max_frac=1e-3)
    assert torch.equal(vc.cpu(), vref)


def test_silu_mul(dev):
    fused, _ = K()
    g = _g(dev, 4)
    gu = (3 * torch.randn(4, 2 * 9728, device=dev, generator=g)).to(BF)
    out = torch.empty(4, 9728, device=dev, dtype=BF)
    fused.silu_mul(gu, out)
    torch.cuda.synchronize()
    assert_bf16_close(out.cpu(), O.silu_mul(gu.cpu()))


def test_embed_ss(dev):
    _, gemv = K()
    g = _g(dev, 5)
    emb = torch.randn(151936, 2560, device=dev, generator=g).to(BF)
    ids = torch.tensor([0, 151935, 4242, 7], device=dev)
    h = torch.empty(4, 2560, device=dev, dtype=BF)
    ss = torch.empty(4, device=dev)
    gemv.embed_ss(ids, emb, h, ss)
    torch.cuda.synchronize()
    hr, ssr = O.embed_ss(ids.cpu(), emb.cpu())
    assert torch.equal(h.cpu(), hr)
    torch.testing.assert_close(ss.cpu(), ssr, rtol=1e-5, atol=1e-3)


SHAPES = {  # Qwen3-4B decode projections (engine.py:258-264)
    "qkv": (6144, 2560),
    "o": (2560, 4096),
    "gu": (9728, 2560),
    "down": (2560, 9728),
}


def _weights(dev, N, K, seed, rows=None):
    g = _g(dev, seed)
    return (0.02 * torch.randn(rows or N, K, device=dev, generator=g)).to(BF)


CFGS = [(0, 4, 0), (0, 8, 0), (1, 1, 2), (1, 2, 4), (1, 4, 2), (2, 1, 0), (2, 2, 0)]


@pytest.mark.parametrize("M", [1, 2, 3, 4, 16])
@pytest.mark.parametrize("cfg", CFGS)
def test_gemv_epilogues(dev, M, cfg):
    _, gemv = K()
    if cfg[0] == 1 and M > 4:
        pytest.skip("layout 1 serves M <= 4")
    rows = cfg

    def lay(W, swiglu=False):  # layout 2 reads the tiled copy of the weights
        return gemv.tile_weights(W, swiglu=swiglu) if cfg[0] == 2 else W

    g = _g(dev, 10 + M)
    # qkv: NORM + F32, ss computed in-kernel and passed explicitly
    N, Kd = SHAPES["qkv"]
    x = torch.randn(M, Kd, device=dev, generator=g).to(BF)
    nw = (1 + 0.1 * torch.randn(Kd, device=dev, generator=g)).to(BF)
    W = _weights(dev, N, Kd, 20)
    ss = x.float().pow(2).sum(-1)
    want = O.gemv(x.cpu(), W.cpu(), O.EPI_F32, nw=nw.cpu(), ss=ss.cpu())
    for ss_arg in (None, ss):
        y = torch.empty(M, N, device=dev)
        gemv.Gemv(M, N, Kd, gemv.EPI_F32, norm=True)(x, lay(W), y=y, nw=nw, ss=ss_arg, cfg=rows)
        torch.cuda.synchronize()
        torch.testing.assert_close(y.cpu(), want, rtol=2e-3, atol=2e-3)
    # o: RESID with ss_out
    N, Kd = SHAPES["o"]
    a = torch.randn(M, Kd, device=dev, generator=g).to(BF)
    W = _weights(dev, N, Kd, 21)
    h = torch.randn(M, N, device=dev, generator=g).to(BF)
    hr, ssr = O.gemv(a.cpu(), W.cpu(), O.EPI_RESID, h=h.cpu())
    ss_out = torch.full((M,), 5.0, device=dev)
    gemv.Gemv(M, N, Kd, gemv.EPI_RESID, norm=False)(a, lay(W), h=h, ss_out=ss_out, cfg=rows)
    torch.cuda.synchronize()
    assert_bf16_close(h.cpu(), hr, max_frac=0.02, atol=one_ulp_at(hr))
    torch.testing.assert_close(ss_out.cpu(), ssr + 5.0, rtol=1e-3, atol=1e-2)
    # gu: NORM + SWIGLU
    N, Kd = SHAPES["gu"]
    x = torch.randn(M, Kd, device=dev, generator=g).to(BF)
    W = _weights(dev, N, Kd, 22, rows=2 * N)
    y = torch.empty(M, N, device=dev, dtype=BF)
    gemv.Gemv(M, N, Kd, gemv.EPI_SWIGLU, norm=True)(x, lay(W, swiglu=True), y=y, nw=nw, cfg=rows)
    torch.cuda.synchronize()
    want = O.gemv(x.cpu(), W.cpu(), O.EPI_SWIGLU, nw=nw.cpu(), ss=x.cpu().float().pow(2).sum(-1))
    assert_bf16_close(y.cpu(), want, max_ulp=2, max_frac=0.03, atol=one_ulp_at(want))
    # down: BF16 (plain projection)
    N, Kd = SHAPES["down"]
    a = torch.randn(M, Kd, device=dev, generator=g).to(BF)
    W = _weights(dev, N, Kd, 23)
    y = torch.empty(M, N, device=dev, dtype=BF)
    gemv.Gemv(M, N, Kd, gemv.EPI_BF16, norm=False)(a, lay(W), y=y, cfg=rows)
    torch.cuda.synchronize()
    want = O.gemv(a.cpu(), W.cpu(), O.EPI_BF16)
    assert_bf16_close(y.cpu(), want, max_frac=0.02, atol=one_ulp_at(want))


@pytest.mark.parametrize("M", [17, 32, 40])
@pytest.mark.parametrize("cfg", [(2, 1, 2), (2, 2, 2)])
def test_gemv_two_row_tiles(dev, M, cfg):
    """Layout 2 with two row tiles (32 rows of x per weight pass; M = 17 leaves
    one row in the second tile, M = 40 runs a 32-row slice and an 8-row slice on
    one tile). Every row equals the one-tile launch bit for bit (the same MFMA
    steps over the same weights, the same norm sums) and the oracle within the
    bf16 tolerance."""
    _, gemv = K()
    one = (2, cfg[1], 0)
    g = _g(dev, 60 + M)

    def both(op, x, w, **kw):  # the two-tile and the one-tile config, on fresh outputs
        outs = []
        for c in (cfg, one):
            kk = {k: (v.clone() if k in ("y", "h", "ss_out") else v) for k, v in kw.items()}
            op(x, w, cfg=c, **kk)
            torch.cuda.synchronize()
            outs.append(kk)
        return outs

    # qkv: NORM + F32, ss in-kernel and given
    N, Kd = SHAPES["qkv"]
    x = torch.randn(M, Kd, device=dev, generator=g).to(BF)
    nw = (1 + 0.1 * torch.randn(Kd, device=dev, generator=g)).to(BF)
    W = _weights(dev, N, Kd, 61)
    Wt = gemv.tile_weights(W)
    ss = x.float().pow(2).sum(-1)
    want = O.gemv(x.cpu(), W.cpu(), O.EPI_F32, nw=nw.cpu(), ss=ss.cpu())
    op = gemv.Gemv(M, N, Kd, gemv.EPI_F32, norm=True)
    assert cfg in op.candidates()
    for ss_arg in (None, ss):
        a, b = both(op, x, Wt, y=torch.empty(M, N, device=dev), nw=nw, ss=ss_arg)
        assert torch.equal(a["y"], b["y"])
        torch.testing.assert_close(a["y"].cpu(), want, rtol=2e-3, atol=2e-3)
    # o: RESID with ss_out, and BF16
    N, Kd = SHAPES["o"]
    xa = torch.randn(M, Kd, device=dev, generator=g).to(BF)
    W = _weights(dev, N, Kd, 62)
    Wt = gemv.tile_weights(W)
    h = torch.randn(M, N, device=dev, generator=g).to(BF)
    hr, ssr = O.gemv(xa.cpu(), W.cpu(), O.EPI_RESID, h=h.cpu())
    op = gemv.Gemv(M, N, Kd, gemv.EPI_RESID, norm=False)
    assert cfg in op.candidates()
    a, b = both(op, xa, Wt, h=h, ss_out=torch.full((M,), 5.0, device=dev))
    assert torch.equal(a["h"], b["h"])
    assert_resid_close(a["h"].cpu(), hr, O.gemv(xa.cpu(), W.cpu(), O.EPI_F32))
    torch.testing.assert_close(a["ss_out"].cpu(), ssr + 5.0, rtol=1e-3, atol=1e-2)
    op = gemv.Gemv(M, N, Kd, gemv.EPI_BF16, norm=False)
    a, b = both(op, xa, Wt, y=torch.empty(M, N, device=dev, dtype=BF))
    assert torch.equal(a["y"], b["y"])
    want = O.gemv(xa.cpu(), W.cpu(), O.EPI_BF16)
    assert_bf16_close(a["y"].cpu(), want, max_frac=0.02, atol=one_ulp_at(want))
    # gu: NORM + SWIGLU
    N, Kd = SHAPES["gu"]
    W = _weights(dev, N, Kd, 63, rows=2 * N)
    Wt = gemv.tile_weights(W, swiglu=True)
    op = gemv.Gemv(M, N, Kd, gemv.EPI_SWIGLU, norm=True)
    assert cfg in op.candidates()
    a, b = both(op, x, Wt, y=torch.empty(M, N, device=dev, dtype=BF), nw=nw)
    assert torch.equal(a["y"], b["y"])
    want = O.gemv(x.cpu(), W.cpu(), O.EPI_SWIGLU, nw=nw.cpu(), ss=x.cpu().float().pow(2).sum(-1))
    # 4 ulp: where the fp32 gate sum lies on a bf16 rounding tie, bf16(g) may round
    # either way; one ulp of g moves silu(g) by silu'(g) / silu(g) x ulp(g), about
    # 0.9 % at g = 0.52, 3 ulp of the product (seen at M = 40: g = 0.517578 in fp64)
    assert_bf16_close(a["y"].cpu(), want, max_ulp=4, max_frac=0.03, atol=one_ulp_at(want))
    # down (K = 9728) has no two-tile build
    assert cfg not in gemv.Gemv(M, *SHAPES["down"], gemv.EPI_BF16, norm=False).candidates()


@pytest.mark.parametrize("M,waves", [(17, 2), (32, 2), (40, 2), (40, 4), (64, 4), (70, 4)])
def test_gemv_stream_k_two_row_tiles(dev, M, waves):
    """Layout 4 with two or four row tiles (x of rows 0-15, 16-31, ... loaded per K
    step with the weights) at every K it takes (2560, 4096, 9728): each row
    equals the one-tile launch bit for bit and the oracle within the bf16
    tolerance. M = 40 on four tiles leaves the last two part-filled; M = 70 runs
    a 64-row slice and a 6-row slice on one tile."""
    _, gemv = K()
    cfg_mt = (4, 10, waves)
    g = _g(dev, 70 + M + waves)
    cases = [("o", gemv.EPI_RESID), ("o", gemv.EPI_BF16), ("down", gemv.EPI_BF16),
             ("down", gemv.EPI_F32), ("down", gemv.EPI_RESID), ("qkv", gemv.EPI_BF16)]
    for shape, epi in cases:
        N, Kd = SHAPES[shape]
        x = torch.randn(M, Kd, device=dev, generator=g).to(BF)
        W = _weights(dev, N, Kd, 71)
        Wt = gemv.tile_weights(W)
        op = gemv.Gemv(M, N, Kd, epi, norm=False)
        assert cfg_mt in op.candidates()
        outs = []
        h0 = torch.randn(M, N, device=dev, generator=g).to(BF)
        for cfg in (cfg_mt, (4, 10, 0)):
            if epi == gemv.EPI_RESID:
                h, ss_out = h0.clone(), torch.full((M,), 5.0, device=dev)
                op(x, Wt, h=h, ss_out=ss_out, cfg=cfg)
                outs.append((h, ss_out))
            else:
                y = torch.empty(M, N, device=dev, dtype=torch.float32 if epi == gemv.EPI_F32 else BF)
                op(x, Wt, y=y, cfg=cfg)
                outs.append((y,))
            torch.cuda.synchronize()
        assert torch.equal(outs[0][0], outs[1][0]), (shape, epi)
        if epi == gemv.EPI_RESID:
            want, ssr = O.gemv(x.cpu(), W.cpu(), O.EPI_RESID, h=h0.cpu())
            y = O.gemv(x.cpu(), W.cpu(), O.EPI_F32)
            assert_resid_close(outs[0][0].cpu(), want, y)
            torch.testing.assert_close(outs[0][1].cpu(), ssr + 5.0, rtol=1e-3, atol=1e-2)
        elif epi == gemv.EPI_BF16:
            want = O.gemv(x.cpu(), W.cpu(), O.EPI_BF16)
            assert_bf16_close(outs[0][0].cpu(), want, max_frac=0.02, atol=one_ulp_at(want))
        else:
            want = O.gemv(x.cpu(), W.cpu(), O.EPI_F32)
            torch.testing.assert_close(outs[0][0].cpu(), want, rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize("M", [2, 7, 16, 20])
def test_gemv_split_k_layout(dev, M):
    """Layout 3 (MFMA tiles, K cut into slices merged by the last workgroup of
    each tile, in slice order) for every Qwen3-4B projection and every slice
    count it takes, and layout 4 (each tile's 16 K chunks dealt out 10 per
    workgroup, merged in workgroup order) for the projections it takes, against
    the oracle; bit-identical on a second call and on graph replays (the arrival
    counters re-arm); M = 20 runs as 16 + 4 rows on the same counters."""
    _, gemv = K()
    g = _g(dev, 50 + M)
    nw = (1 + 0.1 * torch.randn(2560, device=dev, generator=g)).to(BF)
    cases = []
    # qkv: NORM + BF16 (one slice: the row norm needs the whole row)
    N, Kd = SHAPES["qkv"]
    x = torch.randn(M, Kd, device=dev, generator=g).to(BF)
    W = _weights(dev, N, Kd, 60)
    want = O.gemv(x.cpu(), W.cpu(), O.EPI_BF16, nw=nw.cpu(), ss=x.cpu().float().pow(2).sum(-1))
    cases.append(("qkv", gemv.Gemv(M, N, Kd, gemv.EPI_BF16, norm=True), x,
                  gemv.tile_weights(W), dict(nw=nw), "y", N, want))
    # gu: NORM + SWIGLU
    N, Kd = SHAPES["gu"]
    x = torch.randn(M, Kd, device=dev, generator=g).to(BF)
    W = _weights(dev, N, Kd, 61, rows=2 * N)
    want = O.gemv(x.cpu(), W.cpu(), O.EPI_SWIGLU, nw=nw.cpu(), ss=x.cpu().float().pow(2).sum(-1))
    cases.append(("gu", gemv.Gemv(M, N, Kd, gemv.EPI_SWIGLU, norm=True), x,
                  gemv.tile_weights(W, swiglu=True), dict(nw=nw), "y", N, want))
    # o: RESID; down: BF16
    for name, epi, seed in (("o", gemv.EPI_RESID, 62), ("down", gemv.EPI_BF16, 63)):
        N, Kd = SHAPES[name]
        a = torch.randn(M, Kd, device=dev, generator=g).to(BF)
        W = _weights(dev, N, Kd, seed)
        h0 = torch.randn(M, N, device=dev, generator=g).to(BF)
        if epi == gemv.EPI_RESID:
            want, _ = O.gemv(a.cpu(), W.cpu(), O.EPI_RESID, h=h0.cpu())
        else:
            want = O.gemv(a.cpu(), W.cpu(), O.EPI_BF16)
        cases.append((name, gemv.Gemv(M, N, Kd, epi, norm=False), a, gemv.tile_weights(W),
                      dict(h0=h0), "h" if epi == gemv.EPI_RESID else "y", N, want))
    seen = set()
    for name, op, xin, Wt, extra, out_name, N, want in cases:
        slices = op.ks_slices()
        assert slices, f"{name}: layout 3 offers no slice count"
        cfgs = [(3, sl, 0) for sl in slices] + ([(4, 10, 0)] if op.sk_ok() else [])
        for cfg in cfgs:
            sl = cfg[1] if cfg[0] == 3 else "sk"
            seen.add((name, sl))

            def run():
                kw = {}
                if "nw" in extra:
                    kw["nw"] = extra["nw"]
                if out_name == "h":
                    kw["h"] = extra["h0"].clone()
                    res = kw["h"]
                else:
                    kw["y"] = torch.empty(M, N, device=dev, dtype=BF)
                    res = kw["y"]
                op(xin, Wt, cfg=cfg, **kw)
                return res, kw

            r1, _ = run()
            torch.cuda.synchronize()
            assert_bf16_close(r1.cpu(), want, max_ulp=2, max_frac=0.03, atol=one_ulp_at(want))
            r2, _ = run()
            torch.cuda.synchronize()
            assert torch.equal(r1, r2), f"{name} slices {sl}: not deterministic"
            # graph replays against the eager result
            s_ = torch.cuda.Stream()
            s_.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s_):
                run()
            torch.cuda.current_stream().wait_stream(s_)
            torch.cuda.synchronize()
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                r3, kw3 = run()
            for _ in range(3):
                if out_name == "h":
                    kw3["h"].copy_(extra["h0"])
                torch.cuda.synchronize()
                gr.replay()
                torch.cuda.synchronize()
                assert torch.equal(r3, r1), f"{name} slices {sl}: graph replay differs"
    assert {("o", 4), ("o", 8), ("down", 4), ("down", 19), ("qkv", 1), ("gu", 1), ("o", "sk"),
            ("down", "sk")} <= seen


@pytest.mark.parametrize("M,N,Kd", [(5, 200, 2560), (16, 1000, 2560), (3, 2568, 4096), (16, 48, 9728)])
def test_gemv_stream_k_shapes(dev, M, N, Kd):
    """Layout 4 beyond the model's shapes: N not a multiple of 16 (a part-filled
    last tile), tile counts whose chunks end inside a workgroup, grids smaller
    than the CUs, and K = 512 S for S = 5, 8, 19; BF16, F32 and RESID against the
    oracle, the same on a second call."""
    _, gemv = K()
    g = _g(dev, 110 + M + N)
    x = torch.randn(M, Kd, device=dev, generator=g).to(BF)
    W = _weights(dev, N, Kd, 111 + N)
    Wt = gemv.tile_weights(W)
    cfg = (4, 10, 0)
    for epi in (gemv.EPI_BF16, gemv.EPI_F32, gemv.EPI_RESID):
        op = gemv.Gemv(M, N, Kd, epi, norm=False)
        assert op.sk_ok() and cfg in op.candidates()
        outs = []
        for _ in range(2):
            if epi == gemv.EPI_RESID:
                h = torch.randn(M, N, device=dev, generator=_g(dev, 7)).to(BF)
                h0 = h.clone()
                op(x, Wt, h=h, cfg=cfg)
                outs.append(h)
            else:
                y = torch.empty(M, N, device=dev, dtype=torch.float32 if epi == gemv.EPI_F32 else BF)
                op(x, Wt, y=y, cfg=cfg)
                outs.append(y)
        torch.cuda.synchronize()
        assert torch.equal(outs[0], outs[1]), epi
        if epi == gemv.EPI_RESID:
            want, _ = O.gemv(x.cpu(), W.cpu(), O.EPI_RESID, h=h0.cpu())
            assert_bf16_close(outs[0].cpu(), want, max_ulp=2, max_frac=0.03, atol=one_ulp_at(want))
        elif epi == gemv.EPI_BF16:
            want = O.gemv(x.cpu(), W.cpu(), O.EPI_BF16)
            assert_bf16_close(outs[0].cpu(), want, max_ulp=2, max_frac=0.03, atol=one_ulp_at(want))
        else:
            want = O.gemv(x.cpu(), W.cpu(), O.EPI_F32)
            torch.testing.assert_close(outs[0].cpu(), want.float(), rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("M,N,Kd,cfg", [(20, 200, 2560, (4, 10, 2)), (32, 1000, 4096, (4, 10, 2)),
                                        (40, 2568, 9728, (4, 10, 2)), (40, 200, 2560, (4, 10, 4)),
                                        (64, 1000, 4096, (4, 10, 4)), (50, 2568, 9728, (4, 10, 4)),
                                        (20, 1000, 2560, (2, 1, 2)), (30, 200, 4096, (2, 2, 2))])
def test_gemv_row_tiles_odd_shapes(dev, M, N, Kd, cfg):
    """Two and four row tiles beyond the model's shapes: N not a multiple of 16 (a
    part-filled last tile), few tiles (grids smaller than the CUs, layout-4 chunks
    ending inside a workgroup), part-filled row tiles and 32/64-row slices followed
    by a shorter one. Each output equals the one-tile launch bit for bit and the
    oracle within the bf16 tolerance (F32, BF16, RESID; layout 2 also with the NORM
    prologue, its row norms computed in the kernel)."""
    _, gemv = K()
    one = (cfg[0], cfg[1], 0)
    g = _g(dev, 130 + M + N + cfg[2])
    x = torch.randn(M, Kd, device=dev, generator=g).to(BF)
    nw = (1 + 0.1 * torch.randn(Kd, device=dev, generator=g)).to(BF)
    W = _weights(dev, N, Kd, 131 + N)
    Wt = gemv.tile_weights(W)
    cases = [(gemv.EPI_F32, False), (gemv.EPI_BF16, False), (gemv.EPI_RESID, False)]
    if cfg[0] == 2:
        cases.append((gemv.EPI_F32, True))
    y_f32 = O.gemv(x.cpu(), W.cpu(), O.EPI_F32)
    for epi, norm in cases:
        op = gemv.Gemv(M, N, Kd, epi, norm=norm)
        assert cfg in op.candidates(), (epi, norm)
        kw = {"nw": nw} if norm else {}
        h0 = torch.randn(M, N, device=dev, generator=_g(dev, 9)).to(BF)
        outs = []
        for c in (cfg, one):
            if epi == gemv.EPI_RESID:
                h = h0.clone()
                op(x, Wt, h=h, cfg=c, **kw)
                outs.append(h)
            else:
                y = torch.empty(M, N, device=dev, dtype=torch.float32 if epi == gemv.EPI_F32 else BF)
                op(x, Wt, y=y, cfg=c, **kw)
                outs.append(y)
        torch.cuda.synchronize()
        assert torch.equal(outs[0], outs[1]), (epi, norm)
        got = outs[0].cpu()
        if norm:
            want = O.gemv(x.cpu(), W.cpu(), O.EPI_F32, nw=nw.cpu(), ss=x.cpu().float().pow(2).sum(-1))
            torch.testing.assert_close(got, want, rtol=2e-3, atol=2e-3)
        elif epi == gemv.EPI_RESID:
            want, _ = O.gemv(x.cpu(), W.cpu(), O.EPI_RESID, h=h0.cpu())
            assert_resid_close(got, want, y_f32)
        elif epi == gemv.EPI_BF16:
            want = O.gemv(x.cpu(), W.cpu(), O.EPI_BF16)
            assert_bf16_close(got, want, max_ulp=2, max_frac=0.03, atol=one_ulp_at(want))
        else:
            torch.testing.assert_close(got, y_f32.float(), rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("M,cfg", [(1, (1, 4, 2)), (1, (0, 8, 0)), (3, (1, 2, 4)), (3, (0, 8, 0)),
                                   (4, (0, 4, 0)), (16, (0, 8, 0)),
                                   (3, (2, 1, 0)), (16, (2, 2, 0)),
                                   (20, (2, 1, 2)), (32, (2, 2, 2))])
def test_lm_head_argmax_and_graph_replay(dev, M, cfg):
    _, gemv = K()
    V, H = 151936, 2560
    g = _g(dev, 30)
    E = _weights(dev, V, H, 31)
    x = torch.randn(M, H, device=dev, generator=g).to(BF)
    nw = (1 + 0.1 * torch.randn(H, device=dev, generator=g)).to(BF)
    op = gemv.Gemv(M, V, H, gemv.EPI_ARGMAX, norm=True)
    op.cfg = cfg
    Ew = gemv.tile_weights(E) if cfg[0] == 2 else E  # the GEMV's copy; E stays the table
    logits = torch.empty(M, V, device=dev, dtype=BF)
    ids = torch.empty(M, device=dev, dtype=torch.int64)
    pos = torch.arange(M, device=dev, dtype=torch.int32)
    nxt = torch.zeros(M, H, device=dev, dtype=BF)
    op(x, Ew, y=logits, nw=nw, ids=ids, pos_inc=pos, next_emb=E, next_h=nxt)
    torch.cuda.synchronize()
    assert torch.equal(pos.cpu(), torch.arange(M, dtype=torch.int32) + 1)
    assert torch.equal(nxt, E[ids])
    # self-consistent: ids is the first maximum of the kernel's own bf16 logits
    assert torch.equal(ids.cpu(), O.argmax_first(logits.cpu()))
    # close to the oracle, and the chosen logit is the oracle's maximum within 1 ulp
    want = O.gemv(x.cpu(), E.cpu(), O.EPI_BF16, nw=nw.cpu(), ss=x.cpu().float().pow(2).sum(-1))
    assert_bf16_close(logits.cpu(), want, max_frac=0.02, atol=one_ulp_at(want))
    wmax = want.float().max(-1).values
    picked = want.float().gather(1, ids.cpu()[:, None])[:, 0]
    assert torch.all(wmax - picked <= wmax.abs() * 2 ** -7)
    # graph replays reuse the cross-workgroup counter
    g2 = torch.cuda.CUDAGraph()
    ids2 = torch.zeros_like(ids)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        op(x, Ew, nw=nw, ids=ids2)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g2):
        op(x, Ew, nw=nw, ids=ids2)
    for _ in range(3):
        ids2.zero_()
        g2.replay()
        torch.cuda.synchronize()
        assert torch.equal(ids2, ids)


@pytest.mark.parametrize("M,cfg", [(1, (0, 8, 0)), (2, (1, 2, 4)), (4, (0, 4, 0)),
                                   (16, (2, 1, 0)), (20, (0, 8, 0)), (40, (2, 1, 2))])
def test_lm_head_step_tail(dev, M, cfg):
    """ko_lm_head_argmax: the LM head with the decode step's tail. The ids, logits,
    position advance and embedding gather equal ko_gemv's ARGMAX epilogue; the
    RoPE rows of the advanced positions equal rope_rows (and the table rows, the
    last position clamped to the table); the ids land in the pinned host ring at
    row ring_ctr[m], which advances and wraps, on eager calls and graph replays
    (M = 20 runs as two launch slices of 16 and 4 rows, M = 40 on two row tiles
    as slices of 32 and 8)."""
    fused, gemv = K()
    V, H, d, rows = 151936, 2560, 128, 40
    g = _g(dev, 50)
    E = _weights(dev, V, H, 51)
    x = torch.randn(M, H, device=dev, generator=g).to(BF)
    nw = (1 + 0.1 * torch.randn(H, device=dev, generator=g)).to(BF)
    op = gemv.Gemv(M, V, H, gemv.EPI_ARGMAX, norm=True)
    op.cfg = cfg
    Ew = gemv.tile_weights(E) if cfg[0] == 2 else E
    cos, sin = (t.to(dev) for t in O.rope_tables(rows, d))
    pos0 = torch.arange(M, dtype=torch.int32) * 2 + 5
    pos0[-1] = rows - 1          # advances past the table: the rows clamp to the last
    # the plain ARGMAX epilogue, then the step tail's separate pieces
    ids_a = torch.empty(M, device=dev, dtype=torch.int64)
    lg_a = torch.empty(M, V, device=dev, dtype=BF)
    pos_a = pos0.to(dev)
    nxt_a = torch.zeros(M, H, device=dev, dtype=BF)
    op(x, Ew, y=lg_a, nw=nw, ids=ids_a, pos_inc=pos_a, next_emb=E, next_h=nxt_a)
    rope_a = torch.empty(M, 2, d, device=dev, dtype=BF)
    fused.rope_rows(pos_a, cos, sin, rope_a)
    # the tail in one call
    R = 3
    ring = torch.full((R, M), -1, dtype=torch.int64, pin_memory=True)
    ctr = torch.ones(M, dtype=torch.int32, device=dev)
    ids_b = torch.empty(M, device=dev, dtype=torch.int64)
    lg_b = torch.empty(M, V, device=dev, dtype=BF)
    pos_b = pos0.to(dev)
    nxt_b = torch.zeros(M, H, device=dev, dtype=BF)
    rope_b = torch.zeros(M, 2, d, device=dev, dtype=BF)
    kw = dict(y=lg_b, nw=nw, ids=ids_b, pos_inc=pos_b, next_emb=E, next_h=nxt_b,
              rope=(cos, sin, rope_b), ring=(ring, ctr))
    op(x, Ew, **kw)
    torch.cuda.synchronize()
    assert torch.equal(ids_b, ids_a) and torch.equal(lg_b, lg_a) and torch.equal(nxt_b, nxt_a)
    assert torch.equal(pos_b, pos_a)
    assert torch.equal(rope_b, rope_a)
    p = pos_a.cpu().long().clamp(0, rows - 1)
    assert torch.equal(rope_b[:, 0].cpu(), cos.cpu()[p]) and torch.equal(rope_b[:, 1].cpu(), sin.cpu()[p])
    assert torch.equal(ring[1], ids_a.cpu()) and torch.equal(ring[0], torch.full((M,), -1))
    assert torch.equal(ctr.cpu(), torch.full((M,), 2, dtype=torch.int32))
    # graph replays: rows 2, then 0 (wrapped), then 1
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        op(x, Ew, **kw)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    ring.fill_(-1)
    ctr.fill_(2)
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        op(x, Ew, **kw)
    for want_row, want_ctr in ((2, 0), (0, 1), (1, 2)):
        ring[want_row].fill_(-1)
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(ring[want_row], ids_a.cpu()), want_row
        assert torch.equal(ctr.cpu(), torch.full((M,), want_ctr, dtype=torch.int32))


@pytest.mark.parametrize("M,N,ld", [(5, 151936, 151936), (3, 1003, 1008), (80, 4096, 4104)])
def test_argmax_rows_first_index_and_graph(dev, M, N, ld):
    """ko_argmax_rows against the first-maximum argmax; planted ties (the same
    maximum at two columns) take the lower column; rows with a stride; a tail of
    N % 8 columns; graph replays."""
    _, gemv = K()
    g = _g(dev, 40)
    buf = torch.randn(M, ld, device=dev, generator=g).to(BF)
    x = buf[:, :N]
    lo = torch.randint(0, N // 2, (M,), generator=torch.Generator().manual_seed(41))
    hi = torch.randint(N // 2, N, (M,), generator=torch.Generator().manual_seed(42))
    for m in range(M):
        if m % 2 == 0:
            x[m, lo[m]] = 8.0
            x[m, hi[m]] = 8.0
        else:
            x[m, hi[m]] = 8.0   # the maximum alone (in the tail when N % 8 != 0)
    want = O.argmax_first(x.cpu())
    assert all(int(want[m]) == (lo[m] if m % 2 == 0 else hi[m]) for m in range(M))
    ids = torch.full((M,), -1, device=dev, dtype=torch.int64)
    gemv.argmax_rows(x, ids)
    torch.cuda.synchronize()
    assert torch.equal(ids.cpu(), want)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        gemv.argmax_rows(x, ids)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        gemv.argmax_rows(x, ids)
    for _ in range(3):
        ids.fill_(-1)
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(ids.cpu(), want)


@pytest.mark.parametrize("rows,swiglu", [(37, False), (64, True)])
def test_tile_weights_layout(dev, rows, swiglu):
    """ko_gemv_tile against the layout written out with torch: rows padded to 16,
    then [tile][32-column step][k group][row in tile][8 columns]."""
    _, gemv = K()
    Kd = 96
    W = torch.randn(rows, Kd, device=dev, generator=_g(dev, 40)).to(BF)
    got = gemv.tile_weights(W, swiglu=swiglu)

    def ref(part):
        n = part.shape[0]
        npad = -(-n // 16) * 16
        p = torch.zeros(npad, Kd, dtype=BF)
        p[:n] = part.cpu()
        return p.view(npad // 16, 16, Kd // 32, 4, 8).permute(0, 2, 3, 1, 4).reshape(npad, Kd)

    halves = [W[: rows // 2], W[rows // 2:]] if swiglu else [W]
    want = torch.cat([ref(h) for h in halves])
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), want)


def test_gemv_rejects_bad_shapes(dev):
    _, gemv = K()
    op = gemv.Gemv(1, 64, 128, gemv.EPI_BF16, norm=False)
    x = torch.zeros(1, 128, device=dev, dtype=BF)
    w = torch.zeros(64, 128, device=dev, dtype=BF)
    with pytest.raises(ValueError):
        op(x, w, y=torch.zeros(1, 64, device=dev))          # wrong dtype
    with pytest.raises(ValueError):
        op(x, w[:32], y=torch.zeros(1, 64, device=dev, dtype=BF))
