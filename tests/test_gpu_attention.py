"""GPU parity of the HIP split-K GQA decode attention against the CPU oracle
(engine/kernels/fused.py:138-234 semantics). Tolerance: atol = rtol = 2e-2
against fp32/fp64 references, bf16 inputs."""

import pytest
import torch

from oracle import attention as A

pytestmark = pytest.mark.gpu

TOL = dict(rtol=2e-2, atol=2e-2)


def _fused():
    from kernel_optim_amd.kernels import fused
    return fused


def _inputs(B, T, cap, dev, seeds=(0, 1, 2), nq=32, nkv=8, D=128):
    gq, gk, gv = (torch.Generator(device=dev).manual_seed(s) for s in seeds)
    q = torch.randn(B * T, nq * D, device=dev, generator=gq).to(torch.bfloat16)
    k = torch.randn(B, nkv, cap, D, device=dev, generator=gk).to(torch.bfloat16)
    v = torch.randn(B, nkv, cap, D, device=dev, generator=gv).to(torch.bfloat16)
    return q, k, v


def _gpu_ref_fp32(q, k, v, lens, T=1):
    """Plain PyTorch fp32 attention on the GPU (per sequence, GQA by grouping)."""
    B, nkv, cap, D = k.shape
    nq = q.shape[1] // D
    out = torch.empty(B * T, nq * D, device=q.device, dtype=torch.float32)
    qv = q.float().view(B, T, nkv, nq // nkv, D)
    for b in range(B):
        L = int(lens[b])
        kk = k[b, :, :L].float()                               # [nkv, L, D]
        vv = v[b, :, :L].float()
        qq = qv[b].permute(1, 0, 2, 3).reshape(nkv, -1, D).contiguous()   # [nkv, T*4, D]
        s = torch.bmm(qq, kk.transpose(1, 2).contiguous()) * D ** -0.5    # [nkv, T*4, L]
        s = s.view(nkv, T, nq // nkv, L)
        keys = torch.arange(L, device=q.device)
        for t in range(T):
            s[:, t, :, keys > L - T + t] = float("-inf")
        p = torch.softmax(s.view(nkv, -1, L), dim=-1)
        o = torch.bmm(p, vv).view(nkv, T, nq // nkv, D).permute(1, 0, 2, 3)
        out.view(B, T, nq, D)[b] = o.reshape(T, nq, D)
    return out


def test_config1_b1_ctx512(dev):
    """Config 1 shape: B=1, 32q/8kv, d=128, ctx 512, seeds q=0 k=1 v=2."""
    fused = _fused()
    q, k, v = _inputs(1, 1, 512, dev)
    pos = torch.tensor([511], dtype=torch.int32, device=dev)
    out = torch.empty_like(q)
    att = fused.DecodeAttention(1, 1, 512, 32, 8, 128, dev)
    att(q, k, v, pos, out)
    torch.cuda.synchronize()
    want = A.decode_attention(q.cpu(), k.cpu(), v.cpu(), [512])
    torch.testing.assert_close(out.cpu().double(), want, **TOL)


@pytest.mark.parametrize("unit", [16, 64, 512])
def test_ragged_small_against_oracle(dev, unit):
    fused = _fused()
    B, cap = 6, 320
    q, k, v = _inputs(B, 1, cap, dev, seeds=(4, 5, 6))
    lens = [1, 15, 16, 17, 300, 320]
    pos = torch.tensor([x - 1 for x in lens], dtype=torch.int32, device=dev)
    out = torch.empty_like(q)
    att = fused.DecodeAttention(B, 1, cap, 32, 8, 128, dev, unit=unit)
    att(q, k, v, pos, out)
    torch.cuda.synchronize()
    want = A.decode_attention(q.cpu(), k.cpu(), v.cpu(), lens)
    torch.testing.assert_close(out.cpu().double(), want, **TOL)


@pytest.mark.parametrize("fused_combine", [False, True])
@pytest.mark.parametrize("T", [2, 3, 4, 5, 6, 7, 8])
def test_multi_token_causal(dev, T, fused_combine):
    """T query tokens per sequence, causal within the block (the verify step of
    speculative decoding); T > 4 runs as two launches of 2-4 tokens."""
    fused = _fused()
    B, cap = 3, 200
    q, k, v = _inputs(B, T, cap, dev, seeds=(7, 8, 9))
    first = [0, 37, 200 - T]
    pos = torch.tensor(first, dtype=torch.int32, device=dev)
    att = fused.DecodeAttention(B, T, cap, 32, 8, 128, dev, unit=32, fused_combine=fused_combine)
    want = A.decode_attention(q.cpu(), k.cpu(), v.cpu(), [p + T for p in first], T=T)
    for _ in range(2):  # the fused combine's counters re-arm between launches
        out = torch.zeros_like(q)
        att(q, k, v, pos, out)
        torch.cuda.synchronize()
        torch.testing.assert_close(out.cpu().double(), want, **TOL)
    if fused_combine:
        assert torch.all(att.counters == 0)


@pytest.mark.parametrize("B,T", [(1, 2), (1, 5), (1, 7), (3, 3), (3, 8), (12, 6)])
def test_token_rows_causal(dev, B, T):
    """The T tokens of each sequence as B*T rows of the one-token kernel
    (ko_decode_attn_token_rows): row b*T + t sees keys 0..pos[b]+t. Against the
    oracle's causal T-token attention; B*T = 72 takes the past-64-rows lookup."""
    fused = _fused()
    cap = 300
    q, k, v = _inputs(B, T, cap, dev, seeds=(40, 41, 42))
    g = torch.Generator().manual_seed(43)
    first = torch.randint(0, cap - T + 1, (B,), generator=g).tolist()
    first[0] = 0
    pos = torch.tensor(first, dtype=torch.int32, device=dev)
    att = fused.DecodeAttention(B, T, cap, 32, 8, 128, dev, fused_combine=True, token_rows=True)
    want = A.decode_attention(q.cpu(), k.cpu(), v.cpu(), [p + T for p in first], T=T)
    for _ in range(2):  # the counters re-arm between launches
        out = torch.zeros_like(q)
        att(q, k, v, pos, out)
        torch.cuda.synchronize()
        torch.testing.assert_close(out.cpu().double(), want, **TOL)
    assert torch.all(att.counters == 0)


def test_config2_b16_ctx8192(dev):
    """Config 2: B=16 x 8192, against fp32 torch on the GPU for every sequence and
    the fp64 CPU oracle for four of them."""
    fused = _fused()
    B, cap = 16, 8192
    q, k, v = _inputs(B, 1, cap, dev)
    pos = torch.full((B,), cap - 1, dtype=torch.int32, device=dev)
    out = torch.empty_like(q)
    att = fused.DecodeAttention(B, 1, cap, 32, 8, 128, dev)
    att(q, k, v, pos, out)
    torch.cuda.synchronize()
    ref = _gpu_ref_fp32(q, k, v, [cap] * B)
    torch.testing.assert_close(out.float(), ref, **TOL)
    sel = [0, 5, 10, 15]
    want = A.decode_attention(q.view(B, -1)[sel].cpu(), k[sel].cpu(), v[sel].cpu(), [cap] * 4)
    torch.testing.assert_close(out.view(B, -1)[sel].cpu().double(), want, **TOL)
    # the same op with the merge in the partial launch (as the engine and the
    # benchmark run it): bit-identical, on repeated launches
    attf = fused.DecodeAttention(B, 1, cap, 32, 8, 128, dev, fused_combine=True)
    for _ in range(3):
        outf = torch.zeros_like(q)
        attf(q, k, v, pos, outf)
        torch.cuda.synchronize()
        assert torch.equal(outf, out)
    assert torch.all(attf.counters == 0)


def test_config3_ragged_padded_tail_unread(dev):
    """Config 3: B=64, lengths ~ U[128, 16384] (seed 3), cache padded to 16384. The
    padded tail is filled with NaN: reading any of it would poison the output."""
    fused = _fused()
    B, cap = 64, 16384
    g = torch.Generator().manual_seed(3)
    lens = torch.randint(128, cap + 1, (B,), generator=g, dtype=torch.int32)
    q, k, v = _inputs(B, 1, cap, dev, seeds=(10, 11, 12))
    for b in range(B):
        k[b, :, int(lens[b]):] = float("nan")
        v[b, :, int(lens[b]):] = float("nan")
    out = torch.empty_like(q)
    att = fused.DecodeAttention(B, 1, cap, 32, 8, 128, dev)
    att.with_lengths(q, k, v, lens.to(dev), out)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    ref = _gpu_ref_fp32(q, k, v, lens.tolist())
    torch.testing.assert_close(out.float(), ref, **TOL)


@pytest.mark.parametrize("fused_combine", [False, True])
def test_long_context_65536(dev, fused_combine):
    """Two sequences of 65536 and 40001 keys in a 65536-slot cache (the sizing rule
    then takes 2048-key units, 32 per KV head) against fp32 attention; the unused
    tail of the shorter sequence is NaN, so reading it would poison the output."""
    fused = _fused()
    B, cap = 2, 65536
    lens = torch.tensor([65536, 40001], dtype=torch.int32)
    q, k, v = _inputs(B, 1, cap, dev, seeds=(20, 21, 22))
    k[1, :, 40001:] = float("nan")
    v[1, :, 40001:] = float("nan")
    out = torch.empty_like(q)
    att = fused.DecodeAttention(B, 1, cap, 32, 8, 128, dev, fused_combine=fused_combine)
    att.with_lengths(q, k, v, lens.to(dev), out)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    ref = _gpu_ref_fp32(q, k, v, lens.tolist())
    torch.testing.assert_close(out.float(), ref, **TOL)
    if fused_combine:
        assert torch.all(att.counters == 0)


@pytest.mark.parametrize("fused_combine", [False, True])
def test_more_than_64_sequences(dev, fused_combine):
    """B = 130: the pair lookup past one wavefront's 64 lengths (three chunks of
    lengths, the last partly filled), ragged lengths in 1..640, NaN beyond each."""
    fused = _fused()
    B, cap = 130, 640
    g = torch.Generator().manual_seed(31)
    lens = torch.randint(1, cap + 1, (B,), generator=g, dtype=torch.int32)
    lens[0], lens[64], lens[129] = 1, cap, 17
    q, k, v = _inputs(B, 1, cap, dev, seeds=(32, 33, 34))
    for b in range(B):
        k[b, :, int(lens[b]):] = float("nan")
        v[b, :, int(lens[b]):] = float("nan")
    out = torch.empty_like(q)
    att = fused.DecodeAttention(B, 1, cap, 32, 8, 128, dev, fused_combine=fused_combine)
    att.with_lengths(q, k, v, lens.to(dev), out)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    torch.testing.assert_close(out.float(), _gpu_ref_fp32(q, k, v, lens.tolist()), **TOL)


def test_deterministic_and_unit_invariant(dev):
    fused = _fused()
    B, cap = 4, 3000
    q, k, v = _inputs(B, 1, cap, dev, seeds=(13, 14, 15))
    pos = torch.tensor([2999, 100, 2048, 1500], dtype=torch.int32, device=dev)
    outs = []
    for unit in (64, 256, 1024):
        att = fused.DecodeAttention(B, 1, cap, 32, 8, 128, dev, unit=unit)
        o1, o2 = torch.empty_like(q), torch.empty_like(q)
        att(q, k, v, pos, o1)
        att(q, k, v, pos, o2)
        torch.cuda.synchronize()
        assert torch.equal(o1, o2)
        outs.append(o1.float())
    for o in outs[1:]:
        torch.testing.assert_close(o, outs[0], **TOL)


def test_graph_replay_tracks_device_positions(dev):
    fused = _fused()
    B, cap = 2, 1024
    q, k, v = _inputs(B, 1, cap, dev, seeds=(16, 17, 18))
    pos = torch.tensor([10, 500], dtype=torch.int32, device=dev)
    out = torch.zeros_like(q)
    att = fused.DecodeAttention(B, 1, cap, 32, 8, 128, dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        att(q, k, v, pos, out)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        att(q, k, v, pos, out)
    for p in ([10, 500], [700, 3], [1023, 1023]):
        pos.copy_(torch.tensor(p, dtype=torch.int32))
        g.replay()
        torch.cuda.synchronize()
        eager = torch.empty_like(q)
        att(q, k, v, pos, eager)
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        want = A.decode_attention(q.cpu(), k.cpu(), v.cpu(), [x + 1 for x in p])
        torch.testing.assert_close(out.cpu().double(), want, **TOL)


def test_bad_arguments_raise_before_launch(dev):
    fused = _fused()
    q, k, v = _inputs(1, 1, 64, dev)
    att = fused.DecodeAttention(1, 1, 64, 32, 8, 128, dev)
    pos = torch.tensor([3], dtype=torch.int32, device=dev)
    with pytest.raises(ValueError):
        att(q, k, v, pos.long(), torch.empty_like(q))
    with pytest.raises(ValueError):
        att(q.float(), k, v, pos, torch.empty_like(q))
    with pytest.raises(ValueError):
        att(q, k[:, :, :32], v, pos, torch.empty_like(q))


@pytest.mark.parametrize("fused", [False, True])
def test_two_launch_and_fused_combine_agree(dev, fused):
    fused_mod = _fused()
    B, cap = 5, 700
    q, k, v = _inputs(B, 1, cap, dev, seeds=(19, 20, 21))
    pos = torch.tensor([699, 0, 63, 64, 350], dtype=torch.int32, device=dev)
    att = fused_mod.DecodeAttention(B, 1, cap, 32, 8, 128, dev, unit=64, fused_combine=fused)
    out = torch.empty_like(q)
    for _ in range(3):  # counters must re-arm between launches
        att(q, k, v, pos, out)
        torch.cuda.synchronize()
        want = A.decode_attention(q.cpu(), k.cpu(), v.cpu(), [int(p) + 1 for p in pos])
        torch.testing.assert_close(out.cpu().double(), want, **TOL)
    if fused:
        assert torch.all(att.counters == 0)


@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("B,cap,unit", [(1, 1300, 64), (4, 600, 128), (16, 256, 64)])
def test_decode_qkv_matches_norm_rope_append_then_attention(dev, B, cap, unit, fused):
    """decode_qkv = qk_norm_rope (fused.py:54-96) then attention over keys 0..pos."""
    from oracle import ops as O
    fused_mod = _fused()
    nq, nkv, d = 32, 8, 128
    g = torch.Generator(device=dev).manual_seed(40 + B)
    qkv = torch.randn(B, (nq + 2 * nkv) * d, device=dev, generator=g).to(torch.bfloat16)
    qw = (1 + 0.2 * torch.randn(d, device=dev, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.2 * torch.randn(d, device=dev, generator=g)).to(torch.bfloat16)
    cos, sin = (t.to(dev) for t in O.rope_tables(cap, d, 1.0e6))
    k = torch.randn(B, nkv, cap, d, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(B, nkv, cap, d, device=dev, generator=g).to(torch.bfloat16)
    pos = torch.randint(0, cap, (B,), device=dev, generator=g).to(torch.int32)
    pos[0] = cap - 1
    if B > 1:
        pos[1] = 0
    kref, vref = k.cpu(), v.cpu()
    qref = O.qk_norm_rope(qkv.cpu(), qw.cpu(), kw.cpu(), cos.cpu(), sin.cpu(), pos.cpu(), kref,
                          vref, 1, 1e-6, nq, nkv, d)
    want = A.decode_attention(qref, kref, vref, [int(p) + 1 for p in pos])
    att = fused_mod.DecodeAttention(B, 1, cap, nq, nkv, d, dev, unit=unit, fused_combine=fused)
    out = torch.empty(B, nq * d, device=dev, dtype=torch.bfloat16)
    att.decode_qkv(qkv, qw, kw, cos, sin, pos, k, v, out, 1e-6)
    if fused:
        assert torch.all(att.counters == 0)
    torch.cuda.synchronize()
    torch.testing.assert_close(out.cpu().double(), want, **TOL)
    # the appended slot holds the normed+roped k and the raw v; nothing else changed
    from tests.bf16util import assert_bf16_close
    assert_bf16_close(k.cpu(), kref, max_frac=1e-3)
    assert torch.equal(v.cpu(), vref)


@pytest.mark.parametrize("B,cap,split", [(3, 1300, 10), (16, 1296, 2), (16, 700, 5),
                                         (64, 600, 1), (2, 2100, 16)])
def test_decode_qkv_units_per_seq(dev, B, cap, split):
    """decode_qkv with each sequence's keys cut into at most `split` equal units from
    its length at the step (units_per_seq): the oracle's qk_norm_rope then
    attention over keys 0..pos, with ragged positions (the last slot, slot 0, 63,
    64, random), over three graph-replayed steps whose positions advance; the
    arrival counters re-arm every step."""
    from oracle import ops as O
    from tests.bf16util import assert_bf16_close
    fused_mod = _fused()
    nq, nkv, d = 32, 8, 128
    g = torch.Generator(device=dev).manual_seed(90 + B + split)
    qkv = torch.randn(B, (nq + 2 * nkv) * d, device=dev, generator=g).to(torch.bfloat16)
    qw = (1 + 0.2 * torch.randn(d, device=dev, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.2 * torch.randn(d, device=dev, generator=g)).to(torch.bfloat16)
    cos, sin = (t.to(dev) for t in O.rope_tables(cap, d, 1.0e6))
    k = torch.randn(B, nkv, cap, d, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(B, nkv, cap, d, device=dev, generator=g).to(torch.bfloat16)
    steps = 3
    pos = torch.randint(0, cap - steps, (B,), device=dev, generator=g).to(torch.int32)
    for i, p0 in enumerate((cap - steps, 0, 62, 63)[:B]):
        pos[i] = p0
    att = fused_mod.DecodeAttention(B, 1, cap, nq, nkv, d, dev, fused_combine=True,
                                    units_per_seq=split)
    out = torch.empty(B, nq * d, device=dev, dtype=torch.bfloat16)
    kref, vref = k.cpu(), v.cpu()
    pos_h = pos.cpu().clone()

    def step():
        att.decode_qkv(qkv, qw, kw, cos, sin, pos, k, v, out, 1e-6)
        pos.add_(1)
    s_ = torch.cuda.Stream()
    s_.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s_):
        step()
    torch.cuda.current_stream().wait_stream(s_)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for j in range(steps):
        if j:
            graph.replay()
        torch.cuda.synchronize()
        p = pos_h + j
        qref = O.qk_norm_rope(qkv.cpu(), qw.cpu(), kw.cpu(), cos.cpu(), sin.cpu(), p, kref, vref,
                              1, 1e-6, nq, nkv, d)
        want = A.decode_attention(qref, kref, vref, [int(x) + 1 for x in p])
        torch.testing.assert_close(out.cpu().double(), want, **TOL)
        assert torch.all(att.counters == 0)
    assert_bf16_close(k.cpu(), kref, max_frac=1e-3)
    assert torch.equal(v.cpu(), vref)


def test_rope_rows_are_the_table_rows(dev):
    """rope_rows copies cos[p], sin[p] for each sequence's position, with p clamped
    to the table."""
    from oracle import ops as O
    fused_mod = _fused()
    cos, sin = (t.to(dev) for t in O.rope_tables(300, 128, 1.0e6))
    pos = torch.tensor([0, 17, 299, 4000, -3], dtype=torch.int32, device=dev)
    out = torch.full((5, 2, 128), 7.0, device=dev, dtype=torch.bfloat16)
    fused_mod.rope_rows(pos, cos, sin, out)
    torch.cuda.synchronize()
    p = pos.clamp(0, 299).long()
    assert torch.equal(out[:, 0], cos[p]) and torch.equal(out[:, 1], sin[p])


@pytest.mark.parametrize("B,cap,pos0,unit", [(1, 1296, 1024, None), (1, 1296, 0, None),
                                             (1, 1296, 1295, None), (1, 1296, 700, 256),
                                             (1, 8192, 5000, 1024), (2, 640, 517, None)])
def test_decode_qkv_with_rope_rows_is_bit_equal(dev, B, cap, pos0, unit):
    """The attention with the step's RoPE rows passed in (and, at B = 1, its first
    loads issued before the position is read, keys clamped to the cache) equals
    the table-lookup path bit for bit: output, appended K and V."""
    from oracle import ops as O
    fused_mod = _fused()
    nq, nkv, d = 32, 8, 128
    g = torch.Generator(device=dev).manual_seed(70 + B + pos0)
    qkv = torch.randn(B, (nq + 2 * nkv) * d, device=dev, generator=g).to(torch.bfloat16)
    qw = (1 + 0.2 * torch.randn(d, device=dev, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.2 * torch.randn(d, device=dev, generator=g)).to(torch.bfloat16)
    cos, sin = (t.to(dev) for t in O.rope_tables(cap, d, 1.0e6))
    k0 = torch.randn(B, nkv, cap, d, device=dev, generator=g).to(torch.bfloat16)
    v0 = torch.randn(B, nkv, cap, d, device=dev, generator=g).to(torch.bfloat16)
    pos = torch.tensor([pos0, max(pos0 - 300, 0)][:B], dtype=torch.int32, device=dev)
    res = []
    for use_rope in (False, True):
        att = fused_mod.DecodeAttention(B, 1, cap, nq, nkv, d, dev, unit=unit, fused_combine=True)
        k, v = k0.clone(), v0.clone()
        out = torch.zeros(B, nq * d, device=dev, dtype=torch.bfloat16)
        rope = None
        if use_rope:
            rope = torch.empty(B, 2, d, device=dev, dtype=torch.bfloat16)
            fused_mod.rope_rows(pos, cos, sin, rope)
        att.decode_qkv(qkv, qw, kw, cos, sin, pos, k, v, out, 1e-6, rope=rope)
        torch.cuda.synchronize()
        assert torch.all(att.counters == 0)
        res.append((out.cpu(), k.cpu(), v.cpu()))
    for a, b in zip(*res):
        assert torch.equal(a, b)


@pytest.mark.parametrize("B,cap,pos0", [(1, 1296, 1024), (1, 1296, 0), (2, 640, 517)])
def test_decode_qkv_oproj_equals_attention_then_o_gemv(dev, B, cap, pos0):
    """The one-launch attention + o projection equals decode_qkv followed by the RESID
    GEMV (engine.py:328-331) bit for bit -- same merged attention rows, same
    dot-product order -- including the KV append, over several graph replays whose
    positions advance (the launch re-arms its counters every time). The one-launch
    side takes the step's RoPE rows from rope_rows (inside the graph, as the
    engine does), the other the tables."""
    from oracle import ops as O
    from kernel_optim_amd.kernels import gemv as GV
    fused_mod = _fused()
    nq, nkv, d, H = 32, 8, 128, 2560
    g = torch.Generator(device=dev).manual_seed(60 + B)
    qkv = torch.randn(B, (nq + 2 * nkv) * d, device=dev, generator=g).to(torch.bfloat16)
    qw = (1 + 0.2 * torch.randn(d, device=dev, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.2 * torch.randn(d, device=dev, generator=g)).to(torch.bfloat16)
    cos, sin = (t.to(dev) for t in O.rope_tables(cap, d, 1.0e6))
    k0 = torch.randn(B, nkv, cap, d, device=dev, generator=g).to(torch.bfloat16)
    v0 = torch.randn(B, nkv, cap, d, device=dev, generator=g).to(torch.bfloat16)
    w_o = (0.02 * torch.randn(H, nq * d, device=dev, generator=g)).to(torch.bfloat16)
    h0 = torch.randn(B, H, device=dev, generator=g).to(torch.bfloat16)
    pos_start = torch.tensor([pos0, max(pos0 - 300, 0)][:B], dtype=torch.int32, device=dev)

    def run(fused_launch, steps):
        k, v, h = k0.clone(), v0.clone(), h0.clone()
        pos = pos_start.clone()
        att = fused_mod.DecodeAttention(B, 1, cap, nq, nkv, d, dev, fused_combine=True)
        o = GV.Gemv(B, H, nq * d, GV.EPI_RESID, norm=False)
        out = torch.zeros(B, nq * d, device=dev, dtype=torch.bfloat16)
        rope = torch.zeros(B, 2, d, device=dev, dtype=torch.bfloat16)

        def step():
            if fused_launch:
                fused_mod.rope_rows(pos, cos, sin, rope)
                att.decode_qkv_oproj(qkv, qw, kw, cos, sin, pos, k, v, out, 1e-6, w_o, h,
                                     rope=rope)
            else:
                att.decode_qkv(qkv, qw, kw, cos, sin, pos, k, v, out, 1e-6)
                o(out, w_o, h=h, cfg=(0, 8, 0))
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
        assert torch.all(att.counters == 0)
        if fused_launch:
            # every group word holds (launches so far, 0 workgroups started)
            words = att.sync[32:].view(32, 32)[:, 16:18].cpu()
            assert torch.all(words[:, 0] == 0) and torch.all(words[:, 1] == steps), words
        assert int(att.err.item()) == 0, "the o projection's wait gave up"
        return out.cpu(), h.cpu(), k.cpu(), v.cpu()

    want = run(False, 4)
    got = run(True, 4)
    for name, a, b in zip(("out", "h", "k", "v"), got, want):
        assert torch.equal(a, b), name
