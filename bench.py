#!/usr/bin/env python3
"""Benchmark of the split-K GQA decode-attention hot path on one MI355X.

Workload (one "step"): one decode-attention call at Qwen3-4B layer shape,
B=16 sequences x 8192 cached keys, 32 query / 8 KV heads, head_dim 128, bf16,
contiguous KV cache [16, 8, 8192, 128] with seeded N(0,1) values; the split-K
partial kernel plus the log-sum-exp combine. Three KV buffers (1.6 GB) are
rotated so the 256 MB Infinity Cache cannot serve a step from the previous
one. Inputs are resident in HBM before the timed region starts.

Prints one JSON line: value = algorithmic HBM GB/s (K+V of every valid key +
q + out) over the timed steps; ``roofline`` for the dominant kernel
(the split-K partial kernel) timed with HIP events on its launch stream;
``cpu_baseline`` = the reference's CPU path (torch SDPA in bf16, as
Transformers' sdpa attention runs it) on the same workload, timed on the host.
``decode_b1`` = the metric's second half: Qwen3-4B-architecture greedy decode
tok/s at batch 1 (prompt 1024, 256 new tokens) against the weight-streaming
roofline, with its own CPU baseline (Transformers' Qwen3ForCausalLM on the
host, same weights and prompt). ``decode_b16`` = the same at batch 16;
``layer_2048`` = one decoder layer at 2048 cached keys, batch 1, 4 and 16;
``attention_ragged_b64`` = ragged decode attention at batch 64.
"""

import argparse
import json
import os
import sys
import time

METRIC = "decode-attn HBM GB/s (% of peak) @B16×8K ctx; Qwen3-4B-arch decode tok/s @B1"
PEAK_HBM_GBS = 8000.0
B, NQ, NKV, D, CTX = 16, 32, 8, 128, 8192


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-decode", action="store_true", help="skip the B1 decode measurement")
    ap.add_argument("--no-attn", action="store_true",
                    help="skip the attention measurement (profiling the decode step alone)")
    ap.add_argument("--no-ragged", action="store_true",
                    help="skip the ragged B=64 attention measurement (profiling B16 x 8K alone)")
    ap.add_argument("--prompt", type=int, default=1024)
    ap.add_argument("--new-tokens", type=int, default=256)
    ap.add_argument("--no-decode-b16", action="store_true",
                    help="skip the B=16 decode measurement (same workload at batch 16)")
    ap.add_argument("--no-layer", action="store_true",
                    help="skip the one-layer measurement (B=1, 4, 16 with 2048 cached keys)")
    ap.add_argument("--decode-batches", default="",
                    help="comma-separated further batch sizes of the same decode workload "
                         "(e.g. 32,64), reported as decode_b<B>; not in the default run")
    ap.add_argument("--spec", action="store_true",
                    help="also measure B=1 decode with prompt-lookup speculation (the same "
                         "random prompt, and a prompt of a repeated 64-token pattern)")
    return ap.parse_args()


PMC_SUMMARY = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                           "attn_kernel_b16_ctx8192_pmc.json")


def pmc_traffic():
    """HBM bytes per launch of the partial kernel from the committed FETCH_SIZE /
    WRITE_SIZE summary (two rocprofv3 --pmc passes, calibrated on a 1 GiB copy)."""
    try:
        with open(PMC_SUMMARY) as f:
            return json.load(f)["traffic_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def attn_bytes():
    return 2 * B * NKV * CTX * D * 2 + 2 * B * NQ * D * 2


def cpu_baseline(seconds):
    """The reference's CPU path for this attention call: torch SDPA in bf16, the
    call Transformers' sdpa attention makes for a decode step (one query token,
    enable_gqa), on the full workload (B=16 x 8192 keys, the same shapes and
    seeded N(0,1) values as the GPU leg), repeated for about ``seconds``; GB/s of
    the same algorithmic bytes."""
    import torch
    import torch.nn.functional as F
    g = torch.Generator().manual_seed(0)
    q = torch.randn(B, NQ, 1, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, NKV, CTX, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, NKV, CTX, D, generator=g).to(torch.bfloat16)
    F.scaled_dot_product_attention(q, k, v, scale=D ** -0.5, enable_gqa=True)  # warm
    n, t0 = 0, time.perf_counter()
    while True:
        F.scaled_dot_product_attention(q, k, v, scale=D ** -0.5, enable_gqa=True)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return {
        "value": round(attn_bytes() * n / el / 1e9, 3),
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "reference",
        "sample": f"torch scaled_dot_product_attention, bf16, enable_gqa (Transformers' sdpa "
                  f"decode attention), the full B=16 x 8192-key workload, {n} calls in {el:.1f} s; "
                  f"{torch.get_num_threads()} threads, affinity {len(os.sched_getaffinity(0))} cpus",
    }


def hf_qwen3_cpu(cfg, w):
    """Transformers' Qwen3ForCausalLM (sdpa attention) on the CPU in bf16 with the
    given decode-layout weights (kernel_optim_amd.model.to_hf_state_dict): built
    on the meta device and given the weights in place, so no random init runs."""
    import torch
    from transformers import Qwen3Config as HC, Qwen3ForCausalLM
    from kernel_optim_amd.model import to_hf_state_dict
    hc = HC(hidden_size=cfg.hidden, intermediate_size=cfg.inter, num_hidden_layers=cfg.layers,
            num_attention_heads=cfg.nq, num_key_value_heads=cfg.nkv, head_dim=cfg.head_dim,
            vocab_size=cfg.vocab, rms_norm_eps=cfg.eps, rope_theta=cfg.theta,
            tie_word_embeddings=cfg.tied, max_position_embeddings=40960,
            attn_implementation="sdpa")
    with torch.device("meta"):
        m = Qwen3ForCausalLM(hc)
    m = m.to_empty(device="cpu").to(torch.bfloat16)
    missing, unexpected = m.load_state_dict(to_hf_state_dict(cfg, w), strict=False, assign=True)
    assert not unexpected and all(k == "lm_head.weight" for k in missing), (missing, unexpected)
    if cfg.tied:
        m.lm_head.weight = m.model.embed_tokens.weight
    m.model.rotary_emb.__init__(hc)  # its inv_freq buffer was left on the meta device
    return m.eval()


def bench_decode(args, eng=None, B=1):
    """Qwen3-4B architecture (36 layers, random N(0,0.02) bf16 weights, seed 0),
    batch B, prompts of seeded uniform-random ids, greedy decode of ``new_tokens``
    through Engine.generate (hipGraph step, pipelined replays). tok/s counts the
    decode steps after the first token (which comes from the prefill), over all
    B sequences."""
    import torch
    from kernel_optim_amd.engine import Engine
    eng = eng or Engine("random")
    cfg = eng.cfg
    S, N = args.prompt, args.new_tokens
    prompt = torch.randint(0, cfg.vocab, (B, S), generator=torch.Generator().manual_seed(0)).tolist()
    for _ in eng.generate(prompt, N):      # setup, tuning, capture, warm-up
        pass
    torch.cuda.synchronize()
    t0 = None
    steps = []
    for i, toks in enumerate(eng.generate(prompt, N)):
        if i == 0:
            t0 = time.perf_counter()
        steps.append(toks)
    el = time.perf_counter() - t0
    out = [t[0] for t in steps]
    tok_s = B * (N - 1) / el
    step_ms = eng.time_step(min(50, N - 1))
    kv_per_key = cfg.layers * 2 * cfg.nkv * cfg.head_dim * 2
    avg_keys = S + 1 + (N - 2) / 2.0            # keys read by decode steps 1..N-1
    step_bytes = cfg.weight_bytes_per_step() + B * (kv_per_key * avg_keys + kv_per_key)
    roof_tok_s = B * PEAK_HBM_GBS * 1e9 / step_bytes
    res = {
        "workload": f"Qwen3-4B architecture greedy decode, B={B}, prompt {S}, {N} new tokens, "
                    "random-init bf16 weights (seed 0), hipGraph decode step",
        "tok_s": round(tok_s, 2),
        "ms_per_token": round(1e3 / tok_s, 4),
        "graph_step_ms": round(step_ms, 4),
        "bytes_per_step": int(step_bytes),
        "roofline": {"bound": "hbm", "tok_s_at_peak": round(roof_tok_s, 1),
                     "frac": round(tok_s / roof_tok_s, 4),
                     # weights alone (the KV cache reads left out of the bytes)
                     "weights_only_frac": round(
                         tok_s / (B * PEAK_HBM_GBS * 1e9 / cfg.weight_bytes_per_step()), 4),
                     "achieved_gbs": round(step_bytes * tok_s / B / 1e9, 1),
                     "graph_step_frac": round((step_bytes / (step_ms * 1e-3) / 1e9) / PEAK_HBM_GBS, 4)},
        "first_tokens": out[:8],
        "decode_graph": eng.step_kind,
        "graph_ms_at_setup": eng.step_times,
    }
    if eng.step_kind == "fused":
        res["gemv_cfg"] = {k: [list(g.cfg), round(g.us, 2)] for k, g in eng.gv.items()}
    if not args.no_cpu:
        hf = hf_cpu_model(args, eng)
        if hf is not None:
            # the contract's quality rule: the emitted tokens replayed teacher-forced
            # through native Qwen (Transformers, CPU), one full forward per sequence
            seqs = list(range(min(B, 2)))
            res["quality"] = hf_teacher_forced_quality(hf, prompt, steps, seqs)
        if B == 1:
            cb = cpu_decode_baseline(eng, prompt, args.cpu_seconds, hf)
            if "first_token" in cb:   # the prefill's greedy token, on both paths
                cb["first_token_matches_gpu"] = cb["first_token"] == out[0]
        else:
            cb = cpu_decode_baseline_cached(eng, hf, B, S, args.cpu_seconds)
        res["cpu_baseline"] = cb
    return res


def hf_cpu_model(args, eng):
    """Transformers' Qwen3ForCausalLM on the CPU with the engine's weights, built
    once per run (None where Transformers is not importable)."""
    if getattr(args, "_hf", None) is None:
        try:
            from kernel_optim_amd.model import weights_to
            args._hf = hf_qwen3_cpu(eng.cfg, weights_to(eng.w, "cpu"))
        except ImportError:
            args._hf = False
    return args._hf or None


def hf_teacher_forced_quality(m, prompt, steps, seqs, margin=2.0):
    """The reference contract's quality check (QWEN_ENGINE_CONTRACT.md, "The
    quality rule"): each emitted token must be native Qwen's argmax given the
    tokens emitted before it, or within ``margin`` logits of it. Native Qwen here
    is Transformers' Qwen3ForCausalLM (sdpa, bf16) on the CPU with the same
    weights; sequence b's prompt and its first N-1 emitted tokens go through one
    forward and the logits of the last N positions are compared. ``steps``: the
    N yielded lists of B ids; ``seqs``: the sequences replayed."""
    import torch
    N = len(steps)
    toks = torch.tensor(steps, dtype=torch.int64).T          # [B, N]
    agree = total = over = 0
    worst = 0.0
    t0 = time.perf_counter()
    with torch.inference_mode():
        for b in seqs:
            ids = torch.tensor([list(prompt[b]) + toks[b, :N - 1].tolist()], dtype=torch.int64)
            lg = m(input_ids=ids, logits_to_keep=N).logits[0].float()   # [N, V]
            chosen = lg.gather(1, toks[b][:, None])[:, 0]
            gap = lg.max(-1).values - chosen
            agree += int((lg.argmax(-1) == toks[b]).sum())
            total += N
            over += int((gap > margin).sum())
            worst = max(worst, float(gap.max()))
    return {"judge": "teacher-forced replay through Transformers Qwen3ForCausalLM (sdpa, "
                     "bf16, CPU), one forward per sequence",
            "sequences": len(seqs), "positions": total,
            "greedy_agreement": round(agree / total, 4),
            "max_gap_to_argmax_logits": round(worst, 4), "tie_margin_logits": margin,
            "positions_over_margin": over, "pass": over == 0,
            "replay_s": round(time.perf_counter() - t0, 1)}


def bench_spec(args, eng, B=1):
    """Greedy decode with prompt-lookup speculation (Engine(spec=True)), same
    model and sizes as bench_decode, two prompts: seeded uniform-random ids (the
    decode workload: lookup rarely matches, so the engine falls back to the
    one-token graph after its first acceptance check) and a 64-token seeded
    pattern repeated to the prompt length (lookup matches). tok/s counts the
    tokens after the first over all sequences; the verify-step and one-token
    step times are the engine's own graph timings at setup."""
    import torch
    cfg = eng.cfg
    S, N = args.prompt, args.new_tokens
    g = torch.Generator().manual_seed(0)
    prompts = {
        "random": torch.randint(0, cfg.vocab, (B, S), generator=g).tolist(),
        "repeated_pattern": torch.randint(0, cfg.vocab, (B, 64), generator=g)
                                 .repeat(1, -(-S // 64))[:, :S].tolist(),
    }
    res = {"workload": f"Qwen3-4B architecture greedy decode with prompt-lookup speculation, "
                       f"B={B}, prompt {S}, {N} new tokens, random-init bf16 weights (seed 0)"}
    for name, prompt in prompts.items():
        for _ in eng.generate(prompt, N):      # setup, tuning, capture, warm-up
            pass
        torch.cuda.synchronize()
        t0 = None
        for i, _ in enumerate(eng.generate(prompt, N)):
            if i == 0:
                t0 = time.perf_counter()
        el = time.perf_counter() - t0
        res[name] = {"tok_s": round(B * (N - 1) / el, 2), "verify_steps": eng.spec_steps}
    res.update({"K": eng.K, "verify_rows": B * (eng.K + 1),
                "verify_path": "fused GEMV" if eng.verify_fused else "hipBLASLt",
                "t_step_ms": round(eng.t_step_ms, 4), "t_verify_ms": round(eng.t_verify_ms, 4),
                "breakeven_tokens_per_verify": round(eng.breakeven, 3)})
    return res


def bench_layer(Bs=(1, 4, 16), ctx=2048, nsets=4, reps=30):
    """One fused Qwen3-4B decoder layer decode step (qkv GEMV with RMSNorm prologue,
    attention with q/k norm + RoPE + KV append at position 2048, combine, o GEMV +
    residual, gate/up GEMV with RMSNorm + SwiGLU, down GEMV + residual), random
    N(0, 0.02) weights, 2048 cached keys: the engine's own layer body
    (kernel_optim_amd.engine.decode_layer) with its tuned GEMVs. ``nsets``
    independent layers (weights and caches) are rotated so the Infinity Cache
    cannot serve a replay; the replays are captured in one graph and timed with
    events."""
    import torch
    from kernel_optim_amd.engine import (OPROJ_DELAY_NS, _rope_tables, attn_units_per_seq,
                                         build_decode_gemvs, decode_layer)
    from kernel_optim_amd.kernels.fused import DecodeAttention, rope_rows
    from kernel_optim_amd.kernels.gemv import tile_weights
    from kernel_optim_amd.model import Qwen3Config, random_weights
    cfg = Qwen3Config(layers=nsets)
    dev = torch.device("cuda:0")
    w = random_weights(cfg, seed=1, device=dev)
    cap = ctx + 16
    cos, sin = _rope_tables(cap, cfg.head_dim, cfg.theta, dev)
    L = w["layers"]
    raw = {name: [l[name] for l in L] for name in ("qkv", "o", "gu", "down")}
    tiles = {}

    def tiled_fn(name, ws):
        if name not in tiles:
            tiles[name] = [tile_weights(w_, swiglu=name == "gu") for w_ in ws]
        return tiles[name]

    res = {}
    for B in Bs:
        g = torch.Generator(device=dev).manual_seed(B)
        kc = [torch.randn(B, cfg.nkv, cap, cfg.head_dim, device=dev, generator=g).to(torch.bfloat16)
              for _ in range(nsets)]
        vc = [torch.randn_like(k) for k in kc]
        pos = torch.full((B,), ctx, dtype=torch.int32, device=dev)
        h = torch.randn(B, cfg.hidden, device=dev, generator=g).to(torch.bfloat16)
        qkv = torch.empty(B, cfg.nqkv, device=dev, dtype=torch.bfloat16)
        att_out = torch.empty(B, cfg.nq * cfg.head_dim, device=dev, dtype=torch.bfloat16)
        act = torch.empty(B, cfg.inter, device=dev, dtype=torch.bfloat16)
        # the engine's decode step: fused combine, the step's RoPE rows once, and the
        # o projection in the attention's launch where it fits (B <= 2)
        att = DecodeAttention(B, 1, cap, cfg.nq, cfg.nkv, cfg.head_dim, dev, fused_combine=True,
                              units_per_seq=attn_units_per_seq(B, cfg.nkv))
        att.oproj_delay_ns = OPROJ_DELAY_NS
        rope = torch.empty(B, 2, cfg.head_dim, device=dev, dtype=torch.bfloat16)
        fuse_o = att.oproj_fusable()
        ops, W = build_decode_gemvs(cfg, B, raw, time.monotonic() + 20, tiled_fn)

        def layers():
            rope_rows(pos, cos, sin, rope)
            for i in range(nsets):
                decode_layer(ops, W, i, L[i], att, h, qkv, att_out, act, kc[i], vc[i], cos, sin,
                             pos, rope, cfg.eps, fuse_o)

        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            layers()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            layers()
        graph.replay()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            graph.replay()
        b.record()
        torch.cuda.synchronize()
        att.check_sync()
        us = a.elapsed_time(b) * 1e3 / (reps * nsets)
        nbytes = cfg.layer_bytes() + B * (ctx + 1) * cfg.nkv * cfg.head_dim * 2 * 2 + \
            B * cfg.nkv * cfg.head_dim * 2 * 2
        res[f"B{B}"] = {"us_per_layer": round(us, 2), "bytes": int(nbytes),
                        "gbs": round(nbytes / us / 1e3, 1),
                        "roofline_frac": round(nbytes / us / 1e3 / PEAK_HBM_GBS, 4),
                        "gemv_cfgs": {k: v.cfg for k, v in ops.items() if k in W},
                        "o_proj": "in the attention launch" if fuse_o else "own launch"}
        del kc, vc
        torch.cuda.empty_cache()
    return res


def cpu_decode_baseline(eng, prompt, seconds, m=None):
    """The reference's CPU path for the decode workload: Transformers'
    Qwen3ForCausalLM (sdpa attention) in bf16 with the engine's weights, greedy
    with a DynamicCache on the same 1024-token prompt; the prefill is timed on
    its own, then one-token decode steps for about ``seconds`` (a bounded sample
    of the 255 steps). Falls back to the oracle's eager forward (kind "port")
    where Transformers is not importable."""
    import torch
    from kernel_optim_amd.model import weights_to
    if m is None:
        return cpu_decode_baseline_port(eng, weights_to(eng.w, "cpu"), seconds)
    from transformers import DynamicCache
    ids = torch.tensor(prompt, dtype=torch.int64)
    with torch.inference_mode():
        t0 = time.perf_counter()
        out = m(input_ids=ids, past_key_values=DynamicCache(), use_cache=True)
        prefill_s = time.perf_counter() - t0
        tok = out.logits[:, -1].float().argmax(-1, keepdim=True)
        first = int(tok[0, 0])
        n, t0 = 0, time.perf_counter()
        while True:
            out = m(input_ids=tok, past_key_values=out.past_key_values, use_cache=True)
            tok = out.logits[:, -1].float().argmax(-1, keepdim=True)
            n += 1
            el = time.perf_counter() - t0
            if el >= seconds or n >= 255:
                break
    return {"value": round(n / el, 4), "unit": "tok/s", "cores": torch.get_num_threads(),
            "kind": "reference",
            "prefill_s": round(prefill_s, 3), "first_token": first,
            "sample": f"Transformers {__import__('transformers').__version__} Qwen3ForCausalLM "
                      f"(sdpa), bf16, the same 36-layer weights, B=1, the same 1024-token "
                      f"prompt with a DynamicCache: prefill {prefill_s:.1f} s, then {n} greedy "
                      f"decode steps in {el:.1f} s; {torch.get_num_threads()} threads, affinity "
                      f"{len(os.sched_getaffinity(0))} cpus"}


def _random_cache(cfg, B, S, layers):
    """A DynamicCache holding S random bf16 keys and values per layer (the
    decode step's cost does not depend on their values)."""
    import torch
    from transformers import DynamicCache
    cache = DynamicCache()
    g = torch.Generator().manual_seed(5)
    for i in range(layers):
        k = torch.empty(B, cfg.nkv, S, cfg.head_dim, dtype=torch.bfloat16)
        k.copy_(torch.randn(k.shape, generator=g))
        cache.update(k, k.clone(), i)
    return cache


def cpu_decode_baseline_cached(eng, m, B, S, seconds):
    """The reference's CPU path for batched decode: Transformers'
    Qwen3ForCausalLM (sdpa, bf16) with the engine's weights, greedy one-token
    steps of B sequences from a DynamicCache already holding S keys per
    sequence and layer (random values: the B x S-token prefill alone would take
    minutes on the host), for about ``seconds``."""
    import torch
    if m is None:
        return None
    cache = _random_cache(eng.cfg, B, S, eng.cfg.layers)
    tok = torch.randint(0, eng.cfg.vocab, (B, 1), generator=torch.Generator().manual_seed(6))
    with torch.inference_mode():
        out = m(input_ids=tok, past_key_values=cache, use_cache=True)      # warm
        tok = out.logits[:, -1].float().argmax(-1, keepdim=True)
        n, t0 = 0, time.perf_counter()
        while True:
            out = m(input_ids=tok, past_key_values=cache, use_cache=True)
            tok = out.logits[:, -1].float().argmax(-1, keepdim=True)
            n += 1
            el = time.perf_counter() - t0
            if el >= seconds or n >= 255:
                break
    del cache
    return {"value": round(B * n / el, 3), "unit": "tok/s", "cores": torch.get_num_threads(),
            "kind": "reference",
            "sample": f"Transformers {__import__('transformers').__version__} Qwen3ForCausalLM "
                      f"(sdpa), bf16, the same {eng.cfg.layers}-layer weights, B={B} greedy one-token decode "
                      f"steps from a DynamicCache of {S} random keys per sequence, {n} steps "
                      f"in {el:.1f} s; {torch.get_num_threads()} threads, affinity "
                      f"{len(os.sched_getaffinity(0))} cpus"}


def cpu_layer_baseline(cfg, Bs, ctx, seconds):
    """The reference's CPU path for one decoder layer's decode step:
    Transformers' Qwen3DecoderLayer (sdpa, bf16, weights N(0, 0.02)) at B
    sequences over a DynamicCache of ``ctx`` random keys, one new token at
    position ctx (its K/V appended, then cropped away again), for about
    ``seconds`` per batch size; us per layer and GB/s of the GPU leg's bytes."""
    import torch
    from transformers import Qwen3Config as HC
    from transformers.models.qwen3.modeling_qwen3 import Qwen3DecoderLayer, Qwen3RotaryEmbedding
    hc = HC(hidden_size=cfg.hidden, intermediate_size=cfg.inter, num_hidden_layers=1,
            num_attention_heads=cfg.nq, num_key_value_heads=cfg.nkv, head_dim=cfg.head_dim,
            vocab_size=cfg.vocab, rms_norm_eps=cfg.eps, rope_theta=cfg.theta,
            max_position_embeddings=40960, attn_implementation="sdpa")
    layer = Qwen3DecoderLayer(hc, layer_idx=0).to(torch.bfloat16).eval()
    g = torch.Generator().manual_seed(7)
    with torch.no_grad():
        for p in layer.parameters():
            if p.dim() == 2:
                p.copy_(0.02 * torch.randn(p.shape, generator=g))
    rot = Qwen3RotaryEmbedding(hc)
    res = {}
    for B in Bs:
        cache = _random_cache(cfg, B, ctx, 1)
        hs = torch.randn(B, 1, cfg.hidden, generator=g).to(torch.bfloat16)
        pid = torch.full((B, 1), ctx, dtype=torch.int64)
        with torch.inference_mode():
            pe = rot(hs, pid)
            step = lambda: (layer(hs, attention_mask=None, position_ids=pid, past_key_values=cache,
                                  use_cache=True, position_embeddings=pe), cache.crop(-1))
            step()
            n, t0 = 0, time.perf_counter()
            while True:
                step()
                n += 1
                el = time.perf_counter() - t0
                if el >= seconds:
                    break
        us = el / n * 1e6
        nbytes = cfg.layer_bytes() + B * (ctx + 1) * cfg.nkv * cfg.head_dim * 2 * 2 + \
            B * cfg.nkv * cfg.head_dim * 2 * 2
        res[f"B{B}"] = {"us_per_layer": round(us, 1), "gbs": round(nbytes / us / 1e3, 3),
                        "calls": n}
        del cache
    return {"value": res, "unit": "us per layer", "cores": torch.get_num_threads(),
            "kind": "reference",
            "sample": f"Transformers {__import__('transformers').__version__} Qwen3DecoderLayer "
                      f"(sdpa), bf16, one token at position {ctx} over {ctx} cached keys, "
                      f"B = {', '.join(str(b) for b in Bs)}, about {seconds:.0f} s each; "
                      f"{torch.get_num_threads()} threads, affinity "
                      f"{len(os.sched_getaffinity(0))} cpus"}


def cpu_ragged_baseline(seconds):
    """The reference's CPU path for the ragged attention workload: torch SDPA
    in bf16 with enable_gqa (Transformers' sdpa decode attention) per sequence
    over its valid keys only, the same 64 lengths as the GPU leg; whole passes
    over the 64 sequences for about ``seconds``; GB/s of the valid bytes."""
    import torch
    import torch.nn.functional as F
    Bg = 64
    lens = torch.randint(128, 16385, (Bg,), generator=torch.Generator().manual_seed(3),
                         dtype=torch.int32).tolist()
    g = torch.Generator().manual_seed(4)
    flat = torch.empty(2 * NKV * D * sum(lens), dtype=torch.bfloat16)
    for i in range(0, flat.numel(), 1 << 26):
        seg = flat[i:i + (1 << 26)]
        seg.copy_(torch.randn(seg.shape, generator=g))
    kv, off = [], 0
    for L in lens:
        n = NKV * L * D
        kv.append((flat[off:off + n].view(1, NKV, L, D), flat[off + n:off + 2 * n].view(1, NKV, L, D)))
        off += 2 * n
    q = torch.randn(Bg, 1, NQ, 1, D, generator=g).to(torch.bfloat16)

    def one_pass():
        for b, (k, v) in enumerate(kv):
            F.scaled_dot_product_attention(q[b], k, v, scale=D ** -0.5, enable_gqa=True)

    one_pass()
    n, t0 = 0, time.perf_counter()
    while True:
        one_pass()
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    nbytes = 4096 * sum(lens) + 2 * Bg * NQ * D * 2
    del flat, kv
    return {"value": round(nbytes * n / el / 1e9, 3), "unit": "GB/s",
            "cores": torch.get_num_threads(), "kind": "reference",
            "sample": f"torch scaled_dot_product_attention, bf16, enable_gqa, per sequence over "
                      f"its valid keys (B = 64, lengths U[128, 16384], seed 3, {sum(lens)} keys), "
                      f"{n} passes in {el:.1f} s; {torch.get_num_threads()} threads, affinity "
                      f"{len(os.sched_getaffinity(0))} cpus"}


def cpu_decode_baseline_port(eng, w, seconds):
    """The oracle's eager Qwen3 forward on the host CPU with the same weights
    (used only where Transformers is not importable): prefill a 16-token prompt,
    then time single-token decode steps for about ``seconds``."""
    import torch
    from oracle.qwen3 import Qwen3Oracle
    n_max = 64
    orc = Qwen3Oracle(eng.cfg, w, B=1, cap=16 + n_max)
    prompt = torch.randint(0, eng.cfg.vocab, (1, 16), generator=torch.Generator().manual_seed(0))
    logits = orc.forward(prompt, 0)[:, -1]
    tok = logits.float().argmax(-1)
    n, t0 = 0, time.perf_counter()
    while n < n_max - 1:
        logits = orc.forward(tok[:, None], 16 + n)[:, -1]
        tok = logits.float().argmax(-1)
        n += 1
        if time.perf_counter() - t0 >= seconds:
            break
    el = time.perf_counter() - t0
    return {"value": round(n / el, 4), "unit": "tok/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"oracle.qwen3.Qwen3Oracle (bf16 F.linear, fp32 attention) on the CPU, same "
                      f"36-layer weights, B=1, 16-token prompt, {n} decode steps in {el:.1f} s"}


def bench_attention(args):
    import torch
    from kernel_optim_amd import _lib
    from kernel_optim_amd.kernels.fused import DecodeAttention

    dev = torch.device("cuda:0")
    nbuf = 3
    gens = [torch.Generator(device=dev).manual_seed(s) for s in range(2 * nbuf + 1)]
    q = torch.randn(B, NQ * D, device=dev, generator=gens[0]).to(torch.bfloat16)
    ks = [torch.randn(B, NKV, CTX, D, device=dev, generator=gens[1 + i]).to(torch.bfloat16)
          for i in range(nbuf)]
    vs = [torch.randn(B, NKV, CTX, D, device=dev, generator=gens[1 + nbuf + i]).to(torch.bfloat16)
          for i in range(nbuf)]
    pos = torch.full((B,), CTX - 1, dtype=torch.int32, device=dev)
    out = torch.empty_like(q)
    # the reference's two-launch form (partials, then a combine launch)
    att = DecodeAttention(B, 1, CTX, NQ, NKV, D, dev)
    # the form the engine runs: partials and the LSE merge in one launch
    att2 = DecodeAttention(B, 1, CTX, NQ, NKV, D, dev, fused_combine=True)
    print(f"[bench] attention B={B} ctx={CTX} unit={att.unit} units={att.max_units * B * NKV} "
          f"grid_waves={att.grid_waves}", file=sys.stderr, flush=True)

    for i in range(args.warmup):
        att(q, ks[i % nbuf], vs[i % nbuf], pos, out)
        att2(q, ks[i % nbuf], vs[i % nbuf], pos, out)
    torch.cuda.synchronize()

    # ---- timed region: K steps, synchronised on both sides ----
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    e0.record()
    for i in range(args.steps):
        att(q, ks[i % nbuf], vs[i % nbuf], pos, out)
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    ms_step = e0.elapsed_time(e1) / args.steps
    nbytes = attn_bytes()
    gbs = nbytes / (ms_step * 1e-3) / 1e9

    # ---- dominant kernel alone, HIP events on its launch stream ----
    stream = torch.cuda.current_stream()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(args.steps)]
    for i in range(args.steps):
        k, v = ks[i % nbuf], vs[i % nbuf]
        evs[i][0].record(stream)
        _lib.call("ko_decode_attn_partial", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(pos),
                  1, CTX, k.stride(0), k.stride(1), B, 1, NKV, D, att.unit, att.max_units,
                  att.grid_waves, att.scale, _lib.ptr(att.o_part), _lib.ptr(att.ml),
                  stream.cuda_stream)
        evs[i][1].record(stream)
    torch.cuda.synchronize()
    k_ms = sum(a.elapsed_time(b) for a, b in evs) / len(evs)
    k_gbs = nbytes / (k_ms * 1e-3) / 1e9

    # ---- the one-launch form (the merge by the last unit of each pair) ----
    e0.record()
    for i in range(args.steps):
        att2(q, ks[i % nbuf], vs[i % nbuf], pos, out)
    e1.record()
    torch.cuda.synchronize()
    ms2 = e0.elapsed_time(e1) / args.steps
    del ks, vs

    # ---- measured copy bandwidth for reference ----
    src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    c0.record()
    for _ in range(5):
        dst.copy_(src)
    c1.record()
    torch.cuda.synchronize()
    copy_gbs = 2 * src.numel() * 5 / (c0.elapsed_time(c1) * 1e-3) / 1e9
    del src, dst
    torch.cuda.empty_cache()
    return {
        "value": round(gbs, 2),
        "ms_per_step": round(ms_step, 5),
        "config": {"workload": "split-K GQA decode attention, B16 x 8192 ctx, 32q/8kv, d128, "
                               "bf16 contiguous KV cache, partial + LSE combine",
                   "batch": B, "ctx": CTX, "q_heads": NQ, "kv_heads": NKV, "head_dim": D,
                   "unit_keys": att.unit, "grid_waves": att.grid_waves},
        "pct_of_peak": round(100 * gbs / PEAK_HBM_GBS, 2),
        "wall_s_timed": round(wall, 4),
        "roofline": {"bound": "hbm",
                     "kernel": f"attn1_kernel<false, {att.waves_per_unit}, false> (split-K partials)",
                     "achieved": round(k_gbs, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(k_gbs / PEAK_HBM_GBS, 4), "traffic": pmc_traffic(),
                     "avg_kernel_us": round(k_ms * 1e3, 3),
                     "algorithmic_bytes_per_launch": nbytes},
        "one_launch": {"gbs": round(nbytes / (ms2 * 1e-3) / 1e9, 2), "ms_per_op": round(ms2, 5),
                       "form": "partials and the LSE merge in one launch (fused_combine=True, "
                               "as the engine runs it)"},
        "measured_copy_gbs": round(copy_gbs, 1),
    }


def bench_attention_ragged(reps=20):
    """Ragged decode attention: B=64, one query token per sequence, lengths
    randint(128, 16385) (seed 3) over a cache padded to 16384 keys, N(0, 1) bf16
    K/V. GB/s counts only the valid keys (4096 B per key over 8 KV heads x K and
    V) plus q and out; the padded tail is never read."""
    import torch
    from kernel_optim_amd.kernels.fused import DecodeAttention
    dev = torch.device("cuda:0")
    Bg, cap = 64, 16384
    lens = torch.randint(128, 16385, (Bg,), generator=torch.Generator().manual_seed(3),
                         dtype=torch.int32)
    g = torch.Generator(device=dev).manual_seed(4)
    k = torch.randn(Bg, NKV, cap, D, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(Bg, NKV, cap, D, device=dev, generator=g).to(torch.bfloat16)
    q = torch.randn(Bg, NQ * D, device=dev, generator=g).to(torch.bfloat16)
    out = torch.empty_like(q)
    lens_d = lens.to(dev)
    att = DecodeAttention(Bg, 1, cap, NQ, NKV, D, dev)
    for _ in range(3):
        att.with_lengths(q, k, v, lens_d, out)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        att.with_lengths(q, k, v, lens_d, out)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / reps
    nbytes = 4096 * int(lens.sum()) + 2 * Bg * NQ * D * 2
    del k, v
    torch.cuda.empty_cache()
    return {"workload": "ragged GQA decode attention, B=64, lengths U[128, 16384] (seed 3), "
                        "cache padded to 16384, 32q/8kv, d128, bf16, partial + LSE combine",
            "us_per_call": round(us, 2), "valid_bytes": nbytes,
            "gbs": round(nbytes / us / 1e3, 1),
            "frac_of_peak": round(nbytes / us / 1e3 / PEAK_HBM_GBS, 4),
            "unit_keys": att.unit, "grid_waves": att.grid_waves}


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}): the decode path "
              "is built and measured on one GPU's share of the work.", file=sys.stderr)
        sys.exit(2)
    import torch
    torch.cuda.set_device(0)
    line = {"metric": METRIC, "value": None, "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": None, "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic"}
    if not args.no_attn:
        line.update(bench_attention(args))
        if not args.no_cpu:
            line["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    if not args.no_decode:
        from kernel_optim_amd.engine import Engine
        eng = Engine("random")
        line["decode_b1"] = bench_decode(args, eng, B=1)
        if not args.no_decode_b16:
            line["decode_b16"] = bench_decode(args, eng, B=16)
        for b in (int(x) for x in args.decode_batches.split(",") if x.strip()):
            line[f"decode_b{b}"] = bench_decode(args, eng, B=b)
        del eng
        torch.cuda.empty_cache()
    if args.spec:
        from kernel_optim_amd.engine import Engine
        eng = Engine("random", spec=True)
        line["decode_b1_spec"] = bench_spec(args, eng, B=1)
        del eng
        torch.cuda.empty_cache()
    args._hf = None
    if not args.no_attn and not args.no_ragged:
        line["attention_ragged_b64"] = bench_attention_ragged()
        if not args.no_cpu:
            line["attention_ragged_b64"]["cpu_baseline"] = cpu_ragged_baseline(args.cpu_seconds / 2)
    if not args.no_layer:
        line["layer_2048"] = bench_layer()
        if not args.no_cpu:
            from kernel_optim_amd.model import Qwen3Config
            try:
                line["layer_2048"]["cpu_baseline"] = cpu_layer_baseline(
                    Qwen3Config(), (1, 4, 16), 2048, args.cpu_seconds / 4)
            except ImportError:
                pass
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
