"""Qwen3 decode engine on the gfx950 HIP kernels.

Surface of the reference (engine/engine.py:119-533):
    Engine(model_path).generate(input_ids: list[list[int]], max_new_tokens: int)
yields one ``list[int]`` of length B per generated step, exactly
``max_new_tokens`` times, greedy, with no EOS stop.

``model_path`` is a local Hugging Face Qwen3 directory (config.json and
*.safetensors), or ``"random"`` / ``"random:<seed>"`` for the Qwen3-4B
architecture with seeded N(0, 0.02) weights. A directory with only config.json
raises FileNotFoundError unless ENGINE_RANDOM_INIT=1 asks for random weights
over that config (seed ENGINE_SEED).

Per shape (B, S, N) the engine allocates a static KV cache
[layers, B, 8, cap, 128] bf16, prefills the prompt with PyTorch-ROCm ops
(kernel_optim_amd.prefill), and captures one decode step in a hipGraph
(torch.cuda.CUDAGraph) that is replayed per token. The decode step is
5 kernels per layer, all from libkoptim (the reference's 7, engine.py:274-292,
with the q/k norm + RoPE + KV append and the split-K combine folded into the
attention launch):
  qkv GEMV (RMSNorm prologue) -> attention (q/k norm + RoPE + KV append
  prologue, split-K partials, last-unit LSE combine) -> o GEMV (+residual) ->
  gate/up GEMV (RMSNorm prologue, SwiGLU epilogue) -> down GEMV (+residual)
and after the layers the LM head with the greedy argmax fused into it; its
finalize kernel also advances the positions and gathers the chosen tokens'
embedding rows, the next step's input. Replays are pipelined: the next step is queued before
the host waits for the previous step's ids (engine.py:509-522).

With ENGINE_SPEC=1 (off by default, as in the reference, engine.py:40-42) the
engine also drafts tokens by prompt lookup (NgramIndex) and checks them with a
second captured graph, the verify step: B*(K+1) rows through the same layers,
attention causal within each sequence's block, greedy ids at every row. The
longest agreeing prefix plus the model's own next token is accepted per
sequence; when the accepted tokens per verify step fall below the measured
break-even, decoding finishes on the pipelined one-token graph
(engine.py:403-508).
"""

import os
import sys
import time

import torch

from .kernels.fused import DecodeAttention, add_rms_norm, qk_norm_rope, rope_rows, silu_mul
from .kernels.gemv import (EPI_ARGMAX, EPI_BF16, EPI_RESID, EPI_SWIGLU, Gemv, argmax_rows,
                           embed_ss, tile_weights, uses_tiled)
from .model import Qwen3Config, load_checkpoint, random_weights
from .prefill import prefill

DEVICE = "cuda:0"
LOG = os.environ.get("ENGINE_LOG", "0") == "1"
TUNE = os.environ.get("ENGINE_TUNE", "1") == "1"
TUNE_BUDGET_S = 60.0
# attention and the o projection in one launch for 1-2 sequences (ENGINE_FUSE_OPROJ=0: two)
FUSE_OPROJ = os.environ.get("ENGINE_FUSE_OPROJ", "1") == "1"
# how long the o projection's workgroups hold their weight loads so the attention's
# first loads go ahead (B = 1 decode, same box: 250 ns 564.9, 500 ns 569.0, 750-1100 ns
# 572-575, 1500 ns 569.1, 2000 ns 564.7, 3000 ns 558.2 tok/s)
OPROJ_DELAY_NS = int(os.environ.get("ENGINE_OPROJ_DELAY_NS", "1000"))
# keys per decode-attention unit (0: DecodeAttention's sizing rule)
ATTN_UNIT = int(os.environ.get("ENGINE_ATTN_UNIT", "0"))
# units per sequence of the one-token attention at B >= 3 (-1: one round of the
# 256 CUs, 256 // (B * KV heads); 0: fixed units of ATTN_UNIT or the sizing rule)
ATTN_SPLIT = int(os.environ.get("ENGINE_ATTN_SPLIT", "-1"))
# decode-step graph: "auto" takes the fused-GEMV step up to FUSED_MAX_B sequences
# and the hipBLASLt step above; "timed" captures both up to FUSED_MAX_TIMED and
# keeps the faster, as the reference does (engine.py:197-208); "fused" or
# "hipblaslt" takes one
DECODE_GRAPH = os.environ.get("ENGINE_DECODE_GRAPH", "auto")
# The fused GEMVs read each weight once for up to 32 rows (B = 32: 8,619 tok/s
# against 7,544 on hipBLASLt); at 33..64 rows qkv, gate/up and the LM head take
# two weight passes (B = 64: 9,538 against 11,599 tok/s on hipBLASLt).
FUSED_MAX_B = 32
FUSED_MAX_TIMED = 64  # "timed": both graphs up to here (engine.py:44)
# verify-step attention: the K+1 tokens of a sequence as rows of the one-token
# kernel (one launch) rather than T-token tiles (two launches and a merge)
VERIFY_TOKEN_ROWS = os.environ.get("ENGINE_VERIFY_TOKEN_ROWS", "1") == "1"
# speculative decoding by prompt lookup (engine.py:35-57)
SPEC = os.environ.get("ENGINE_SPEC", "0") == "1"
NGRAMS = (3, 2, 1)       # lookup order: the longest suffix first
WINDOW = 8               # verify steps between two acceptance checks
HOST_MS = 0.2            # host time per verify step (wait, draft, copies)
MIN_ADVANCE = (float(os.environ["ENGINE_MIN_ADVANCE"]) if "ENGINE_MIN_ADVANCE" in os.environ
               else None)
FUSED_VERIFY_ROWS = 16   # verify rows the fused GEMVs take in one weight pass


def draft_len(B):
    """Drafted tokens per sequence and verify step (engine.py:48-57): the verify
    rows B*(K+1) stay few enough to be weight-streaming bound."""
    if B <= 4:
        return 6
    if B <= 16:
        return 4
    if B <= 32:
        return 2
    return 0


class NgramIndex:
    """Prompt-lookup drafts for one sequence (the reference's _Lookup,
    engine.py:60-93). ``after[n]`` maps every n-gram of the sequence that has a
    successor to the index of that successor at its latest occurrence; a draft
    follows the latest earlier occurrence of the sequence's last 3, else 2,
    else 1 tokens, and repeats the last token when none occurred before."""

    def __init__(self, tokens):
        self.seq = []
        self.after = {n: {} for n in NGRAMS}
        self.extend(tokens)

    def extend(self, tokens):
        seq = self.seq
        for t in tokens:
            i = len(seq)        # t succeeds the n-grams that end at i - 1
            seq.append(int(t))
            for n in NGRAMS:
                if i >= n:
                    self.after[n][tuple(seq[i - n:i])] = i

    def draft(self, K):
        seq = self.seq
        L = len(seq)
        for n in NGRAMS:
            if L < n:
                continue
            j = self.after[n].get(tuple(seq[L - n:]))
            if j is None:
                continue
            out = []
            for k in range(K):
                # past the end the continuation reads the draft itself (a loop)
                out.append(seq[j + k] if j + k < L else out[j + k - L])
            return out
        return [seq[-1]] * K


def accept(draft_row, got_row):
    """Tokens accepted from one verify row (engine.py:477-484): draft_row is the
    verified input [last, d_1..d_K], got_row the greedy ids at those positions;
    the drafts agree while d_{i+1} == got_i, and the model's next token follows
    the agreeing prefix."""
    K = len(draft_row) - 1
    a = 0
    while a < K and draft_row[a + 1] == got_row[a]:
        a += 1
    return list(got_row[:a + 1])


def _rope_tables(n, d, theta, device):
    """cos/sin [n, d] bf16 for positions 0..n-1, computed as the reference takes
    them from model.rotary_emb on the GPU (engine.py:164-171): Qwen3RotaryEmbedding's
    inv_freq built in fp32 on the host, the frequencies as its fp32 product with
    the positions, cos and sin in fp32 on the device, rounded to bf16."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float) / d))
    inv = inv_freq[None, :, None].float().to(device)
    pos = torch.arange(n, device=device)[None, None, :].float()
    freqs = (inv @ pos).transpose(1, 2)
    emb = torch.cat((freqs, freqs), dim=-1)
    return (emb.cos()[0].to(torch.bfloat16).contiguous(),
            emb.sin()[0].to(torch.bfloat16).contiguous())


def _log(msg):
    if LOG:
        print(f"[engine] {msg}", file=sys.stderr, flush=True)


def attn_units_per_seq(B, nkv):
    """Units per sequence of the one-token decode attention at batch B: at 3..64
    sequences each sequence's keys are cut at every step into at most
    256 // (B * nkv) equal units (one round of workgroups over the 256 CUs at
    equal lengths); at B <= 2 (the attention + o projection launch) fixed units.
    ENGINE_ATTN_SPLIT >= 0 overrides (0: fixed units)."""
    if ATTN_SPLIT >= 0:
        return ATTN_SPLIT
    return max(1, 256 // (B * nkv)) if 3 <= B <= 64 else 0


def build_decode_gemvs(cfg, M, raw, deadline, tiled_fn=None, tune=True, log=""):
    """The decode step's five fused projections for M rows (the reference's
    _setup_fused set, engine.py:256-262, with the LM head's greedy selection
    fused in): qkv (RMSNorm prologue, bf16 out), o (+ residual), gate/up (RMSNorm
    prologue, SwiGLU), down (+ residual), LM head (RMSNorm prologue, ARGMAX).
    ``raw`` maps each name to its per-layer row-major weights; with ``tune`` each
    Gemv is timed over them (Gemv.tune). ``tiled_fn(name, weights)`` returns the
    MFMA-tiled copies for a projection that has tiled candidates (None: tune
    makes them). Returns (gemvs, weights in each one's launch layout)."""
    H, e = cfg.hidden, cfg.eps
    gv = dict(
        qkv=Gemv(M, cfg.nqkv, H, EPI_BF16, norm=True, eps=e),
        o=Gemv(M, H, cfg.nq * cfg.head_dim, EPI_RESID, norm=False, eps=e),
        gu=Gemv(M, cfg.inter, H, EPI_SWIGLU, norm=True, eps=e),
        down=Gemv(M, H, cfg.inter, EPI_RESID, norm=False, eps=e),
        lm=Gemv(M, cfg.vocab, H, EPI_ARGMAX, norm=True, eps=e),
    )
    W = {}
    for name, g in gv.items():
        if name not in raw:
            continue
        tiled = None
        if any(uses_tiled(c) for c in g.candidates()):
            tiled = (tiled_fn(name, raw[name]) if tiled_fn is not None
                     else [tile_weights(w, swiglu=name == "gu") for w in raw[name]])
        if tune:
            g.tune(raw[name], deadline, tiled=tiled)
            _log(f"{log}gemv {name} M={M} cfg={g.cfg} {g.us:.1f}us candidates={g.tune_log}")
        W[name] = tiled if uses_tiled(g.cfg) else raw[name]
    return gv, W


def decode_layer(gv, W, i, lw, attn, h, qkv, attn_out, act, k_cache, v_cache, cos, sin, pos,
                 rope, eps, fuse_o):
    """Layer i of the one-token decode step (engine.py:278-287 in this package's
    launches): qkv GEMV (RMSNorm prologue) -> attention (q/k norm + RoPE + KV
    append at pos, split-K partials, last-unit merge), with the o projection and
    its residual add in the same launch when ``fuse_o`` -> o GEMV (+ residual)
    otherwise -> gate/up GEMV (RMSNorm prologue, SwiGLU) -> down GEMV (+ residual).
    h [B, H] is the residual stream, updated in place; k_cache/v_cache are the
    layer's [B, nkv, cap, d] slices; rope the step's RoPE rows (rope_rows)."""
    gv["qkv"](h, W["qkv"][i], y=qkv, nw=lw["w_in"])
    if fuse_o:
        attn.decode_qkv_oproj(qkv, lw["q_norm"], lw["k_norm"], cos, sin, pos, k_cache, v_cache,
                              attn_out, eps, lw["o"], h, rope=rope)
    else:
        attn.decode_qkv(qkv, lw["q_norm"], lw["k_norm"], cos, sin, pos, k_cache, v_cache,
                        attn_out, eps, rope=rope)
        gv["o"](attn_out, W["o"][i], h=h)
    gv["gu"](h, W["gu"][i], y=act, nw=lw["w_post"])
    gv["down"](act, W["down"][i], h=h)


class Engine:
    def __init__(self, model_path: str, keep_logits: bool = False, spec=None,
                 decode_graph=None) -> None:
        self._t0 = time.monotonic()
        if model_path.startswith("random"):
            seed = int(model_path.split(":", 1)[1]) if ":" in model_path else 0
            cfg = Qwen3Config()
            w = random_weights(cfg, seed=seed, device=DEVICE)
        elif os.path.isdir(model_path) and any(f.endswith(".safetensors")
                                                for f in os.listdir(model_path)):
            cfg, w = load_checkpoint(model_path, device=DEVICE)
        elif os.environ.get("ENGINE_RANDOM_INIT", "0") == "1":
            # a config-only directory, random weights asked for explicitly
            cfg = Qwen3Config.from_hf_json(os.path.join(model_path, "config.json"))
            seed = int(os.environ.get("ENGINE_SEED", "0"))
            print(f"[engine] {model_path}: random N(0, 0.02) weights, seed {seed} "
                  "(ENGINE_RANDOM_INIT=1)", file=sys.stderr, flush=True)
            w = random_weights(cfg, seed=seed, device=DEVICE)
        else:
            raise FileNotFoundError(
                f"{model_path}: no *.safetensors weights (pass 'random[:seed]' or set "
                "ENGINE_RANDOM_INIT=1 for random weights over its config.json)")
        self._init(cfg, w, keep_logits, spec, decode_graph)

    @classmethod
    def from_weights(cls, cfg, weights, keep_logits=False, spec=None, decode_graph=None):
        """Engine over weights already in the decode layout (moved to the GPU)."""
        from .model import weights_to
        self = cls.__new__(cls)
        self._t0 = time.monotonic()
        self._init(cfg, weights_to(weights, DEVICE), keep_logits, spec, decode_graph)
        return self

    def _init(self, cfg, w, keep_logits, spec=None, decode_graph=None):
        """spec: prompt-lookup speculation on (True) or off (False); None takes
        ENGINE_SPEC (off unless set to 1). decode_graph: "auto" (the fused-GEMV
        decode graph up to FUSED_MAX_B sequences, the hipBLASLt graph above),
        "timed" (capture both up to FUSED_MAX_TIMED sequences, time them at setup
        and keep the faster), "fused" or "hipblaslt"; None takes
        ENGINE_DECODE_GRAPH (auto unless set)."""
        self.spec = SPEC if spec is None else bool(spec)
        self.min_advance = MIN_ADVANCE   # None: the measured break-even
        kind = DECODE_GRAPH if decode_graph is None else decode_graph
        if kind not in ("auto", "timed", "fused", "hipblaslt"):
            raise ValueError(f"decode_graph must be auto, timed, fused or hipblaslt, not {kind!r}")
        self.decode_graph = kind
        if cfg.head_dim != 128 or cfg.nq != 4 * cfg.nkv:
            raise ValueError("the decode kernels serve head_dim 128 with 4 query heads per KV head")
        self.cfg, self.w = cfg, w
        self.keep_logits = keep_logits
        self._cos = self._sin = None
        self._shape = None
        self.g1 = None
        self._tile_cache = {}
        # polls of a done flag before an attention + o projection wait gives up
        # (-1: the library's bound; 0: at once, which tests of that path use);
        # taken at the next setup
        self.oproj_spin = -1

    # ------------------------------------------------------------------ setup
    def _tables(self, n):
        if self._cos is None or self._cos.shape[0] < n:
            self._cos, self._sin = _rope_tables(n, self.cfg.head_dim, self.cfg.theta, DEVICE)

    def _setup(self, B, S, N):
        key = (B, S, N)
        if self._shape == key:
            return
        self._shape = None
        self.g1 = self.gk = None
        self.k_cache = self.v_cache = None
        torch.cuda.empty_cache()
        cfg = self.cfg
        self.K = draft_len(B) if self.spec and N > 2 else 0
        # with speculation a sequence can run ahead of the slowest by N + K tokens
        need = S + 2 * N + 2 * self.K + 2 if self.K else S + N + 1
        cap = -(-need // 16) * 16
        self.B, self.S, self.cap = B, S, cap
        self._tables(cap)
        dev = DEVICE
        bf = torch.bfloat16
        self.k_cache = torch.zeros(cfg.layers, B, cfg.nkv, cap, cfg.head_dim, dtype=bf, device=dev)
        self.v_cache = torch.zeros_like(self.k_cache)
        self.pos = torch.zeros(B, dtype=torch.int32, device=dev)
        self.ids = torch.zeros(B, dtype=torch.int64, device=dev)
        self.h = torch.zeros(B, cfg.hidden, dtype=bf, device=dev)
        self.qkv = torch.zeros(B, cfg.nqkv, dtype=bf, device=dev)
        self.q1 = torch.zeros(B, cfg.nq * cfg.head_dim, dtype=bf, device=dev)
        self.attn_out = torch.zeros_like(self.q1)
        self.act = torch.zeros(B, cfg.inter, dtype=bf, device=dev)
        self.rope = torch.zeros(B, 2, cfg.head_dim, dtype=bf, device=dev)
        self.logits = (torch.zeros(B, cfg.vocab, dtype=bf, device=dev) if self.keep_logits
                       else None)
        # ids of step j land in row j: the prefill's by a copy, the decode steps'
        # straight from the LM head's tail (ring_ctr: the next row it writes)
        self.pin_ids = torch.empty(N + 1, B, dtype=torch.int64, pin_memory=True)
        self._ring_np = self.pin_ids.numpy()
        self.ring_ctr = torch.zeros(B, dtype=torch.int32, device=dev)
        self.events = [torch.cuda.Event() for _ in range(N + 1)]
        self.attn = DecodeAttention(B, 1, cap, cfg.nq, cfg.nkv, cfg.head_dim, dev,
                                    unit=ATTN_UNIT or None, fused_combine=True,
                                    units_per_seq=attn_units_per_seq(B, cfg.nkv))
        self.attn.oproj_delay_ns = OPROJ_DELAY_NS
        self.attn.oproj_spin = self.oproj_spin
        L = self.w["layers"]
        raw = dict(qkv=[l["qkv"] for l in L], o=[l["o"] for l in L], gu=[l["gu"] for l in L],
                   down=[l["down"] for l in L], lm=[self.w["lm_head"]])
        deadline = time.monotonic() + TUNE_BUDGET_S
        kind = self.decode_graph
        if kind == "auto":
            kind = "fused" if B <= FUSED_MAX_B else "hipblaslt"
        elif kind == "timed" and B > FUSED_MAX_TIMED:
            kind = "hipblaslt"
        self.step_times = {}
        g_fused = g_mm = None
        if kind in ("timed", "fused"):
            g_fused = self._setup_fused(raw, deadline)
        if kind in ("timed", "hipblaslt"):
            g_mm = self._setup_mm()
        if kind == "timed":
            # keep whichever decode graph is faster here, measured during setup
            t_f = min(self._time_graph(g_fused) for _ in range(2))
            t_m = min(self._time_graph(g_mm) for _ in range(2))
            self.step_times = {"fused_ms": round(t_f, 4), "hipblaslt_ms": round(t_m, 4)}
            _log(f"decode step B={B}: fused {t_f * 1e3:.0f}us hipBLASLt {t_m * 1e3:.0f}us")
            kind = "fused" if t_f < t_m else "hipblaslt"
        self.step_kind = kind
        self.g1 = g_fused if kind == "fused" else g_mm
        self.gk = None
        if self.K:
            self._setup_verify(raw, deadline)
        self._shape = key

    def _setup_fused(self, raw, deadline):
        """The fused-GEMV decode step: tuned GEMVs (with MFMA weight copies where
        the tuner takes them) and its captured graph."""
        self.gv, self.gw = build_decode_gemvs(self.cfg, self.B, raw, deadline, self._tiled,
                                              tune=TUNE)
        return self._capture(self._step1)

    def _setup_mm(self):
        """The hipBLASLt decode step (the reference's cuBLAS step, engine.py:388-401):
        its buffers and captured graph."""
        cfg, B, dev, bf = self.cfg, self.B, DEVICE, torch.bfloat16
        self.nrm = torch.zeros(B, cfg.hidden, dtype=bf, device=dev)
        self.gu_mm = torch.zeros(B, 2 * cfg.inter, dtype=bf, device=dev)
        self.logits_mm = (self.logits if self.logits is not None
                          else torch.zeros(B, cfg.vocab, dtype=bf, device=dev))
        return self._capture(self._step1_mm)

    def _setup_verify(self, raw, deadline):
        """Buffers, GEMVs and the captured graph of the verify step, and the
        break-even tokens per verify step (engine.py:209-223)."""
        cfg, B, dev, bf = self.cfg, self.B, DEVICE, torch.bfloat16
        T = self.K + 1
        M = B * T
        H, e = cfg.hidden, cfg.eps
        self.T = T
        self.vin = torch.zeros(B, T, dtype=torch.int64, device=dev)
        self.vout = torch.zeros(B, T, dtype=torch.int64, device=dev)
        self.pin_vin = torch.empty(B, T, dtype=torch.int64, pin_memory=True)
        self.pin_vout = torch.empty(B, T, dtype=torch.int64, pin_memory=True)
        self.pin_pos = torch.empty(B, dtype=torch.int32, pin_memory=True)
        self.hT = torch.zeros(M, H, dtype=bf, device=dev)
        self.qkvT = torch.zeros(M, cfg.nqkv, dtype=bf, device=dev)
        self.qT = torch.zeros(M, cfg.nq * cfg.head_dim, dtype=bf, device=dev)
        self.attT = torch.zeros_like(self.qT)
        self.actT = torch.zeros(M, cfg.inter, dtype=bf, device=dev)
        if VERIFY_TOKEN_ROWS:
            # the B*T tokens as rows of the one-token kernel, each row merged by
            # its last unit: one launch
            self.attnk = DecodeAttention(B, T, self.cap, cfg.nq, cfg.nkv, cfg.head_dim, dev,
                                         fused_combine=True, token_rows=True)
        else:
            # T-token tiles and the merge as its own launch: one wavefront per row,
            # where the fused combine would merge a pair's T x 4 rows in one wavefront
            self.attnk = DecodeAttention(B, T, self.cap, cfg.nq, cfg.nkv, cfg.head_dim, dev)
        self.verify_fused = M <= FUSED_VERIFY_ROWS
        if self.verify_fused:   # one weight pass per projection on the fused GEMVs
            self.gvk, self.gwk = build_decode_gemvs(cfg, M, raw, deadline, self._tiled,
                                                    tune=TUNE, log="verify ")
        else:                   # hipBLASLt GEMMs between the fused ops
            self.nT = torch.zeros(M, H, dtype=bf, device=dev)
            self.guT = torch.zeros(M, 2 * cfg.inter, dtype=bf, device=dev)
        self.logitsT = (torch.zeros(M, cfg.vocab, dtype=bf, device=dev)
                        if self.keep_logits or not self.verify_fused else None)
        self.gk = self._capture(self._stepk)
        t1 = min(self._time_graph(self.g1) for _ in range(2))
        tk = min(self._time_graph(self.gk) for _ in range(2))
        self.t_step_ms, self.t_verify_ms = t1, tk
        self.breakeven = (tk + HOST_MS) / t1 if self.min_advance is None else self.min_advance
        _log(f"B={B} K={self.K}: step {t1 * 1e3:.0f}us verify {tk * 1e3:.0f}us -> speculate "
             f"while >= {self.breakeven:.3f} tokens/step")

    def _set_pos(self, p):
        """Set the positions (an int or a [B] tensor) and the RoPE rows the next
        one-token step reads for them (the step itself then keeps both current)."""
        if isinstance(p, torch.Tensor):
            self.pos.copy_(p, non_blocking=True)
        else:
            self.pos.fill_(p)
        rope_rows(self.pos, self._cos, self._sin, self.rope)

    def _time_graph(self, g, reps=10):
        """GPU time (ms) of one replay of a captured step: the median of ``reps``
        replays, each between its own pair of events, after one untimed replay.
        The replays start at the prompt's end, or earlier where the cache slots
        they write (one per replay for the one-token step, K + 1 for the verify
        step) would pass the capacity."""
        span = max(reps + 1, self.K + 1) + 1
        torch.cuda.synchronize()
        self._set_pos(max(0, min(self.S, self.cap - span)))
        g.replay()
        marks = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                 for _ in range(reps)]
        for a, b in marks:
            a.record()
            g.replay()
            b.record()
        torch.cuda.synchronize()
        times = sorted(a.elapsed_time(b) for a, b in marks)
        return times[len(times) // 2]

    def _tiled(self, name, weights):
        """MFMA-layout copies of one projection's weights (kernels.gemv.tile_weights),
        made once and kept for every later batch size that uses them."""
        if name not in self._tile_cache:
            self._tile_cache[name] = [tile_weights(w, swiglu=name == "gu") for w in weights]
            torch.cuda.synchronize()
        return self._tile_cache[name]

    def _step1(self):
        """One decode token per sequence at pos[b]; greedy ids; positions advance."""
        cfg = self.cfg
        g, W = self.gv, self.gw  # W: each projection's weights in its launch layout
        # h holds embed[ids] and rope the RoPE rows at pos: both written by the
        # previous step's LM head tail (or by the prefill hand-off)
        h = self.h
        fuse_o = FUSE_OPROJ and self.attn.oproj_fusable()
        for i, lw in enumerate(self.w["layers"]):
            decode_layer(g, W, i, lw, self.attn, h, self.qkv, self.attn_out, self.act,
                         self.k_cache[i], self.v_cache[i], self._cos, self._sin, self.pos,
                         self.rope, cfg.eps, fuse_o)
        # LM head + greedy ids + pos += 1 + the next step's embedding rows and RoPE
        # rows + the ids into the pinned host ring, in one call
        g["lm"](h, W["lm"][0], y=self.logits, nw=self.w["final_norm"], ids=self.ids,
                pos_inc=self.pos, next_emb=self.w["embed"], next_h=h,
                rope=(self._cos, self._sin, self.rope),
                ring=(self.pin_ids, self.ring_ctr, self.attn.err if fuse_o else None))

    def _step1_mm(self):
        """One decode token per sequence with hipBLASLt GEMMs (torch.mm) between
        the fused ops: RMSNorm, the projections, the attention with its q/k norm +
        RoPE + KV append prologue, SwiGLU, the residual adds, the LM head and the
        greedy ids (argmax_rows); then positions advance and the chosen tokens'
        embedding rows become the next step's input, as in the fused step."""
        cfg = self.cfg
        eps = cfg.eps
        h = self.h   # holds embed[ids]
        rope_rows(self.pos, self._cos, self._sin, self.rope)
        for i, lw in enumerate(self.w["layers"]):
            add_rms_norm(h, None, lw["w_in"], self.nrm, eps)
            torch.mm(self.nrm, lw["qkv"].t(), out=self.qkv)
            self.attn.decode_qkv(self.qkv, lw["q_norm"], lw["k_norm"], self._cos, self._sin,
                                 self.pos, self.k_cache[i], self.v_cache[i], self.attn_out, eps,
                                 rope=self.rope)
            h.add_(torch.mm(self.attn_out, lw["o"].t()))   # h <- bf16(h + bf16(x @ W^T))
            add_rms_norm(h, None, lw["w_post"], self.nrm, eps)
            torch.mm(self.nrm, lw["gu"].t(), out=self.gu_mm)
            silu_mul(self.gu_mm, self.act)
            h.add_(torch.mm(self.act, lw["down"].t()))
        add_rms_norm(h, None, self.w["final_norm"], self.nrm, eps)
        torch.mm(self.nrm, self.w["lm_head"].t(), out=self.logits_mm)
        argmax_rows(self.logits_mm, self.ids)
        self.pos.add_(1)
        embed_ss(self.ids, self.w["embed"], h, None)

    def _stepk(self):
        """Verify step (engine.py:403-416): vin[b] = [last accepted token, K drafts]
        at positions pos[b] .. pos[b]+K, through every layer as B*(K+1) rows (K/V
        appended at those slots, attention causal within the block); vout[b, t]
        = greedy id after vin[b, :t+1]. Positions do not advance."""
        cfg = self.cfg
        T = self.T
        eps = cfg.eps
        h = self.hT
        embed_ss(self.vin.view(-1), self.w["embed"], h, None)
        fused = self.verify_fused
        g, W = (self.gvk, self.gwk) if fused else (None, None)
        for i, lw in enumerate(self.w["layers"]):
            if fused:
                g["qkv"](h, W["qkv"][i], y=self.qkvT, nw=lw["w_in"])
            else:
                add_rms_norm(h, None, lw["w_in"], self.nT, eps)
                torch.mm(self.nT, lw["qkv"].t(), out=self.qkvT)
            qk_norm_rope(self.qkvT, lw["q_norm"], lw["k_norm"], self._cos, self._sin, self.pos,
                         self.qT, self.k_cache[i], self.v_cache[i], T, eps, cfg.nq, cfg.nkv,
                         cfg.head_dim)
            self.attnk(self.qT, self.k_cache[i], self.v_cache[i], self.pos, self.attT)
            if fused:
                g["o"](self.attT, W["o"][i], h=h)
                g["gu"](h, W["gu"][i], y=self.actT, nw=lw["w_post"])
                g["down"](self.actT, W["down"][i], h=h)
            else:   # h <- bf16(h + bf16(x @ W^T)), the RESID chain
                h.add_(torch.mm(self.attT, lw["o"].t()))
                add_rms_norm(h, None, lw["w_post"], self.nT, eps)
                torch.mm(self.nT, lw["gu"].t(), out=self.guT)
                silu_mul(self.guT, self.actT)
                h.add_(torch.mm(self.actT, lw["down"].t()))
        if fused:
            g["lm"](h, W["lm"][0], y=self.logitsT, nw=self.w["final_norm"], ids=self.vout.view(-1))
        else:
            add_rms_norm(h, None, self.w["final_norm"], self.nT, eps)
            torch.mm(self.nT, self.w["lm_head"].t(), out=self.logitsT)
            argmax_rows(self.logitsT, self.vout.view(-1))

    def _capture(self, fn, warmups=2):
        """A hipGraph of one call of ``fn`` (torch's documented capture recipe):
        ``fn`` first runs ``warmups`` times eagerly on a side stream, so every
        code object is loaded and every buffer it touches exists, then once
        under capture. The eager calls write cache slot 0 (positions 0), which
        every prefill overwrites."""
        main = torch.cuda.current_stream()
        side = torch.cuda.Stream()
        side.wait_stream(main)
        with torch.cuda.stream(side):
            for _ in range(warmups):
                self._set_pos(0)
                fn()
        main.wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        self._set_pos(0)
        with torch.cuda.graph(graph):
            fn()
        torch.cuda.synchronize()
        return graph

    # ---------------------------------------------------------------- forward
    def _prefill(self, prompt):
        ids, logits = prefill(self.cfg, self.w, prompt, self.k_cache, self.v_cache, self._cos,
                              self._sin)
        self.ids.copy_(ids)
        self._set_pos(prompt.shape[1])
        embed_ss(self.ids, self.w["embed"], self.h, None)   # the first decode step's input
        if self.logits is not None:
            self.logits.copy_(logits)

    @torch.inference_mode()
    def step(self):
        """Replay one decode step (for callers that drive decoding themselves)."""
        self.g1.replay()

    @torch.inference_mode()
    def verify_step(self, rows, pos):
        """Replay the verify graph for rows [B, K+1] (int64: the last accepted token
        and K drafts) at positions pos [B] (of rows[:, 0]); returns the greedy ids
        [B, K+1] and, with keep_logits, the bf16 logits [B*(K+1), V], on the CPU.
        Writes K/V cache slots pos .. pos+K. Needs a setup with speculation."""
        if self.gk is None:
            raise ValueError("verify_step needs an engine set up with speculation (spec=True, "
                             "max_new_tokens > 2, a batch of at most 32)")
        self.vin.copy_(torch.as_tensor(rows, dtype=torch.int64))
        self._set_pos(torch.as_tensor(pos, dtype=torch.int32).to(DEVICE))
        self.gk.replay()
        torch.cuda.synchronize()
        return self.vout.cpu(), (self.logitsT.cpu() if self.keep_logits else None)

    @torch.inference_mode()
    def time_step(self, reps=20):
        """Mean GPU time (ms) of one replayed decode step, from positions S."""
        torch.cuda.synchronize()
        self._set_pos(self.S)
        self.g1.replay()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            self.g1.replay()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / reps

    # --------------------------------------------------------------- generate
    @torch.inference_mode()
    def generate(self, input_ids: list, max_new_tokens: int):
        N = max_new_tokens
        if N <= 0:
            return
        B, S = len(input_ids), len(input_ids[0])
        # nothing from an earlier call may still write the ring or the caches
        torch.cuda.synchronize()
        self._setup(B, S, N)
        stream = torch.cuda.current_stream()
        try:
            prompt = torch.tensor(input_ids, dtype=torch.int64).pin_memory().to(
                DEVICE, non_blocking=True)
            self._prefill(prompt)
            ids_h, ev = self.pin_ids, self.events
            ids_h[0].copy_(self.ids, non_blocking=True)
            ev[0].record(stream)
            if self.K:
                yield from self._generate_spec(input_ids, N, stream)
                return
            # The fused step writes its ids into row ring_ctr of ids_h itself, so
            # the host waits for row j to fill (rows start at -1) instead of
            # recording an event per step; the hipBLASLt step's ids are copied
            # after each replay and waited for with an event.
            ring = self.step_kind == "fused"
            if ring:
                self._ring_np[1:] = -1
                self.ring_ctr.fill_(1)
            # Keep one replay in flight: queue step j before waiting for step j-1.
            if N > 1:
                self.g1.replay()
                if not ring:
                    ids_h[1].copy_(self.ids, non_blocking=True)
                    ev[1].record(stream)
            ev[0].synchronize()
            yield ids_h[0].tolist()
            for j in range(1, N):
                if j + 1 < N:
                    self.g1.replay()
                    if not ring:
                        ids_h[j + 1].copy_(self.ids, non_blocking=True)
                        ev[j + 1].record(stream)
                if ring:
                    self._wait_row(j)   # raises at the step whose o-projection wait failed
                else:
                    ev[j].synchronize()
                yield ids_h[j].tolist()
            self.attn.check_sync()
        finally:
            # a caller that stops early (or an error) leaves no replay in flight
            torch.cuda.synchronize()

    def _wait_row(self, j, timeout_s=60.0):
        """Wait until the decode step that writes row j of the pinned id ring has
        stored every sequence's id (the LM head's tail stores them from the GPU;
        the rows start at -1). A row of -2 is a step whose attention + o
        projection wait gave up: raise (DecodeAttention.check_sync) at that step."""
        row = self._ring_np[j]
        t_end = None
        while (row == -1).any():
            if t_end is None:
                t_end = time.monotonic() + timeout_s
            elif time.monotonic() > t_end:
                torch.cuda.synchronize()
                if (row == -1).any():
                    raise RuntimeError(f"decode step {j} stored no ids in the host ring")
        if (row < 0).any():
            torch.cuda.synchronize()
            self.attn.check_sync()
            raise RuntimeError(f"decode step {j}: the ring holds no ids")

    def _generate_spec(self, input_ids, N, stream):
        """generate() with prompt-lookup speculation (engine.py:435-508): verify
        steps while they pay for themselves, then the pipelined one-token graph
        from each sequence's own position. Tokens are yielded as soon as every
        sequence has them; a sequence that has N tokens keeps its position and
        its verify rows are ignored."""
        B, S, K = self.B, self.S, self.K
        look = [NgramIndex(row) for row in input_ids]   # built while prefill runs
        ev, ids_h = self.events, self.pin_ids
        ev[0].synchronize()
        first = ids_h[0].tolist()
        yield first
        if N == 1:
            return
        outs = [[t] for t in first]
        for b in range(B):
            look[b].extend([first[b]])
        emitted, steps, window_base = 1, 0, 1
        vin_h, vout_h, pos_h = self.pin_vin, self.pin_vout, self.pin_pos
        self.spec_steps = 0
        while emitted < N:
            vin_h.copy_(torch.tensor([[lk.seq[-1]] + lk.draft(K) for lk in look]))
            pos_h.copy_(torch.tensor([len(lk.seq) - 1 for lk in look], dtype=torch.int32))
            self.vin.copy_(vin_h, non_blocking=True)
            self.pos.copy_(pos_h, non_blocking=True)
            self.gk.replay()
            vout_h.copy_(self.vout, non_blocking=True)
            ev[1].record(stream)
            ev[1].synchronize()
            steps += 1
            drafts, got = vin_h.tolist(), vout_h.tolist()
            for b in range(B):
                if len(outs[b]) >= N:
                    continue
                new = accept(drafts[b], got[b])
                outs[b].extend(new)
                look[b].extend(new)
            ready = min(len(o) for o in outs)
            while emitted < min(ready, N):
                yield [o[emitted] for o in outs]
                emitted += 1
            if steps % WINDOW == 0 and emitted < N:
                advance = (ready - window_base) / WINDOW
                window_base = ready
                if advance < self.breakeven:
                    break   # not paying for itself: finish on the one-token graph
        self.spec_steps = steps
        _log(f"B={B} S={S} N={N} K={K}: {steps} verify steps, {min(len(o) for o in outs)} "
             f"tokens per sequence")
        if emitted >= N:
            return
        # hand each sequence's last token and position to the one-token graph
        for b in range(B):
            ids_h[0, b] = outs[b][-1]
            pos_h[b] = S + len(outs[b]) - 1
        self.ids.copy_(ids_h[0], non_blocking=True)
        self._set_pos(pos_h)
        embed_ss(self.ids, self.w["embed"], self.h, None)   # the step's input rows
        todo = N - min(len(o) for o in outs)
        ring = self.step_kind == "fused"
        if ring:
            self.ring_ctr.fill_(1)
        # pipelined: step j is queued before the host waits for step j-1
        for j in range(1, todo + 1):
            self.g1.replay()
            if not ring:
                ids_h[j].copy_(self.ids, non_blocking=True)
            ev[j].record(stream)
            if j > 1:
                emitted = yield from self._drain(j - 1, outs, N, emitted)
        emitted = yield from self._drain(todo, outs, N, emitted, last=True)

    def _drain(self, j, outs, N, emitted, last=False):
        self.events[j].synchronize()
        row = self.pin_ids[j].tolist()
        if last or min(row) < 0:   # -2: that step's o-projection wait gave up
            torch.cuda.synchronize()
            self.attn.check_sync()
            if min(row) < 0:
                raise RuntimeError(f"decode step {j}: the ring holds no ids")
        for b, t in enumerate(row):
            outs[b].append(t)
        ready = min(N, min(len(o) for o in outs))
        while emitted < ready:
            yield [o[emitted] for o in outs]
            emitted += 1
        return emitted

    @torch.inference_mode()
    def trace(self, input_ids: list, n: int):
        """Greedy decode without pipelining, returning (tokens [B, n] int64 on the
        CPU, per-step bf16 logits [B, V] on the CPU). Needs keep_logits=True."""
        if not self.keep_logits:
            raise ValueError("trace() needs Engine(..., keep_logits=True)")
        B, S = len(input_ids), len(input_ids[0])
        self._setup(B, S, n)
        prompt = torch.tensor(input_ids, dtype=torch.int64, device=DEVICE)
        self._prefill(prompt)
        toks, logits = [self.ids.cpu()], [self.logits.cpu()]
        for _ in range(1, n):
            self.g1.replay()
            toks.append(self.ids.cpu())
            logits.append(self.logits.cpu())
            self.attn.check_sync()   # raises at the step whose o-projection wait failed
        return torch.stack(toks, 1), logits
