"""Qwen3 decode engine on the gfx950 HIP kernels.

Surface of the reference (engine/engine.py:119-533):
    Engine(model_path).generate(input_ids: list[list[int]], max_new_tokens: int)
yields one ``list[int]`` of length B per generated step, exactly
``max_new_tokens`` times, greedy, with no EOS stop.

``model_path`` is a local Hugging Face Qwen3 directory (config.json and
*.safetensors), a directory with only config.json (random init), or
``"random"`` / ``"random:<seed>"`` for the Qwen3-4B architecture with seeded
N(0, 0.02) weights.

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
"""

import os
import sys
import time

import torch

from .kernels.fused import DecodeAttention, rope_rows
from .kernels.gemv import EPI_ARGMAX, EPI_BF16, EPI_RESID, EPI_SWIGLU, Gemv, embed_ss, tile_weights
from .model import Qwen3Config, load_checkpoint, random_weights
from .prefill import prefill

DEVICE = "cuda:0"
LOG = os.environ.get("ENGINE_LOG", "0") == "1"
TUNE = os.environ.get("ENGINE_TUNE", "1") == "1"
TUNE_BUDGET_S = 60.0
# attention and the o projection in one launch for 1-2 sequences (ENGINE_FUSE_OPROJ=0: two)
FUSE_OPROJ = os.environ.get("ENGINE_FUSE_OPROJ", "1") == "1"
OPROJ_DELAY_NS = int(os.environ.get("ENGINE_OPROJ_DELAY_NS", "1000"))
# keys per decode-attention unit (0: DecodeAttention's sizing rule)
ATTN_UNIT = int(os.environ.get("ENGINE_ATTN_UNIT", "0"))


def _rope_tables(n, d, theta, device):
    """cos/sin [n, d] bf16, Qwen3RotaryEmbedding's construction (fp32 on the CPU,
    rounded to bf16), as the reference takes them from model.rotary_emb
    (engine.py:164-171)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.int64).to(torch.float32) / d))
    pos = torch.arange(n, dtype=torch.int64).to(torch.float32)
    freqs = pos[:, None] * inv_freq[None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    return (emb.cos().to(torch.bfloat16).to(device).contiguous(),
            emb.sin().to(torch.bfloat16).to(device).contiguous())


def _log(msg):
    if LOG:
        print(f"[engine] {msg}", file=sys.stderr, flush=True)


class Engine:
    def __init__(self, model_path: str, keep_logits: bool = False) -> None:
        self._t0 = time.monotonic()
        if model_path.startswith("random"):
            seed = int(model_path.split(":", 1)[1]) if ":" in model_path else 0
            cfg = Qwen3Config()
            w = random_weights(cfg, seed=seed, device=DEVICE)
        elif os.path.isdir(model_path) and any(f.endswith(".safetensors")
                                                for f in os.listdir(model_path)):
            cfg, w = load_checkpoint(model_path, device=DEVICE)
        else:
            cfg = Qwen3Config.from_hf_json(os.path.join(model_path, "config.json"))
            w = random_weights(cfg, seed=int(os.environ.get("ENGINE_SEED", "0")), device=DEVICE)
        self._init(cfg, w, keep_logits)

    @classmethod
    def from_weights(cls, cfg, weights, keep_logits=False):
        """Engine over weights already in the decode layout (moved to the GPU)."""
        from .model import weights_to
        self = cls.__new__(cls)
        self._t0 = time.monotonic()
        self._init(cfg, weights_to(weights, DEVICE), keep_logits)
        return self

    def _init(self, cfg, w, keep_logits):
        if cfg.head_dim != 128 or cfg.nq != 4 * cfg.nkv:
            raise ValueError("the decode kernels serve head_dim 128 with 4 query heads per KV head")
        self.cfg, self.w = cfg, w
        self.keep_logits = keep_logits
        self._cos = self._sin = None
        self._shape = None
        self.g1 = None
        self._tile_cache = {}

    # ------------------------------------------------------------------ setup
    def _tables(self, n):
        if self._cos is None or self._cos.shape[0] < n:
            self._cos, self._sin = _rope_tables(n, self.cfg.head_dim, self.cfg.theta, DEVICE)

    def _setup(self, B, S, N):
        key = (B, S, N)
        if self._shape == key:
            return
        self._shape = None
        self.g1 = None
        self.k_cache = self.v_cache = None
        torch.cuda.empty_cache()
        cfg = self.cfg
        cap = -(-(S + N + 1) // 16) * 16
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
        self.pin_ids = torch.empty(N + 1, B, dtype=torch.int64, pin_memory=True)
        self.events = [torch.cuda.Event() for _ in range(N + 1)]
        self.attn = DecodeAttention(B, 1, cap, cfg.nq, cfg.nkv, cfg.head_dim, dev,
                                    unit=ATTN_UNIT or None, fused_combine=True)
        self.attn.oproj_delay_ns = OPROJ_DELAY_NS
        H, L = cfg.hidden, self.w["layers"]
        e = cfg.eps
        self.gv = dict(
            qkv=Gemv(B, cfg.nqkv, H, EPI_BF16, norm=True, eps=e),
            o=Gemv(B, H, cfg.nq * cfg.head_dim, EPI_RESID, norm=False, eps=e),
            gu=Gemv(B, cfg.inter, H, EPI_SWIGLU, norm=True, eps=e),
            down=Gemv(B, H, cfg.inter, EPI_RESID, norm=False, eps=e),
            lm=Gemv(B, cfg.vocab, H, EPI_ARGMAX, norm=True, eps=e),
        )
        raw = dict(qkv=[l["qkv"] for l in L], o=[l["o"] for l in L], gu=[l["gu"] for l in L],
                   down=[l["down"] for l in L], lm=[self.w["lm_head"]])
        deadline = time.monotonic() + TUNE_BUDGET_S
        self.gw = {}
        for name, g in self.gv.items():
            tiled = None
            if any(c[0] == 2 for c in g.candidates()):
                tiled = self._tiled(name, raw[name])
            if TUNE:
                g.tune(raw[name], deadline, tiled=tiled)
                _log(f"gemv {name} B={B} cfg={g.cfg} {g.us:.1f}us candidates={g.tune_log}")
            self.gw[name] = tiled if g.cfg[0] == 2 else raw[name]
        self.g1 = self._capture(self._step1)
        self._shape = key

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
        h = self.h   # holds embed[ids]: written by the previous step's LM head (or prefill)
        fuse_o = FUSE_OPROJ and self.attn.oproj_fusable()
        rope_rows(self.pos, self._cos, self._sin, self.rope)  # the step's RoPE rows, once
        for i, lw in enumerate(self.w["layers"]):
            g["qkv"](h, W["qkv"][i], y=self.qkv, nw=lw["w_in"])
            if fuse_o:  # attention + o projection + residual in one launch
                self.attn.decode_qkv_oproj(self.qkv, lw["q_norm"], lw["k_norm"], self._cos,
                                           self._sin, self.pos, self.k_cache[i], self.v_cache[i],
                                           self.attn_out, cfg.eps, lw["o"], h, rope=self.rope)
            else:
                self.attn.decode_qkv(self.qkv, lw["q_norm"], lw["k_norm"], self._cos, self._sin,
                                     self.pos, self.k_cache[i], self.v_cache[i], self.attn_out,
                                     cfg.eps, rope=self.rope)
                g["o"](self.attn_out, W["o"][i], h=h)
            g["gu"](h, W["gu"][i], y=self.act, nw=lw["w_post"])
            g["down"](self.act, W["down"][i], h=h)
        g["lm"](h, W["lm"][0], y=self.logits, nw=self.w["final_norm"], ids=self.ids,
                pos_inc=self.pos, next_emb=self.w["embed"], next_h=h)

    def _capture(self, fn):
        # Warm up on a side stream, then capture. Warm-up steps write cache slot 0,
        # which the prefill of every generate() call overwrites.
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(2):
                self.pos.zero_()
                fn()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        self.pos.zero_()
        with torch.cuda.graph(g):
            fn()
        torch.cuda.synchronize()
        return g

    # ---------------------------------------------------------------- forward
    def _prefill(self, prompt):
        ids, logits = prefill(self.cfg, self.w, prompt, self.k_cache, self.v_cache, self._cos,
                              self._sin)
        self.ids.copy_(ids)
        self.pos.fill_(prompt.shape[1])
        embed_ss(self.ids, self.w["embed"], self.h, None)   # the first decode step's input
        if self.logits is not None:
            self.logits.copy_(logits)

    @torch.inference_mode()
    def step(self):
        """Replay one decode step (for callers that drive decoding themselves)."""
        self.g1.replay()

    @torch.inference_mode()
    def time_step(self, reps=20):
        """Mean GPU time (ms) of one replayed decode step, from positions S."""
        torch.cuda.synchronize()
        self.pos.fill_(self.S)
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
        self._setup(B, S, N)
        stream = torch.cuda.current_stream()
        prompt = torch.tensor(input_ids, dtype=torch.int64).pin_memory().to(DEVICE,
                                                                            non_blocking=True)
        self._prefill(prompt)
        ids_h, ev = self.pin_ids, self.events
        ids_h[0].copy_(self.ids, non_blocking=True)
        ev[0].record(stream)
        # Keep one replay in flight: queue step j before waiting for step j-1.
        if N > 1:
            self.g1.replay()
            ids_h[1].copy_(self.ids, non_blocking=True)
            ev[1].record(stream)
        ev[0].synchronize()
        yield ids_h[0].tolist()
        for j in range(1, N):
            if j + 1 < N:
                self.g1.replay()
                ids_h[j + 1].copy_(self.ids, non_blocking=True)
                ev[j + 1].record(stream)
            ev[j].synchronize()
            yield ids_h[j].tolist()

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
        return torch.stack(toks, 1), logits
