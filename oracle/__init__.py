"""CPU oracle for the decode hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU with PyTorch (fp32/fp64), the algorithms of
the reference's decode path (engine/kernels/fused.py, engine/kernels/gemv.py,
engine/engine.py) and of the Transformers Qwen3 eager forward it mirrors.
Each function cites the reference file:line it follows.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import it, and only as the reference results are compared with (or the timed
CPU baseline). The product path (kernel_optim_amd) never imports or calls
anything here.

Pinning (how each function is checked independently of its own formula):
- attention.decode_attention: fp64 closed form; checked against torch SDPA
  (library routine), brute-force Python loops on tiny inputs, and closed-form
  special cases (uniform scores -> mean of V, one dominant key -> its V row).
- attention.decode_attention_splitk: the reference's split-K algorithm
  (fused.py:138-201) restated; checked to equal the closed form for every
  split count, and an empty split contributes nothing.
- ops.*: cast chains checked bit-for-bit (or to 1 bf16 ulp where only a
  reduction order differs) against the Transformers Qwen3 modules
  (Qwen3RMSNorm, Qwen3RotaryEmbedding, apply_rotary_pos_emb, Qwen3MLP) and
  torch library routines (F.linear, F.silu, torch.argmax).
- qwen3.*: the full forward checked against transformers' Qwen3ForCausalLM at
  random init (logits within tolerance, identical greedy tokens).
"""
