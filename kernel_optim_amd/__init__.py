"""MI355X-native (gfx950) split-K GQA decode attention and fused Qwen3 decode ops.

Host code is Python on PyTorch-ROCm; the kernels are hand-written HIP for
CDNA4 in ``csrc/``, compiled into the in-tree ``libkoptim.so`` (see
``kernel_optim_amd.build``) and called through its C ABI
(``include/koptim.h``) with ctypes.

- ``kernel_optim_amd.kernels.fused`` / ``.gemv``: the op library, with the
  signatures of the reference's engine/kernels/fused.py and gemv.py.
- ``kernel_optim_amd.engine.Engine``: ``Engine(model_path).generate(input_ids,
  max_new_tokens)``, the reference's engine surface.
"""
