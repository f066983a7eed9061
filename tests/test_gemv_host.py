"""Host logic of the Gemv op (CPU, no kernel launches): the drop-in rule for the
MFMA-tiled layouts. The reference engine builds ``Gemv`` objects, calls
``tune(weights, deadline)`` with its row-major weights only and a load-time
deadline that may have passed (engine/engine.py:245-272), then calls them with
those row-major weights. So the default configuration must read row-major
weights, an expired deadline must leave it in place, and a tiled configuration
must never read a row-major tensor as if it were tiled."""

import time

import pytest
import torch

from kernel_optim_amd.kernels.gemv import (EPI_ARGMAX, EPI_BF16, EPI_F32, EPI_RESID, EPI_SWIGLU,
                                           Gemv, is_tiled, uses_tiled)

H, I, NQKV, V = 2560, 9728, 6144, 151936
# the reference decode step's projections (engine.py:256-262)
SHAPES = [(NQKV, H, EPI_F32, True), (H, 4096, EPI_RESID, False), (I, H, EPI_SWIGLU, True),
          (H, I, EPI_RESID, False), (V, H, EPI_BF16, True), (V, H, EPI_ARGMAX, True)]


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 16, 17, 64])
def test_default_config_reads_row_major_weights(M):
    for N, K, epi, norm in SHAPES:
        g = Gemv(M, N, K, epi, norm, allow_split=True)
        assert not uses_tiled(g.cfg), (M, N, K, epi, g.cfg)
        assert g.cfg == g.candidates()[0]


@pytest.mark.parametrize("M", [5, 16])
def test_expired_deadline_keeps_the_row_major_default(M):
    """The case the reference hits once its tuning budget is spent (engine.py:45,265)."""
    w = [torch.zeros(NQKV, H, dtype=torch.bfloat16) for _ in range(2)]
    g = Gemv(M, NQKV, H, EPI_F32, True, allow_split=True)
    cfg = g.tune(w, time.monotonic() - 1.0)
    assert cfg == g.cfg and not uses_tiled(cfg)


def test_tiled_config_refuses_a_row_major_weight_without_a_copy():
    g = Gemv(16, NQKV, H, EPI_BF16, True)
    w = torch.zeros(NQKV, H, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="no tiled copy"):
        g._weight_for(w, (2, 2, 0))
    # with a copy remembered by tune, the row-major weight maps to it
    t = torch.zeros(NQKV, H, dtype=torch.bfloat16)
    t._ko_tiled = True
    g._remember_tiles([w], [t])
    assert g._weight_for(w, (2, 2, 0)) is t
    assert g._weight_for(t, (3, 1, 0)) is t
    # another tensor of the same shape is not mapped
    with pytest.raises(ValueError):
        g._weight_for(w.clone(), (2, 2, 0))


def test_row_major_config_refuses_a_tiled_copy():
    g = Gemv(1, NQKV, H, EPI_BF16, True)
    t = torch.zeros(NQKV, H, dtype=torch.bfloat16)
    t._ko_tiled = True
    assert is_tiled(t)
    with pytest.raises(ValueError, match="row-major"):
        g._weight_for(t, (0, 8, 0))
    w = torch.zeros(NQKV, H, dtype=torch.bfloat16)
    assert g._weight_for(w, (0, 8, 0)) is w


def test_engine_refuses_a_directory_without_weights(tmp_path, monkeypatch):
    """A config.json with no *.safetensors is not a model: the engine raises instead
    of decoding random weights, unless ENGINE_RANDOM_INIT=1 asks for them."""
    import json
    from kernel_optim_amd.engine import Engine
    from kernel_optim_amd.model import Qwen3Config
    (tmp_path / "config.json").write_text(json.dumps(Qwen3Config().to_hf_json()))
    (tmp_path / "pytorch_model.bin").write_bytes(b"")
    monkeypatch.delenv("ENGINE_RANDOM_INIT", raising=False)
    with pytest.raises(FileNotFoundError, match="safetensors"):
        Engine(str(tmp_path))
