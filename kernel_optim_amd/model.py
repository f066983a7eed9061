"""Qwen3 model description and weights in the decode layout.

The engine keeps, per layer, the concatenated q|k|v projection [6144, 2560] and
gate|up projection [19456, 2560] exactly as the reference builds them
(engine/engine.py:143-154), so each decode projection is one weight stream.

Weights come from a local checkpoint directory (config.json + *.safetensors,
read with safetensors, nothing executed from the files) or are drawn at random
from N(0, 0.02) with a seed (norm gains 1, tied embedding), the synthetic
Qwen3-4B-architecture model the benchmarks run.
"""

import glob
import json
import os
from dataclasses import dataclass

import torch

BF16 = torch.bfloat16


@dataclass
class Qwen3Config:
    hidden: int = 2560
    inter: int = 9728
    layers: int = 36
    nq: int = 32
    nkv: int = 8
    head_dim: int = 128
    vocab: int = 151936
    eps: float = 1e-6
    theta: float = 1.0e6
    tied: bool = True

    @property
    def nqkv(self):
        return (self.nq + 2 * self.nkv) * self.head_dim

    @classmethod
    def from_hf_json(cls, path):
        """Read a Hugging Face config.json (Qwen3ForCausalLM keys)."""
        with open(path) as f:
            c = json.load(f)
        theta = c.get("rope_theta")
        if theta is None:
            theta = (c.get("rope_parameters") or {}).get("rope_theta", 1.0e6)
        return cls(hidden=c["hidden_size"], inter=c["intermediate_size"],
                   layers=c["num_hidden_layers"], nq=c["num_attention_heads"],
                   nkv=c["num_key_value_heads"],
                   head_dim=c.get("head_dim") or c["hidden_size"] // c["num_attention_heads"],
                   vocab=c["vocab_size"], eps=c.get("rms_norm_eps", 1e-6), theta=float(theta),
                   tied=bool(c.get("tie_word_embeddings", True)))

    def to_hf_json(self):
        return {"architectures": ["Qwen3ForCausalLM"], "model_type": "qwen3",
                "hidden_size": self.hidden, "intermediate_size": self.inter,
                "num_hidden_layers": self.layers, "num_attention_heads": self.nq,
                "num_key_value_heads": self.nkv, "head_dim": self.head_dim,
                "vocab_size": self.vocab, "rms_norm_eps": self.eps, "rope_theta": self.theta,
                "tie_word_embeddings": self.tied, "hidden_act": "silu",
                "max_position_embeddings": 40960, "torch_dtype": "bfloat16"}

    def layer_bytes(self):
        """bf16 weight bytes of one decoder layer."""
        h, d = self.hidden, self.head_dim
        mats = self.nqkv * h + self.nq * d * h + 2 * self.inter * h + h * self.inter
        return 2 * (mats + 2 * h + 2 * d)

    def weight_bytes_per_step(self):
        """Bytes streamed by one decode step: every layer + final norm + LM head."""
        return self.layers * self.layer_bytes() + 2 * self.hidden + 2 * self.vocab * self.hidden


def random_weights(cfg, seed=0, device="cpu", std=0.02):
    """Seeded N(0, std) bf16 weights in the decode layout; norm gains are 1 (the
    Transformers initialisation of Qwen3RMSNorm); the LM head is the embedding."""
    g = torch.Generator(device=device).manual_seed(seed)

    def randn(*shape):
        return (torch.randn(*shape, generator=g, device=device) * std).to(BF16)

    h, d = cfg.hidden, cfg.head_dim
    ones = lambda n: torch.ones(n, dtype=BF16, device=device)
    embed = randn(cfg.vocab, h)
    layers = []
    for _ in range(cfg.layers):
        layers.append(dict(
            w_in=ones(h), w_post=ones(h),
            qkv=randn(cfg.nqkv, h), q_norm=ones(d), k_norm=ones(d),
            o=randn(h, cfg.nq * d),
            gu=randn(2 * cfg.inter, h),
            down=randn(h, cfg.inter),
        ))
    lm_head = embed if cfg.tied else randn(cfg.vocab, h)
    return dict(embed=embed, lm_head=lm_head, final_norm=ones(h), layers=layers)


def weights_to(w, device):
    out = dict(embed=w["embed"].to(device), final_norm=w["final_norm"].to(device),
               layers=[{k: v.to(device) for k, v in l.items()} for l in w["layers"]])
    out["lm_head"] = out["embed"] if w["lm_head"] is w["embed"] else w["lm_head"].to(device)
    return out


def load_checkpoint(path, device="cpu"):
    """(config, weights) from a local HF Qwen3 directory: config.json and
    *.safetensors shards. Builds the concatenated qkv / gate-up layout."""
    from safetensors.torch import load_file
    cfg = Qwen3Config.from_hf_json(os.path.join(path, "config.json"))
    shards = sorted(glob.glob(os.path.join(path, "*.safetensors")))
    if not shards:
        raise FileNotFoundError(f"no *.safetensors under {path}")
    sd = {}
    for s in shards:
        sd.update(load_file(s, device="cpu"))
    get = lambda k: sd[k].to(BF16)
    layers = []
    for i in range(cfg.layers):
        p = f"model.layers.{i}."
        layers.append(dict(
            w_in=get(p + "input_layernorm.weight"),
            w_post=get(p + "post_attention_layernorm.weight"),
            qkv=torch.cat([get(p + "self_attn.q_proj.weight"), get(p + "self_attn.k_proj.weight"),
                           get(p + "self_attn.v_proj.weight")], 0).contiguous(),
            q_norm=get(p + "self_attn.q_norm.weight"), k_norm=get(p + "self_attn.k_norm.weight"),
            o=get(p + "self_attn.o_proj.weight"),
            gu=torch.cat([get(p + "mlp.gate_proj.weight"), get(p + "mlp.up_proj.weight")],
                         0).contiguous(),
            down=get(p + "mlp.down_proj.weight"),
        ))
    embed = get("model.embed_tokens.weight")
    lm = embed if cfg.tied or "lm_head.weight" not in sd else get("lm_head.weight")
    w = dict(embed=embed, lm_head=lm, final_norm=get("model.norm.weight"), layers=layers)
    return cfg, weights_to(w, device)


def to_hf_state_dict(cfg, weights):
    """CPU state dict with the Hugging Face Qwen3ForCausalLM parameter names."""
    nq, nkv, d, I = cfg.nq, cfg.nkv, cfg.head_dim, cfg.inter
    sd = {"model.embed_tokens.weight": weights["embed"].cpu().contiguous(),
          "model.norm.weight": weights["final_norm"].cpu().contiguous()}
    sd["lm_head.weight"] = (sd["model.embed_tokens.weight"] if cfg.tied
                            else weights["lm_head"].cpu().contiguous())
    for i, l in enumerate(weights["layers"]):
        p = f"model.layers.{i}."
        qkv = l["qkv"].cpu()
        sd[p + "self_attn.q_proj.weight"] = qkv[:nq * d].contiguous()
        sd[p + "self_attn.k_proj.weight"] = qkv[nq * d:(nq + nkv) * d].contiguous()
        sd[p + "self_attn.v_proj.weight"] = qkv[(nq + nkv) * d:].contiguous()
        sd[p + "self_attn.o_proj.weight"] = l["o"].cpu().contiguous()
        sd[p + "self_attn.q_norm.weight"] = l["q_norm"].cpu().contiguous()
        sd[p + "self_attn.k_norm.weight"] = l["k_norm"].cpu().contiguous()
        sd[p + "mlp.gate_proj.weight"] = l["gu"][:I].cpu().contiguous()
        sd[p + "mlp.up_proj.weight"] = l["gu"][I:].cpu().contiguous()
        sd[p + "mlp.down_proj.weight"] = l["down"].cpu().contiguous()
        sd[p + "input_layernorm.weight"] = l["w_in"].cpu().contiguous()
        sd[p + "post_attention_layernorm.weight"] = l["w_post"].cpu().contiguous()
    return sd


def save_checkpoint(path, cfg, weights):
    """Write weights in the HF layout (config.json + model.safetensors)."""
    from safetensors.torch import save_file
    os.makedirs(path, exist_ok=True)
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(cfg.to_hf_json(), f, indent=1)
    sd = to_hf_state_dict(cfg, weights)
    if cfg.tied:
        del sd["lm_head.weight"]
    save_file(sd, os.path.join(path, "model.safetensors"))

