"""Seeded random-init Qwen3-shape checkpoints (config.json + HF tensor names).

There is no network and no real checkpoint here, so the decode path is exercised on synthetic
weights of the real architecture: bf16 weights ~ N(0, 0.02), RMSNorm weights 1 + N(0, 0.02)
(the distribution the workload configs name). Tensors are produced in a fixed order from one
seeded ``torch.Generator`` on the requested device, so the same (config, seed, device) always
yields the same bits; CPU and GPU generators differ, so share weights by copying, not by
regenerating on the other device.

Tensor names follow the HF Qwen3 layout the reference loader reads (engine.py:286-308).
"""
import json
import os

import torch

QWEN3_4B = {
    "architectures": ["Qwen3ForCausalLM"],
    "model_type": "qwen3",
    "vocab_size": 151936,
    "hidden_size": 2560,
    "intermediate_size": 9728,
    "num_hidden_layers": 36,
    "num_attention_heads": 32,
    "num_key_value_heads": 8,
    "head_dim": 128,
    "rms_norm_eps": 1e-6,
    "rope_theta": 5000000.0,
    "tie_word_embeddings": True,
    "max_position_embeddings": 40960,
    "hidden_act": "silu",
    "torch_dtype": "bfloat16",
}


def qwen3_config(**overrides):
    """The Qwen3-4B shape, with any field overridden (e.g. num_hidden_layers=2)."""
    cfg = dict(QWEN3_4B)
    cfg.update(overrides)
    return cfg


def tensor_shapes(cfg):
    """(name, shape, kind) in generation order; kind is 'w' (N(0, .02)) or 'n' (1 + N(0, .02))."""
    H, I, V = cfg["hidden_size"], cfg["intermediate_size"], cfg["vocab_size"]
    nh, nkv = cfg["num_attention_heads"], cfg["num_key_value_heads"]
    hd = cfg.get("head_dim") or H // nh
    out = [("model.embed_tokens.weight", (V, H), "w")]
    for i in range(cfg["num_hidden_layers"]):
        p = f"model.layers.{i}."
        out += [
            (p + "input_layernorm.weight", (H,), "n"),
            (p + "self_attn.q_proj.weight", (nh * hd, H), "w"),
            (p + "self_attn.k_proj.weight", (nkv * hd, H), "w"),
            (p + "self_attn.v_proj.weight", (nkv * hd, H), "w"),
            (p + "self_attn.q_norm.weight", (hd,), "n"),
            (p + "self_attn.k_norm.weight", (hd,), "n"),
            (p + "self_attn.o_proj.weight", (H, nh * hd), "w"),
            (p + "post_attention_layernorm.weight", (H,), "n"),
            (p + "mlp.gate_proj.weight", (I, H), "w"),
            (p + "mlp.up_proj.weight", (I, H), "w"),
            (p + "mlp.down_proj.weight", (H, I), "w"),
        ]
    out.append(("model.norm.weight", (H,), "n"))
    if not cfg.get("tie_word_embeddings", True):
        out.append(("lm_head.weight", (V, H), "w"))
    return out


@torch.no_grad()
def random_weights(cfg, seed=0, device="cpu", dtype=torch.bfloat16, std=0.02):
    """dict name -> tensor, generated in ``tensor_shapes`` order from one seeded generator."""
    g = torch.Generator(device=device).manual_seed(seed)
    w = {}
    for name, shape, kind in tensor_shapes(cfg):
        t = torch.randn(shape, generator=g, device=device, dtype=torch.float32).mul_(std)
        if kind == "n":
            t.add_(1.0)
        w[name] = t.to(dtype)
    return w


def write_model(path, cfg, weights):
    """Write config.json + model.safetensors (HF names) into ``path``."""
    from safetensors.torch import save_file
    os.makedirs(path, exist_ok=True)
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(cfg, f, indent=1)
    save_file({k: v.contiguous().cpu() for k, v in weights.items()},
              os.path.join(path, "model.safetensors"))
