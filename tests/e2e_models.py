"""Tiny Llama / Qwen2 configs and checkpoints for loader and decoder tests
(random weights written locally with safetensors; nothing is downloaded)."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch


def tiny_llama_config(layers: int = 2, vocab: int = 512):
    from transformers import LlamaConfig

    return LlamaConfig(vocab_size=vocab, hidden_size=512, intermediate_size=1024, num_hidden_layers=layers,
                       num_attention_heads=4, num_key_value_heads=2, head_dim=128, rope_theta=5e5,
                       max_position_embeddings=4096, tie_word_embeddings=True, rms_norm_eps=1e-5,
                       attn_implementation="sdpa")


def tiny_qwen2_config(layers: int = 2, vocab: int = 512):
    from transformers import Qwen2Config

    return Qwen2Config(vocab_size=vocab, hidden_size=512, intermediate_size=1024, num_hidden_layers=layers,
                       num_attention_heads=4, num_key_value_heads=2, rope_theta=1e6,
                       max_position_embeddings=4096, tie_word_embeddings=False, rms_norm_eps=1e-6,
                       attn_implementation="sdpa")


def write_checkpoint(config, out_dir: Path, seed: int = 0, shards: int = 1) -> dict:
    """Random weights (N(0, 0.02); norms 1) saved as safetensors shards + config.json."""
    from safetensors.torch import save_file
    from transformers import AutoModelForCausalLM

    torch.manual_seed(seed)
    model = AutoModelForCausalLM.from_config(config, dtype=torch.bfloat16)
    sd = {}
    g = torch.Generator().manual_seed(seed)
    for name, p in model.state_dict().items():
        if name == "lm_head.weight" and getattr(config, "tie_word_embeddings", False):
            continue
        if "norm" in name:
            sd[name] = torch.ones_like(p)
        else:
            sd[name] = (torch.randn(p.shape, generator=g) * 0.02).to(torch.bfloat16)
    out_dir.mkdir(parents=True, exist_ok=True)
    config.save_pretrained(out_dir)
    keys = sorted(sd)
    if shards == 1:
        save_file({k: sd[k].contiguous() for k in keys}, str(out_dir / "model.safetensors"))
    else:
        import json

        per = -(-len(keys) // shards)
        wmap = {}
        for i in range(shards):
            part = keys[i * per:(i + 1) * per]
            fname = f"model-{i + 1:05d}-of-{shards:05d}.safetensors"
            save_file({k: sd[k].contiguous() for k in part}, str(out_dir / fname))
            wmap.update({k: fname for k in part})
        with open(out_dir / "model.safetensors.index.json", "w") as f:
            json.dump({"metadata": {}, "weight_map": wmap}, f)
    return sd


def target_shapes(config, model_type: str = "llama") -> dict:
    """full module name -> (out, in) of every target linear of the config."""
    from accelerate import init_empty_weights
    from transformers import AutoModelForCausalLM
    from tilequant_amd.rules import iter_target_linears

    with init_empty_weights():
        model = AutoModelForCausalLM.from_config(config)
    return {full: tuple(lin.weight.shape) for _, _, full, lin in iter_target_linears(model, {}, model_type)}


def write_tile_maps(config, keep_dir: Path, frac: float = 0.1, seed: int = 0, model_type: str = "llama") -> dict:
    """Decision/-format archive with seeded uniform BF16 tile masks for every target."""
    from tilequant_amd import mask_io

    rng = np.random.default_rng(seed)
    masks = {}
    for name, (m, k) in target_shapes(config, model_type).items():
        n_tr, n_tc = -(-m // 64), -(-k // 64)
        mask = np.zeros((n_tr, n_tc), np.uint8)
        kk = max(1, int(np.ceil(frac * n_tr * n_tc)))
        mask.reshape(-1)[rng.choice(n_tr * n_tc, size=kk, replace=False)] = 1
        masks[mask_io.layer_name_to_stem(name)] = mask
    mask_io.save_mask_keep_archive(keep_dir, masks)
    return masks


# the Llama-3.2-3B architecture (28 layers, hidden 3072,
# 24 q / 8 kv heads of 128, MLP 8192, vocab 128256, tied embeddings, RMSNorm,
# RoPE theta 5e5), random-initialised -- the same dictionary bench.py uses.
LLAMA32_3B = dict(vocab_size=128256, hidden_size=3072, intermediate_size=8192, num_hidden_layers=28,
                  num_attention_heads=24, num_key_value_heads=8, head_dim=128, rope_theta=5e5, rms_norm_eps=1e-5,
                  max_position_embeddings=131072, tie_word_embeddings=True)


def llama32_3b_config():
    from transformers import LlamaConfig

    return LlamaConfig(**LLAMA32_3B, attn_implementation="sdpa")
