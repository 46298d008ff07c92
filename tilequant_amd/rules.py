"""Which nn.Linear modules become MixedLinear (mirror of src/models/rules.py).

Targets are the decoder projections q/k/v/o/gate/up/down of Llama- and
Qwen-family models (rules.py:9-28), optionally narrowed by fnmatch patterns in
``cfg.module_filters`` (rules.py:43-48).
"""
from __future__ import annotations

import fnmatch
from typing import Any, List, Tuple

import torch.nn as nn

TARGET_SUFFIXES = ("q_proj", "k_proj", "v_proj", "o_proj", "up_proj", "down_proj", "gate_proj")
LLAMA_TARGET_SUFFIXES = TARGET_SUFFIXES
QWEN_TARGET_SUFFIXES = TARGET_SUFFIXES


def _cfg_get(cfg: Any, key: str, default=None):
    if isinstance(cfg, dict):
        return cfg.get(key, default)
    return getattr(cfg, key, default)


def _suffixes(model_type: str):
    return QWEN_TARGET_SUFFIXES if "qwen" in model_type.lower() else LLAMA_TARGET_SUFFIXES


def should_quantize_name(full_name: str, cfg: Any) -> bool:
    patterns = _cfg_get(cfg, "module_filters", None)
    return not patterns or any(fnmatch.fnmatch(full_name, p) for p in patterns)


def iter_target_linears(model: nn.Module, cfg: Any, model_type: str = "llama") -> List[Tuple[nn.Module, str, str, nn.Linear]]:
    """(parent, attribute name, full name, linear) for every target linear."""
    suffixes = _suffixes(model_type)
    modules = dict(model.named_modules())
    found = []
    for full_name, module in model.named_modules():
        if not isinstance(module, nn.Linear) or not full_name.endswith(suffixes):
            continue
        if not should_quantize_name(full_name, cfg):
            continue
        if "." in full_name:
            parent_name, attr = full_name.rsplit(".", 1)
            parent = modules[parent_name]
        else:
            parent, attr = model, full_name
        found.append((parent, attr, full_name, module))
    return found
