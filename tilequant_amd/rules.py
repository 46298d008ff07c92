"""Selection of the nn.Linear modules that become MixedLinear (the role of
src/models/rules.py).

A module is a target when its qualified name ends in one of the decoder
projection names of its model family (rules.py:9-28) and, when
``cfg.module_filters`` holds fnmatch patterns, matches at least one of them
(rules.py:43-48).
"""
from __future__ import annotations

import fnmatch
from typing import Any, List, Tuple

import torch.nn as nn

from ._config import cfg_value

TARGET_SUFFIXES = ("q_proj", "k_proj", "v_proj", "o_proj", "up_proj", "down_proj", "gate_proj")
# Both supported families name their projections alike; the per-family names
# stay public for callers that import them.
LLAMA_TARGET_SUFFIXES = TARGET_SUFFIXES
QWEN_TARGET_SUFFIXES = TARGET_SUFFIXES
_FAMILY_SUFFIXES = (("qwen", QWEN_TARGET_SUFFIXES),)


def target_suffixes(model_type: str) -> Tuple[str, ...]:
    """Projection-name suffixes for a model type string ("llama", "qwen2", ...)."""
    kind = model_type.lower()
    return next((names for family, names in _FAMILY_SUFFIXES if family in kind), LLAMA_TARGET_SUFFIXES)


def should_quantize_name(full_name: str, cfg: Any) -> bool:
    """True unless cfg.module_filters is set and no pattern matches the name."""
    patterns = cfg_value(cfg, "module_filters")
    return not patterns or any(fnmatch.fnmatch(full_name, pattern) for pattern in patterns)


def iter_target_linears(model: nn.Module, cfg: Any,
                        model_type: str = "llama") -> List[Tuple[nn.Module, str, str, nn.Linear]]:
    """(parent module, attribute name, qualified name, linear) of every target,
    in module registration order."""
    names = target_suffixes(model_type)
    by_name = dict(model.named_modules())
    targets = []
    for qualified, module in by_name.items():
        if isinstance(module, nn.Linear) and qualified.endswith(names) and should_quantize_name(qualified, cfg):
            parent, _, attr = qualified.rpartition(".")
            targets.append((by_name[parent], attr, qualified, module))
    return targets
