"""Configuration lookup shared by the modules that take the reference's cfg
objects: a mapping, a dataclass such as ``types.ApplyConfig``, or any
attribute namespace."""
from __future__ import annotations

from collections.abc import Mapping
from typing import Any


def cfg_value(cfg: Any, key: str, default: Any = None) -> Any:
    """``cfg[key]`` for mappings, ``cfg.key`` otherwise; ``default`` when the
    key is absent or there is no cfg at all."""
    if cfg is None:
        return default
    if isinstance(cfg, Mapping):
        return cfg.get(key, default)
    return getattr(cfg, key, default)
