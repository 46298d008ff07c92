"""Load-time packing driver (mirror of src/quantization/api.py).

``load_mixed_precision_model_from_masks`` keeps the reference's signature,
checks, statistics and errors (api.py:80-310): it builds the model skeleton
without memory, validates every target's Decision/ tile map against its
weight shape, streams the safetensors shards on the host, packs each target
weight as it arrives (this build's packer runs on the ROCm device) and swaps in
``MixedLinear``, loads every other tensor to the device, stacks Q/K/V and
Gate/Up into projection groups and ties the embeddings.

``build_mixed_precision_model`` is this build's direct path for a model that
exists only as a config (random initialisation, no checkpoint round trip):
weights are drawn on the device, packed there and never stored dense.
"""
from __future__ import annotations

import json
import math
import time
from pathlib import Path
from types import SimpleNamespace
from typing import Callable, Dict, Iterable, Optional, Tuple

import numpy as np
import torch
import torch.nn as nn

from .mask_io import load_fp16_keep_ids_for_layer
from .mixed_linear import MixedLinear, fuse_projection_groups
from .pack import pack_weight_from_tile_ids
from .rules import iter_target_linears
from .types import ApplyConfig


def _expected_tile_grid(shape: Iterable[int], tile_m: int, tile_n: int) -> Tuple[int, int]:
    m, k = (int(v) for v in list(shape)[:2])
    return -(-m // tile_m), -(-k // tile_n)


def _make_cfg(apply_cfg: ApplyConfig):
    """The cfg object every MixedLinear / packer call reads (api.py:48-59)."""
    return SimpleNamespace(
        tile_m=int(apply_cfg.tile.tile_m),
        tile_n=int(apply_cfg.tile.tile_n),
        precision_map_source="mask_keep",
        act_quant="per_tensor_absmax",
        weight_quant="per_tile_absmax",
        quant_style=str(getattr(apply_cfg, "quant_style", "gi")),
        dtype_out=str(apply_cfg.dtype_out),
        pad_to_tile=True,
        module_filters=list(apply_cfg.module_filters),
    )


def infer_model_type(model_dir_or_config) -> str:
    """'qwen' or 'llama' from a config's model_type (or a checkpoint's config.json)."""
    if isinstance(model_dir_or_config, (str, Path)):
        with open(Path(model_dir_or_config) / "config.json", "r", encoding="utf-8") as f:
            mt = str(json.load(f).get("model_type", "llama"))
    else:
        mt = str(getattr(model_dir_or_config, "model_type", "llama"))
    return "qwen" if "qwen" in mt.lower() else "llama"


def _load_iaa_channel_stats(keep_dir: Path, apply_cfg: ApplyConfig) -> Dict[str, torch.Tensor]:
    override = getattr(apply_cfg, "iaa_channel_stats_path", None)
    path = Path(str(override)) if override else Path(keep_dir).parent.parent / "iaa_channel_mean_abs.npz"
    if not path.exists():
        raise FileNotFoundError(
            f"IAA channel stats not found: {path}. "
            "Generate via build_decisions.py --quant_style iaa or pass --iaa_channel_stats_path."
        )
    with np.load(path, allow_pickle=False) as data:
        return {key: torch.from_numpy(np.asarray(data[key], dtype=np.float32)).contiguous() for key in data.files}


def _split_ids(fp16_ids: torch.Tensor, n_tr: int, n_tc: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """(fp16 ids int32, complementary int8 ids int32), ascending."""
    total = n_tr * n_tc
    keep = torch.zeros((total,), dtype=torch.bool)
    if fp16_ids.numel():
        keep[fp16_ids.to(torch.int64)] = True
    int8_ids = torch.nonzero(~keep, as_tuple=False).reshape(-1).to(torch.int32).contiguous()
    return fp16_ids.to(torch.int32).contiguous(), int8_ids


def validate_fp16_ids_coverage_and_shapes(model: nn.Module, keep_dir, apply_cfg: ApplyConfig
                                          ) -> Dict[str, Tuple[torch.Tensor, torch.Tensor, int, int]]:
    """Tile map of every target linear, checked against its weight (api.py:80-118):
    name -> (fp16 ids, int8 ids, n_tr, n_tc)."""
    cfg = _make_cfg(apply_cfg)
    targets = iter_target_linears(model, cfg=cfg, model_type=apply_cfg.model_type)
    if not targets:
        raise RuntimeError(f"No target linears found for model_type={apply_cfg.model_type}.")
    out: Dict[str, Tuple[torch.Tensor, torch.Tensor, int, int]] = {}
    for _, _, full_name, linear in targets:
        fp16_ids, (n_tr, n_tc) = load_fp16_keep_ids_for_layer(keep_dir=keep_dir, layer_name=full_name,
                                                             tile_m=cfg.tile_m, tile_n=cfg.tile_n)
        expected = _expected_tile_grid(linear.weight.shape, cfg.tile_m, cfg.tile_n)
        if (n_tr, n_tc) != expected:
            raise RuntimeError(f"FP16 keep-id shape mismatch for {full_name}: "
                               f"archive={(n_tr, n_tc)} expected={expected}")
        total = n_tr * n_tc
        if fp16_ids.numel() > 0:
            lo, hi = int(fp16_ids.min()), int(fp16_ids.max())
            if lo < 0 or hi >= total:
                raise RuntimeError(f"FP16 keep-id out of range for {full_name}: total_tiles={total} "
                                   f"min={lo} max={hi}")
        f16, i8 = _split_ids(fp16_ids, n_tr, n_tc)
        out[full_name] = (f16, i8, int(n_tr), int(n_tc))
    return out


def _resolve_safetensor_shards(local_model_dir: Path) -> Iterable[Path]:
    local_model_dir = Path(local_model_dir)
    index_path = local_model_dir / "model.safetensors.index.json"
    if index_path.exists():
        with open(index_path, "r", encoding="utf-8") as f:
            weight_map = json.load(f).get("weight_map", {})
        if not isinstance(weight_map, dict) or not weight_map:
            raise RuntimeError(f"Invalid or empty weight_map in index: {index_path}")
        for rel in sorted(set(weight_map.values())):
            shard = local_model_dir / rel
            if not shard.exists():
                raise RuntimeError(f"Missing shard file listed in index: {shard}")
            yield shard
        return
    single = local_model_dir / "model.safetensors"
    if single.exists():
        yield single
        return
    raise RuntimeError(f"No safetensors checkpoint found in {local_model_dir}. "
                       "Expected model.safetensors or model.safetensors.index.json.")


def _cast_loaded_tensor(tensor: torch.Tensor, torch_dtype: torch.dtype) -> torch.Tensor:
    return tensor.to(dtype=torch_dtype) if tensor.is_floating_point() else tensor


def _empty_model(config, torch_dtype: torch.dtype, attn_implementation: Optional[str]):
    from accelerate import init_empty_weights
    from transformers import AutoModelForCausalLM

    kwargs = {"attn_implementation": attn_implementation} if attn_implementation else {}
    with init_empty_weights():
        return AutoModelForCausalLM.from_config(config, dtype=torch_dtype, **kwargs)


def _buffers_to_device(model: nn.Module, device: torch.device) -> None:
    """Buffers the checkpoint does not hold (RoPE inv_freq ...) are created on
    the host by from_config; move them so no forward copies host -> device
    (which graph capture would reject), as the reference does (api.py:281-292)."""
    for module in model.modules():
        for name, buf in list(module._buffers.items()):
            if buf is not None and buf.device != device and buf.device.type != "meta":
                module._buffers[name] = buf.to(device)
        for attr in ("original_inv_freq",):
            value = getattr(module, attr, None)
            if isinstance(value, torch.Tensor) and value.device != device:
                setattr(module, attr, value.to(device))


def _finish(model: nn.Module, device: torch.device) -> int:
    _buffers_to_device(model, device)
    fused = fuse_projection_groups(model)
    if hasattr(model, "tie_weights"):
        model.tie_weights()
    model.eval()
    return fused


def load_mixed_precision_model_from_masks(local_model_dir, keep_dir, apply_cfg: ApplyConfig,
                                          torch_dtype: torch.dtype, device, attn_implementation: Optional[str] = None):
    """Load checkpoint shards and pack the target linears during the load (api.py:154-310)."""
    from accelerate.utils.modeling import set_module_tensor_to_device
    from safetensors import safe_open
    from transformers import AutoConfig

    local_model_dir = Path(local_model_dir)
    started = time.perf_counter()
    cfg = _make_cfg(apply_cfg)
    device = torch.device(device)
    config_kwargs = {"attn_implementation": attn_implementation} if attn_implementation else {}
    config = AutoConfig.from_pretrained(str(local_model_dir), **config_kwargs)
    model = _empty_model(config, torch_dtype, attn_implementation)

    targets = iter_target_linears(model, cfg=cfg, model_type=apply_cfg.model_type)
    if not targets:
        raise RuntimeError(f"No target linears found for model_type={apply_cfg.model_type}.")
    target_meta = {full_name: (parent, attr) for parent, attr, full_name, _ in targets}
    fp16_data = validate_fp16_ids_coverage_and_shapes(model=model, keep_dir=keep_dir, apply_cfg=apply_cfg)
    target_names = set(fp16_data)
    quant_style = str(getattr(apply_cfg, "quant_style", "gi")).lower()
    iaa_stats = _load_iaa_channel_stats(Path(keep_dir), apply_cfg) if quant_style == "iaa" else {}

    pending_bias: Dict[str, torch.Tensor] = {}
    loaded_non_target = replaced = 0
    pack_total = non_target_total = 0.0
    for shard in _resolve_safetensor_shards(local_model_dir):
        with safe_open(str(shard), framework="pt", device="cpu") as sf:
            for key in sf.keys():
                tensor = sf.get_tensor(key)
                if key.endswith(".weight") and key[: -len(".weight")] in target_names:
                    name = key[: -len(".weight")]
                    t0 = time.perf_counter()
                    parent, attr = target_meta[name]
                    fp16_ids, int8_ids, n_tr, n_tc = fp16_data[name]
                    imp = iaa_stats.get(name.replace(".", "_")) if quant_style == "iaa" else None
                    pack = pack_weight_from_tile_ids(_cast_loaded_tensor(tensor, torch_dtype), int8_tile_ids=int8_ids,
                                                     fp16_tile_ids=fp16_ids, n_tr=n_tr, n_tc=n_tc,
                                                     iaa_col_importance=imp, cfg=cfg)
                    mod = MixedLinear(pack=pack, bias=None, cfg=cfg).to(device)
                    setattr(parent, attr, mod)
                    replaced += 1
                    if name in pending_bias:
                        bias = _cast_loaded_tensor(pending_bias.pop(name), torch_dtype)
                        mod.bias = nn.Parameter(bias.to(device=device).detach().clone(), requires_grad=False)
                    pack_total += time.perf_counter() - t0
                    continue
                if key.endswith(".bias") and key[: -len(".bias")] in target_names:
                    name = key[: -len(".bias")]
                    mod = dict(model.named_modules()).get(name)
                    if isinstance(mod, MixedLinear):
                        bias = _cast_loaded_tensor(tensor, torch_dtype)
                        mod.bias = nn.Parameter(bias.to(device=device).detach().clone(), requires_grad=False)
                    else:
                        pending_bias[name] = tensor
                    continue
                t0 = time.perf_counter()
                set_module_tensor_to_device(model, key, device, value=_cast_loaded_tensor(tensor, torch_dtype))
                non_target_total += time.perf_counter() - t0
                loaded_non_target += 1
    if pending_bias:
        raise RuntimeError("Found target bias tensors without corresponding target weight loads, "
                           f"e.g. {list(pending_bias)[:3]}")
    modules = dict(model.named_modules())
    for name in target_names:
        if not isinstance(modules.get(name), MixedLinear):
            raise RuntimeError(f"Target module is not MixedLinear after load-time apply: {name}")
    fused = _finish(model, device)
    return model, {
        "num_targets": len(target_names),
        "num_replaced": len(target_names),
        "num_replaced_during_load": replaced,
        "num_loaded_non_target_tensors": loaded_non_target,
        "load_total": float(time.perf_counter() - started),
        "quant_pack_total": float(pack_total),
        "non_target_load_total": float(non_target_total),
        "attn_implementation": attn_implementation,
        "fused_projection_groups": int(fused),
    }


def uniform_fp16_tile_ids(n_tr: int, n_tc: int, frac: float, rng: np.random.Generator) -> torch.Tensor:
    """Seeded uniform tile map: k = max(1, ceil(frac * tiles)) BF16 tiles drawn
    without replacement (the reference's k rule, decisions.py:176), ascending."""
    n = n_tr * n_tc
    k = max(1, int(math.ceil(frac * n))) if frac > 0 else 0
    ids = np.sort(rng.choice(n, size=k, replace=False)) if k else np.zeros(0, np.int64)
    return torch.from_numpy(ids.astype(np.int32))


def build_mixed_precision_model(config, apply_cfg: ApplyConfig, device, torch_dtype: torch.dtype = torch.bfloat16,
                                fp16_ids_for: Optional[Callable[[str, int, int], torch.Tensor]] = None,
                                keep_dir=None, keep_frac: float = 0.01, seed: int = 0, init_std: float = 0.02,
                                attn_implementation: str = "sdpa"):
    """Random-init model of ``config`` with every target linear packed as MixedLinear.

    Weights are drawn on the device (seeded N(0, init_std) for every matrix,
    ones for norms), then each target weight is packed with its tile map --
    from ``fp16_ids_for(name, n_tr, n_tc)``, a Decision/ archive ``keep_dir``,
    or seeded uniform masks at ``keep_frac`` -- and dropped.  Returns
    (model, stats) like the checkpoint loader."""
    device = torch.device(device)
    started = time.perf_counter()
    cfg = _make_cfg(apply_cfg)
    model = _empty_model(config, torch_dtype, attn_implementation)
    targets = iter_target_linears(model, cfg=cfg, model_type=apply_cfg.model_type)
    if not targets:
        raise RuntimeError(f"No target linears found for model_type={apply_cfg.model_type}.")
    if keep_dir is not None:
        maps = validate_fp16_ids_coverage_and_shapes(model, keep_dir, apply_cfg)
    rng = np.random.default_rng(seed)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)

    def draw(shape):
        return (torch.randn(shape, generator=gen, device=device, dtype=torch.float32) * init_std).to(torch_dtype)

    target_names = {full for _, _, full, _ in targets}
    pack_total = 0.0
    for parent, attr, full_name, linear in targets:
        shape = tuple(linear.weight.shape)
        n_tr, n_tc = _expected_tile_grid(shape, cfg.tile_m, cfg.tile_n)
        if keep_dir is not None:
            f16, i8, n_tr, n_tc = maps[full_name]
        else:
            ids = fp16_ids_for(full_name, n_tr, n_tc) if fp16_ids_for is not None else uniform_fp16_tile_ids(
                n_tr, n_tc, keep_frac, rng)
            f16, i8 = _split_ids(ids, n_tr, n_tc)
        t0 = time.perf_counter()
        W = draw(shape)
        pack = pack_weight_from_tile_ids(W, n_tr=n_tr, n_tc=n_tc, int8_tile_ids=i8, fp16_tile_ids=f16, cfg=cfg)
        del W
        bias = draw((shape[0],)) if linear.bias is not None else None
        setattr(parent, attr, MixedLinear(pack=pack, bias=bias, cfg=cfg).to(device))
        pack_total += time.perf_counter() - t0
    # every remaining parameter / buffer: materialise on the device
    for name, p in list(model.named_parameters()):
        if p.device.type != "meta":
            continue
        mod_name, _, leaf = name.rpartition(".")
        owner = model.get_submodule(mod_name) if mod_name else model
        if leaf == "weight" and "norm" in mod_name.lower():
            value = torch.ones(p.shape, device=device, dtype=torch_dtype)
        else:
            value = draw(tuple(p.shape))
        owner._parameters[leaf] = nn.Parameter(value, requires_grad=False)
    for mod in model.modules():
        for bname, buf in list(mod._buffers.items()):
            if buf is not None and buf.device.type == "meta":
                raise RuntimeError(f"buffer {bname} of {type(mod).__name__} has no value")
    if getattr(config, "tie_word_embeddings", False) and hasattr(model, "lm_head"):
        model.lm_head.weight = model.get_input_embeddings().weight
    fused = _finish(model, device)
    return model, {"num_targets": len(target_names), "quant_pack_total": float(pack_total),
                   "load_total": float(time.perf_counter() - started), "fused_projection_groups": int(fused)}
