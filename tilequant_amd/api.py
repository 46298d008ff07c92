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
from typing import Callable, Dict, Iterable, Iterator, List, Optional, Tuple

import numpy as np
import torch
import torch.nn as nn
from accelerate.utils.modeling import set_module_tensor_to_device

from .mask_io import load_fp16_keep_ids_for_layer
from .mixed_linear import MixedLinear, fuse_projection_groups
from .pack import pack_weight_from_tile_ids
from .rules import iter_target_linears
from .types import ApplyConfig


def _tile_grid(weight_shape: Iterable[int], tile_m: int, tile_n: int) -> Tuple[int, int]:
    """(row tiles, column tiles) of a weight padded to whole tiles."""
    rows, cols = (int(v) for v in list(weight_shape)[:2])
    return -(-rows // tile_m), -(-cols // tile_n)


def _make_cfg(apply_cfg: ApplyConfig):
    """The cfg object every MixedLinear / packer call reads (the reference's
    field set, api.py:48-59)."""
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
        text = (Path(model_dir_or_config) / "config.json").read_text(encoding="utf-8")
        model_type = str(json.loads(text).get("model_type", "llama"))
    else:
        model_type = str(getattr(model_dir_or_config, "model_type", "llama"))
    return "qwen" if "qwen" in model_type.lower() else "llama"


def _load_iaa_channel_stats(keep_dir: Path, apply_cfg: ApplyConfig) -> Dict[str, torch.Tensor]:
    """stem -> fp32 per-input-channel importance for IAA packing: the file
    named by apply_cfg.iaa_channel_stats_path, else iaa_channel_mean_abs.npz two
    levels above the keep directory (the Decision/ layout)."""
    override = getattr(apply_cfg, "iaa_channel_stats_path", None)
    path = Path(str(override)) if override else Path(keep_dir).parent.parent / "iaa_channel_mean_abs.npz"
    if not path.is_file():
        raise FileNotFoundError(
            f"IAA channel stats not found: {path}. "
            "Generate via build_decisions.py --quant_style iaa or pass --iaa_channel_stats_path."
        )
    with np.load(path, allow_pickle=False) as archive:
        stems = list(archive.files)
        return {stem: torch.tensor(archive[stem], dtype=torch.float32) for stem in stems}


def _split_ids(fp16_ids: torch.Tensor, n_tr: int, n_tc: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """(16-bit tile ids, the complementary INT8 tile ids), both int32 ascending."""
    keep = np.zeros(n_tr * n_tc, dtype=bool)
    keep[fp16_ids.numpy().astype(np.int64)] = True
    return (fp16_ids.to(torch.int32).contiguous(),
            torch.from_numpy(np.flatnonzero(~keep).astype(np.int32)))


def _targets(model: nn.Module, cfg, apply_cfg: ApplyConfig):
    found = iter_target_linears(model, cfg=cfg, model_type=apply_cfg.model_type)
    if not found:
        raise RuntimeError(f"No target linears found for model_type={apply_cfg.model_type}.")
    return found


def _checked_tile_map(name: str, weight_shape, keep_dir, cfg) -> Tuple[torch.Tensor, torch.Tensor, int, int]:
    """One target's Decision/ tile map, checked against its weight: the grid
    must match the padded weight and every id must name a tile of it."""
    fp16_ids, grid = load_fp16_keep_ids_for_layer(keep_dir=keep_dir, layer_name=name, tile_m=cfg.tile_m,
                                                  tile_n=cfg.tile_n)
    want = _tile_grid(weight_shape, cfg.tile_m, cfg.tile_n)
    if tuple(grid) != want:
        raise RuntimeError(f"FP16 keep-id shape mismatch for {name}: archive={tuple(grid)} expected={want}")
    n_tiles = want[0] * want[1]
    if fp16_ids.numel():
        lo, hi = int(fp16_ids.min()), int(fp16_ids.max())
        if lo < 0 or hi >= n_tiles:
            raise RuntimeError(f"FP16 keep-id out of range for {name}: total_tiles={n_tiles} min={lo} max={hi}")
    return (*_split_ids(fp16_ids, *want), want[0], want[1])


def validate_fp16_ids_coverage_and_shapes(model: nn.Module, keep_dir, apply_cfg: ApplyConfig
                                          ) -> Dict[str, Tuple[torch.Tensor, torch.Tensor, int, int]]:
    """Tile map of every target linear, checked against its weight (the
    reference's contract, api.py:80-118): name -> (fp16 ids, int8 ids, n_tr, n_tc)."""
    cfg = _make_cfg(apply_cfg)
    return {name: _checked_tile_map(name, linear.weight.shape, keep_dir, cfg)
            for _, _, name, linear in _targets(model, cfg, apply_cfg)}


def _resolve_safetensor_shards(local_model_dir) -> List[Path]:
    """Shard files of a safetensors checkpoint: the files an index names (each
    once, sorted), else the single model.safetensors."""
    root = Path(local_model_dir)
    index = root / "model.safetensors.index.json"
    if not index.exists():
        if (root / "model.safetensors").exists():
            return [root / "model.safetensors"]
        raise RuntimeError(f"No safetensors checkpoint found in {root}. "
                           "Expected model.safetensors or model.safetensors.index.json.")
    weight_map = json.loads(index.read_text(encoding="utf-8")).get("weight_map", {})
    if not isinstance(weight_map, dict) or not weight_map:
        raise RuntimeError(f"Invalid or empty weight_map in index: {index}")
    shards = [root / name for name in sorted(set(weight_map.values()))]
    for shard in shards:
        if not shard.exists():
            raise RuntimeError(f"Missing shard file listed in index: {shard}")
    return shards


def _empty_model(config, torch_dtype: torch.dtype, attn_implementation: Optional[str]):
    from accelerate import init_empty_weights
    from transformers import AutoModelForCausalLM

    kwargs = {"attn_implementation": attn_implementation} if attn_implementation else {}
    with init_empty_weights():
        return AutoModelForCausalLM.from_config(config, dtype=torch_dtype, **kwargs)


def _move_host_tensors(model: nn.Module, device: torch.device) -> None:
    """from_config leaves some tensors on the host: buffers the checkpoint does
    not hold (RoPE inv_freq) and plain tensor attributes of modules (the rotary
    module's original_inv_freq).  They go to the device, so no forward copies
    host -> device (graph capture forbids it)."""
    for qualified, buf in list(model.named_buffers()):
        if buf.device.type != "meta" and buf.device != device:
            owner, _, leaf = qualified.rpartition(".")
            model.get_submodule(owner)._buffers[leaf] = buf.to(device)
    for module in model.modules():
        for attr, value in list(vars(module).items()):
            if isinstance(value, torch.Tensor) and value.device.type != "meta" and value.device != device:
                setattr(module, attr, value.to(device))


def _finish(model: nn.Module, device: torch.device) -> int:
    _move_host_tensors(model, device)
    fused = fuse_projection_groups(model)
    if hasattr(model, "tie_weights"):
        model.tie_weights()
    model.eval()
    return fused


class _CheckpointRouter:
    """Takes the tensors of a checkpoint one at a time and puts each where it
    belongs in a meta-device model: a target's weight is packed (on the device)
    into a MixedLinear that replaces the nn.Linear; a target's bias goes onto
    that MixedLinear (held back until its weight has arrived); any other tensor
    is materialised on the device.  Counts and times what it did."""

    def __init__(self, model: nn.Module, targets, tile_maps, importance, cfg, device, dtype) -> None:
        self.model, self.cfg, self.device, self.dtype = model, cfg, device, dtype
        self.slot = {name: (parent, attr) for parent, attr, name, _ in targets}
        self.tile_maps, self.importance = tile_maps, importance
        self.packed: Dict[str, MixedLinear] = {}
        self.early_bias: Dict[str, torch.Tensor] = {}
        self.non_target = 0
        self.pack_s = self.non_target_s = 0.0

    def _cast(self, tensor: torch.Tensor) -> torch.Tensor:
        return tensor.to(dtype=self.dtype) if tensor.is_floating_point() else tensor

    def _attach_bias(self, module: MixedLinear, bias: torch.Tensor) -> None:
        module.bias = nn.Parameter(self._cast(bias).to(self.device).detach().clone(), requires_grad=False)

    def take(self, key: str, tensor: torch.Tensor) -> None:
        owner, _, leaf = key.rpartition(".")
        t0 = time.perf_counter()
        if owner in self.slot and leaf == "weight":
            fp16_ids, int8_ids, n_tr, n_tc = self.tile_maps[owner]
            pack = pack_weight_from_tile_ids(self._cast(tensor), int8_tile_ids=int8_ids, fp16_tile_ids=fp16_ids,
                                             n_tr=n_tr, n_tc=n_tc, iaa_col_importance=self.importance.get(owner),
                                             cfg=self.cfg)
            module = MixedLinear(pack=pack, bias=None, cfg=self.cfg).to(self.device)
            parent, attr = self.slot[owner]
            setattr(parent, attr, module)
            self.packed[owner] = module
            if owner in self.early_bias:
                self._attach_bias(module, self.early_bias.pop(owner))
            self.pack_s += time.perf_counter() - t0
        elif owner in self.slot and leaf == "bias":
            if owner in self.packed:
                self._attach_bias(self.packed[owner], tensor)
            else:
                self.early_bias[owner] = tensor
        else:
            set_module_tensor_to_device(self.model, key, self.device, value=self._cast(tensor))
            self.non_target += 1
            self.non_target_s += time.perf_counter() - t0

    def check_complete(self) -> None:
        if self.early_bias:
            raise RuntimeError("Found target bias tensors without corresponding target weight loads, "
                               f"e.g. {list(self.early_bias)[:3]}")
        for name in self.slot:
            if not isinstance(self.model.get_submodule(name), MixedLinear):
                raise RuntimeError(f"Target module is not MixedLinear after load-time apply: {name}")


def _checkpoint_tensors(local_model_dir) -> Iterator[Tuple[str, torch.Tensor]]:
    """(key, host tensor) for every tensor of every shard, shard by shard."""
    from safetensors import safe_open

    for shard in _resolve_safetensor_shards(local_model_dir):
        with safe_open(str(shard), framework="pt", device="cpu") as reader:
            for key in reader.keys():
                yield key, reader.get_tensor(key)


def load_mixed_precision_model_from_masks(local_model_dir, keep_dir, apply_cfg: ApplyConfig,
                                          torch_dtype: torch.dtype, device, attn_implementation: Optional[str] = None):
    """Load a safetensors checkpoint with every target linear packed as it
    arrives (the reference's load-time apply, api.py:154-310): signature,
    statistics and errors as the reference; the packing runs on the device."""
    from transformers import AutoConfig

    started = time.perf_counter()
    device = torch.device(device)
    cfg = _make_cfg(apply_cfg)
    config_kwargs = {"attn_implementation": attn_implementation} if attn_implementation else {}
    model = _empty_model(AutoConfig.from_pretrained(str(local_model_dir), **config_kwargs), torch_dtype,
                         attn_implementation)
    targets = _targets(model, cfg, apply_cfg)
    tile_maps = validate_fp16_ids_coverage_and_shapes(model=model, keep_dir=keep_dir, apply_cfg=apply_cfg)
    importance: Dict[str, torch.Tensor] = {}
    if str(getattr(apply_cfg, "quant_style", "gi")).lower() == "iaa":
        by_stem = _load_iaa_channel_stats(Path(keep_dir), apply_cfg)
        importance = {name: by_stem[name.replace(".", "_")] for name in tile_maps
                      if name.replace(".", "_") in by_stem}
    router = _CheckpointRouter(model, targets, tile_maps, importance, cfg, device, torch_dtype)
    for key, tensor in _checkpoint_tensors(local_model_dir):
        router.take(key, tensor)
    router.check_complete()
    fused = _finish(model, device)
    return model, {
        "num_targets": len(tile_maps),
        "num_replaced": len(router.packed),
        "num_replaced_during_load": len(router.packed),
        "num_loaded_non_target_tensors": router.non_target,
        "load_total": float(time.perf_counter() - started),
        "quant_pack_total": float(router.pack_s),
        "non_target_load_total": float(router.non_target_s),
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
    targets = _targets(model, cfg, apply_cfg)
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
        n_tr, n_tc = _tile_grid(shape, cfg.tile_m, cfg.tile_n)
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
