"""Load-time driver host logic on the CPU (mirror of src/quantization/api.py):
tile-map validation against weight shapes, shard resolution, model-type
inference, error paths.  The packing itself runs on the GPU (test_gpu_e2e)."""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from e2e_models import target_shapes, tiny_llama_config, tiny_qwen2_config, write_tile_maps
from tilequant_amd import api, mask_io
from tilequant_amd.types import ApplyConfig, TileConfig


def _empty(config):
    return api._empty_model(config, torch.bfloat16, "sdpa")


def test_target_selection_and_tile_grids(tmp_path):
    cfg = tiny_llama_config()
    shapes = target_shapes(cfg)
    assert len(shapes) == 2 * 7
    assert shapes["model.layers.0.self_attn.q_proj"] == (512, 512)
    assert shapes["model.layers.1.self_attn.k_proj"] == (256, 512)
    assert shapes["model.layers.0.mlp.down_proj"] == (512, 1024)
    masks = write_tile_maps(cfg, tmp_path / "keep10", frac=0.1, seed=3)
    apply_cfg = ApplyConfig(model_type="llama", dtype_out="bf16", tile=TileConfig())
    data = api.validate_fp16_ids_coverage_and_shapes(_empty(cfg), tmp_path / "keep10", apply_cfg)
    assert set(data) == set(shapes)
    for name, (f16, i8, n_tr, n_tc) in data.items():
        mask = masks[mask_io.layer_name_to_stem(name)].reshape(-1)
        assert (n_tr, n_tc) == (-(-shapes[name][0] // 64), -(-shapes[name][1] // 64))
        assert f16.dtype == torch.int32 and i8.dtype == torch.int32
        assert np.array_equal(f16.numpy(), np.flatnonzero(mask == 1))
        assert np.array_equal(i8.numpy(), np.flatnonzero(mask == 0))   # INT8 ids = complement, ascending


def test_tile_grid_mismatch_and_missing_maps_raise(tmp_path):
    cfg = tiny_llama_config()
    apply_cfg = ApplyConfig(model_type="llama", dtype_out="bf16")
    # archive written for a wider model: grid mismatch
    wide = tiny_llama_config()
    wide.intermediate_size = 2048
    write_tile_maps(wide, tmp_path / "k", frac=0.1)
    with pytest.raises(RuntimeError, match="shape mismatch"):
        api.validate_fp16_ids_coverage_and_shapes(_empty(cfg), tmp_path / "k", apply_cfg)
    # a target without a stem in the archive
    write_tile_maps(tiny_llama_config(layers=1), tmp_path / "k1", frac=0.1)
    with pytest.raises(FileNotFoundError):
        api.validate_fp16_ids_coverage_and_shapes(_empty(cfg), tmp_path / "k1", apply_cfg)
    with pytest.raises(FileNotFoundError):
        api.validate_fp16_ids_coverage_and_shapes(_empty(cfg), tmp_path / "absent", apply_cfg)
    # no targets at all
    empty_filter = ApplyConfig(model_type="llama", dtype_out="bf16", module_filters=["nothing.*"])
    with pytest.raises(RuntimeError, match="No target linears"):
        api.validate_fp16_ids_coverage_and_shapes(_empty(cfg), tmp_path / "k1", empty_filter)


def test_module_filters_narrow_targets(tmp_path):
    cfg = tiny_llama_config()
    write_tile_maps(cfg, tmp_path / "k", frac=0.1)
    apply_cfg = ApplyConfig(model_type="llama", dtype_out="bf16", module_filters=["*.mlp.*"])
    data = api.validate_fp16_ids_coverage_and_shapes(_empty(cfg), tmp_path / "k", apply_cfg)
    assert set(data) == {n for n in target_shapes(cfg) if ".mlp." in n}


def test_shard_resolution(tmp_path):
    with pytest.raises(RuntimeError, match="No safetensors checkpoint"):
        list(api._resolve_safetensor_shards(tmp_path))
    (tmp_path / "model.safetensors").write_bytes(b"")
    assert list(api._resolve_safetensor_shards(tmp_path)) == [tmp_path / "model.safetensors"]
    idx = {"weight_map": {"a": "model-00002-of-00002.safetensors", "b": "model-00001-of-00002.safetensors"}}
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps(idx))
    with pytest.raises(RuntimeError, match="Missing shard"):
        list(api._resolve_safetensor_shards(tmp_path))
    for f in idx["weight_map"].values():
        (tmp_path / f).write_bytes(b"")
    assert [p.name for p in api._resolve_safetensor_shards(tmp_path)] == [
        "model-00001-of-00002.safetensors", "model-00002-of-00002.safetensors"]
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": {}}))
    with pytest.raises(RuntimeError, match="empty weight_map"):
        list(api._resolve_safetensor_shards(tmp_path))


def test_model_type_and_cfg(tmp_path):
    tiny_qwen2_config().save_pretrained(tmp_path)
    assert api.infer_model_type(tmp_path) == "qwen"
    assert api.infer_model_type(tiny_llama_config()) == "llama"
    c = api._make_cfg(ApplyConfig(model_type="qwen", dtype_out="bf16", quant_style="iaa", module_filters=["x"]))
    assert (c.tile_m, c.tile_n, c.dtype_out, c.quant_style, c.pad_to_tile, c.module_filters) == (
        64, 64, "bf16", "iaa", True, ["x"])


def test_iaa_stats_missing_raises(tmp_path):
    apply_cfg = ApplyConfig(model_type="llama", quant_style="iaa", iaa_channel_stats_path=str(tmp_path / "none.npz"))
    with pytest.raises(FileNotFoundError, match="IAA channel stats"):
        api._load_iaa_channel_stats(tmp_path, apply_cfg)


def test_uniform_tile_map_rule():
    rng = np.random.default_rng(0)
    ids = api.uniform_fp16_tile_ids(48, 48, 0.01, rng)
    assert ids.numel() == 24 and bool((ids[1:] > ids[:-1]).all())     # ceil(0.01 * 2304) = 24, sorted, unique
    assert api.uniform_fp16_tile_ids(48, 48, 0.0, rng).numel() == 0
    assert api.uniform_fp16_tile_ids(2, 2, 0.01, rng).numel() == 1    # k = max(1, ...)


def test_decoder_refuses_host_models():
    from tilequant_amd.graph_decode import CudaGraphGreedyDecoder
    from transformers import AutoModelForCausalLM

    model = AutoModelForCausalLM.from_config(tiny_llama_config(layers=1)).eval()
    with pytest.raises(ValueError, match="single-device"):
        CudaGraphGreedyDecoder(model, prompt_tokens=8, max_new_tokens=4, device="cuda:0")
    with pytest.raises(ValueError, match="cuda"):
        CudaGraphGreedyDecoder(model, prompt_tokens=8, max_new_tokens=4, device="cpu")
    with pytest.raises(ValueError):
        CudaGraphGreedyDecoder(model, prompt_tokens=8, max_new_tokens=0, device="cuda:0")
