"""Host-side logic on the CPU: API checks, bookkeeping, Decision/ archives,
target selection, module plumbing.  No GPU; compute entry points must refuse
CPU tensors (there is no CPU fallback)."""
from __future__ import annotations

from pathlib import Path
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from helpers import make_w, oracle_pack, uniform_fp16_ids
from oracle import masks as om
from oracle import packing as opk
from tilequant_amd import mask_io, pack as tpack, quant_utils, rules
from tilequant_amd.gemm_rows_splitk_64x64 import gemm_mixed_rows_splitk
from tilequant_amd.mixed_linear import MixedLinear, fuse_projection_groups, MixedLinearSlice

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_quant_ops_refuse_cpu_tensors():
    x = torch.randn(4, 128).to(torch.bfloat16)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        quant_utils.quantize_activation_tile_absmax(x)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        quant_utils.activation_tile_absmax_scales(x)
    for fn in (quant_utils.quantize_activation_absmax, quant_utils.quantize_activation_per_tensor_absmax,
               quant_utils.quantize_weight_tile_absmax):
        with pytest.raises(RuntimeError, match="no CPU fallback"):
            fn(x)
    with pytest.raises(ValueError):
        quant_utils.quantize_activation_tile_absmax(x.view(2, 2, 128))
    with pytest.raises(ValueError):
        quant_utils.quantize_activation_tile_absmax(x, tile_n=32)


def _cpu_pack(m=128, k=192, frac=0.3, seed=0):
    W = make_w(m, k, seed=seed)
    n_tr, n_tc = -(-m // 64), -(-k // 64)
    ids16 = uniform_fp16_ids(n_tr, n_tc, frac, seed=seed + 1)
    op = oracle_pack(W, ids16)
    t = lambda a, dt=None: torch.from_numpy(np.ascontiguousarray(a)) if dt is None else torch.from_numpy(np.ascontiguousarray(a)).to(dt)
    return tpack.Pack(
        M_orig=m, K_orig=k, M=op.M, K=op.K, tile_m=64, tile_n=64, n_tr=n_tr, n_tc=n_tc,
        int8_tiles=t(op.int8_tiles), int8_scales=t(op.int8_scales), int8_tile_ids=t(op.int8_tile_ids),
        int8_row_ptr=t(op.int8_row_ptr), int8_row_indices=torch.arange(op.int8_tile_ids.size, dtype=torch.int32),
        fp16_tiles=t(op.fp16_tiles.view(np.int16)).view(torch.bfloat16), fp16_tile_ids=t(op.fp16_tile_ids),
        fp16_row_ptr=t(op.fp16_row_ptr), fp16_row_indices=torch.arange(op.fp16_tile_ids.size, dtype=torch.int32),
        tile_layout="row_major"), op


def test_gemm_refuses_cpu_tensors():
    p, _ = _cpu_pack()
    x = torch.zeros(2, 192, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        gemm_mixed_rows_splitk(x_fp=x, x_int8=torch.zeros(2, 192, dtype=torch.int8), sx=torch.ones(3),
                               int8_tiles=p.int8_tiles, int8_scales=p.int8_scales, int8_tile_ids=p.int8_tile_ids,
                               int8_row_ptr=p.int8_row_ptr, fp16_tiles=p.fp16_tiles, fp16_tile_ids=p.fp16_tile_ids,
                               fp16_row_ptr=p.fp16_row_ptr, M=128, K=192, n_tr=2, n_tc=3, out_dtype=torch.bfloat16)


def test_row_schedule_matches_oracle():
    ids = torch.tensor([1, 4, 5, 9, 10, 11], dtype=torch.int64)
    rp, ri = tpack._build_row_schedule(ids, n_tr=4, n_tc=3)
    assert rp.tolist() == opk.row_ptr_of(ids.numpy(), 4, 3).tolist() == [0, 1, 3, 3, 6]
    assert ri.tolist() == list(range(6))
    rp0, ri0 = tpack._build_row_schedule(torch.empty(0, dtype=torch.int64), n_tr=2, n_tc=3)
    assert rp0.tolist() == [0, 0, 0] and ri0.numel() == 0


def test_concat_packs_matches_oracle_and_checks():
    (a, oa), (b, ob) = _cpu_pack(128, 192, 0.3, 1), _cpu_pack(64, 192, 0.5, 2)
    cat = tpack.concat_packs_along_rows([a, b])
    ocat = opk.concat_rows([oa, ob])
    assert cat.n_tr == 3 and cat.M == 192
    for f in ("int8_tile_ids", "int8_row_ptr", "fp16_tile_ids", "fp16_row_ptr", "int8_scales"):
        assert np.array_equal(getattr(cat, f).numpy(), getattr(ocat, f)), f
    c, _ = _cpu_pack(128, 256, 0.3, 3)
    with pytest.raises(ValueError, match="input geometry"):
        tpack.concat_packs_along_rows([a, c])
    d, _ = _cpu_pack(128, 192, 0.3, 4)
    d.tile_layout = "mfma"
    with pytest.raises(ValueError, match="tile layout"):
        tpack.concat_packs_along_rows([a, d])
    with pytest.raises(ValueError):
        tpack.concat_packs_along_rows([])


def test_pack_validation_errors_before_device_work():
    W = make_w(128, 192)
    cfg = {"quant_style": "gi"}
    ids = torch.arange(6, dtype=torch.int32)
    with pytest.raises(ValueError, match="dimensions mismatch"):
        tpack.pack_weight_from_tile_ids(W, n_tr=3, n_tc=3, int8_tile_ids=ids, fp16_tile_ids=ids[:0], cfg=cfg)
    with pytest.raises(ValueError, match="quant_style"):
        tpack.pack_weight_from_tile_ids(W, n_tr=2, n_tc=3, int8_tile_ids=ids, fp16_tile_ids=ids[:0],
                                        cfg={"quant_style": "awq"})
    with pytest.raises(ValueError, match="pad_to_tile=False"):
        tpack.pack_weight_from_tile_ids(make_w(100, 192), n_tr=2, n_tc=3, int8_tile_ids=ids, fp16_tile_ids=ids[:0],
                                        cfg={"pad_to_tile": False})
    with pytest.raises(ValueError):
        tpack.pack_weight_from_tile_ids(W.float(), n_tr=2, n_tc=3, int8_tile_ids=ids, fp16_tile_ids=ids[:0], cfg=cfg)


def test_mask_io_roundtrip_and_errors(tmp_path):
    masks = {"model_layers_0_self_attn_q_proj": np.eye(4, 6, dtype=np.uint8),
             "model_layers_10_mlp_up_proj": np.zeros((2, 3), np.uint8)}
    path = mask_io.save_mask_keep_archive(tmp_path, masks)
    assert path.name == "fp16_keep_ids_tile64x64.npz"
    ids, shape = mask_io.load_fp16_keep_ids_for_layer(tmp_path, "model.layers.0.self_attn.q_proj")
    assert shape == (4, 6) and ids.tolist() == [0, 7, 14, 21] and ids.dtype == torch.int32
    assert torch.equal(mask_io.load_mask_keep_for_layer(tmp_path, "model.layers.0.self_attn.q_proj"),
                       torch.from_numpy(masks["model_layers_0_self_attn_q_proj"]))
    assert set(mask_io.load_mask_keep_stem_dict(tmp_path)) == set(masks)
    # the oracle's independent reader sees the same content
    arch = om.read_archive(path)
    assert arch["model_layers_0_self_attn_q_proj"][1].tolist() == [0, 7, 14, 21]
    with pytest.raises(FileNotFoundError):
        mask_io.load_fp16_keep_ids_for_layer(tmp_path, "model.layers.3.mlp.up_proj")
    with pytest.raises(FileNotFoundError):
        mask_io.load_fp16_keep_ids_for_layer(tmp_path / "nope", "x")
    with pytest.raises(ValueError):
        mask_io.save_mask_keep_archive(tmp_path, {"a": np.full((2, 2), 2)})
    bad = tmp_path / "bad"
    bad.mkdir()
    np.savez_compressed(bad / "fp16_keep_ids_tile64x64.npz", stems=np.asarray(["s"]),
                        shape_0=np.asarray([2, 2], np.int32), ids_0=np.asarray([4], np.uint16))
    with pytest.raises(RuntimeError, match="Out-of-bound"):
        mask_io.load_fp16_keep_ids_for_layer(bad, "s")


def test_mask_io_reads_released_archive_like_oracle():
    keep = GOLDEN / "llama32_3b_gi_keep01"
    arch = mask_io.open_archive(keep)
    oarch = om.read_archive(keep / "fp16_keep_ids_tile64x64.npz")
    assert set(arch) == set(oarch) and len(arch) == 196
    for stem in list(arch)[:20]:
        assert arch[stem].grid == oarch[stem][0] and np.array_equal(arch[stem].ids, oarch[stem][1])
        assert arch[stem].ids.dtype == np.uint16
    assert mask_io.open_archive(keep) is arch   # parsed once per process


def test_mask_io_rereads_a_rewritten_archive_and_uint32_ids(tmp_path):
    """A second save replaces the parsed archive; grids above 65535 tiles
    store uint32 ids (the released format's rule); stems are sorted."""
    small = {"b_proj": np.eye(3, dtype=np.uint8), "a_proj": np.zeros((1, 2), np.uint8)}
    mask_io.save_mask_keep_archive(tmp_path, small)
    first = mask_io.open_archive(tmp_path)
    assert list(first) == ["a_proj", "b_proj"] and first["b_proj"].ids.tolist() == [0, 4, 8]
    big = np.zeros((256, 300), np.uint8)
    big[255, 299] = 1
    path = mask_io.save_mask_keep_archive(tmp_path, {"c_proj": big})
    second = mask_io.open_archive(tmp_path)
    assert second is not first and list(second) == ["c_proj"]
    assert second["c_proj"].ids.dtype == np.uint32 and second["c_proj"].ids.tolist() == [256 * 300 - 1]
    with np.load(path, allow_pickle=False) as npz:
        assert npz["shape_0"].dtype == np.int32 and npz["ids_0"].dtype == np.uint32
    with pytest.raises(ValueError, match="2D"):
        mask_io.save_mask_keep_archive(tmp_path, {"d": np.zeros(3)})
    with pytest.raises(ValueError, match="empty"):
        mask_io.save_mask_keep_archive(tmp_path, {})
    bad = tmp_path / "bad"
    bad.mkdir()
    np.savez(bad / "fp16_keep_ids_tile64x64.npz", stems=np.asarray(["s"]), shape_0=np.asarray([2, 2, 1], np.int32),
             ids_0=np.asarray([1], np.uint16))
    with pytest.raises(RuntimeError, match="Invalid shape metadata"):
        mask_io.load_mask_keep_stem_dict(bad)


def test_iter_target_linears_on_llama_architecture():
    from transformers import LlamaConfig, LlamaForCausalLM

    cfg = LlamaConfig(hidden_size=128, intermediate_size=256, num_hidden_layers=2, num_attention_heads=4,
                      num_key_value_heads=2, vocab_size=64)
    model = LlamaForCausalLM(cfg)
    found = rules.iter_target_linears(model, cfg={}, model_type="llama")
    assert len(found) == 14
    names = {f for _, _, f, _ in found}
    assert "model.layers.1.mlp.down_proj" in names and "lm_head" not in names
    only_attn = rules.iter_target_linears(model, cfg={"module_filters": ["*self_attn*"]}, model_type="llama")
    assert len(only_attn) == 8


def test_mixed_linear_module_plumbing_on_cpu():
    p, _ = _cpu_pack()
    cfg = SimpleNamespace(dtype_out="bf16")
    m = MixedLinear(p, torch.zeros(128, dtype=torch.bfloat16), cfg)
    sd = m.state_dict()
    assert {"int8_tiles", "int8_scales", "int8_tile_ids", "int8_row_ptr", "int8_row_indices", "fp16_tiles",
            "fp16_tile_ids", "fp16_row_ptr", "fp16_row_indices", "bias"} <= set(sd)
    assert sd["_extra_state"] == {"tile_layout": "row_major"}
    m2 = MixedLinear(p, None, cfg)
    m2.tile_layout = "mfma"
    m2.load_state_dict({k: v for k, v in sd.items() if k != "bias"}, strict=False)
    assert m2.tile_layout == "row_major"
    with pytest.raises(ValueError, match="K mismatch"):
        m(torch.zeros(2, 100, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="rank"):
        m(torch.zeros(192, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        m(torch.zeros(2, 3, 192, dtype=torch.bfloat16))
    assert m.to_pack().tile_layout == "row_major"


def test_fuse_projection_groups_structure_on_cpu():
    class Attn(torch.nn.Module):
        pass

    cfg = SimpleNamespace(dtype_out="bf16")
    parent = Attn()
    for i, name in enumerate(("q_proj", "k_proj", "v_proj")):
        p, _ = _cpu_pack(128 if name == "q_proj" else 64, 192, 0.3, 10 + i)
        setattr(parent, name, MixedLinear(p, None, cfg))
    assert fuse_projection_groups(parent) == 1
    assert isinstance(parent.q_proj, MixedLinearSlice)
    assert parent.tilequant_qkv.bounds == ((0, 128), (128, 192), (192, 256))
    assert parent.tilequant_qkv.linear.n_tr == 4


def test_serve_once_hands_each_consumer_one_copy_and_releases():
    """The memo behind the sibling-quantization cache and projection groups:
    a hit needs the same live tensor, the same view/version and a consumer
    that has not taken the value; a full set of consumers, a miss or the
    source's death release it."""
    import gc

    from tilequant_amd.mixed_linear import ServeOnce, _view_key

    memo = ServeOnce(consumers=3)
    x = torch.zeros(4, 8)
    key = _view_key(x)
    assert memo.take(x, key, 0) is None
    memo.put(x, key, 0, "y")
    assert memo.take(x, key, 0) is None              # consumer 0 again: a new pass
    memo.put(x, key, 0, "y2")
    assert memo.take(x, key, 1) == "y2" and memo.take(x, key, 2) == "y2"
    assert memo.take(x, key, 1) is None              # all three served: released
    memo.put(x, key, 0, "y3")
    x.add_(1)                                        # in-place update bumps the version: stale
    assert memo.take(x, _view_key(x), 1) is None
    memo.put(x, _view_key(x), 0, "y4")
    assert memo.take(x[:2], _view_key(x[:2]), 1) is None   # another tensor (a view) is a miss
    memo.put(x, _view_key(x), 0, "y5")
    del x
    gc.collect()
    assert memo._value is None                       # the source died: the value went with it
    unbounded = ServeOnce()
    a = torch.ones(3)
    unbounded.put(a, _view_key(a), "q", 1)
    assert [unbounded.take(a, _view_key(a), c) for c in ("k", "v", "k")] == [1, 1, None]


def test_state_dict_without_layout_record_loads_as_row_major():
    """A state_dict written by the reference has row-major tiles and no
    _extra_state: loading it into a module packed in the MFMA order must
    switch the module to row-major (strict and non-strict)."""
    cfg = SimpleNamespace(dtype_out="bf16")
    p, _ = _cpu_pack(128, 192, 0.3, 40)
    ref_sd = {k: v for k, v in MixedLinear(p, None, cfg).state_dict().items() if not k.endswith("_extra_state")}
    for strict in (True, False):
        p2, _ = _cpu_pack(128, 192, 0.3, 40)
        p2.tile_layout = "mfma"
        m = MixedLinear(p2, None, cfg)
        assert m.tile_layout == "mfma"
        res = m.load_state_dict(ref_sd, strict=strict)
        assert m.tile_layout == "row_major" and not res.missing_keys and not res.unexpected_keys
    # this build's own state_dicts keep their record
    p3, _ = _cpu_pack(128, 192, 0.3, 40)
    p3.tile_layout = "mfma"
    sd = MixedLinear(p3, None, cfg).state_dict()
    m = MixedLinear(_cpu_pack(128, 192, 0.3, 40)[0], None, cfg)
    m.load_state_dict(sd)
    assert m.tile_layout == "mfma"


def test_partial_state_dict_leaves_the_tile_layout_alone():
    """A strict=False load of a dict that does not replace this module's tiles
    (an unrelated parent-model subset, a bias-only dict) must not switch an
    MFMA-order module to row-major: its tiles stay in the MFMA order."""
    cfg = SimpleNamespace(dtype_out="bf16")
    p, _ = _cpu_pack(128, 192, 0.3, 41)
    p.tile_layout = "mfma"
    parent = torch.nn.Sequential(torch.nn.Linear(4, 4), MixedLinear(p, torch.zeros(128, dtype=torch.bfloat16), cfg))
    tiles = parent[1].int8_tiles.clone()
    for partial in ({"0.weight": torch.ones(4, 4)}, {"1.bias": torch.ones(128, dtype=torch.bfloat16)}, {}):
        parent.load_state_dict(partial, strict=False)
        assert parent[1].tile_layout == "mfma", partial
        assert torch.equal(parent[1].int8_tiles, tiles)
    assert torch.equal(parent[1].bias, torch.ones(128, dtype=torch.bfloat16))


def test_fused_decode_refuses_architectures_it_does_not_compute():
    """Qwen3 (per-head q/k RMSNorm), dynamic RoPE and partial rotary are
    rejected; Llama-3.2 (llama3 RoPE) and Qwen2 are accepted."""
    from accelerate import init_empty_weights
    from transformers import AutoModelForCausalLM, LlamaConfig, Qwen2Config, Qwen3Config

    from tilequant_amd.fused_decode import check_fused_architecture

    def attn_of(cfg):
        with init_empty_weights():
            return AutoModelForCausalLM.from_config(cfg).model.layers[0].self_attn

    small = dict(hidden_size=256, intermediate_size=512, num_hidden_layers=1, num_attention_heads=2,
                 num_key_value_heads=1, vocab_size=64, head_dim=128)
    q3 = Qwen3Config(**small)
    with pytest.raises(ValueError, match="model_type"):
        check_fused_architecture(q3, attn_of(q3))
    q3.model_type = "qwen2"   # even under a permitted name, the per-head norms are refused
    with pytest.raises(ValueError, match="q_norm"):
        check_fused_architecture(q3, attn_of(Qwen3Config(**small)))
    dyn = LlamaConfig(**small, rope_scaling={"rope_type": "dynamic", "factor": 2.0})
    with pytest.raises(ValueError, match="rope_type"):
        check_fused_architecture(dyn, attn_of(dyn))
    llama32 = LlamaConfig(**small, max_position_embeddings=131072,
                          rope_scaling={"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0,
                                        "high_freq_factor": 4.0, "original_max_position_embeddings": 8192})
    check_fused_architecture(llama32, attn_of(llama32))
    q2 = Qwen2Config(**small)
    check_fused_architecture(q2, attn_of(q2))
    part = LlamaConfig(**small)
    part.partial_rotary_factor = 0.5
    with pytest.raises(ValueError, match="partial"):
        check_fused_architecture(part, attn_of(LlamaConfig(**small)))


def _plan_from_ids16(ids16, n_tr, n_tc):
    from tilequant_amd.gemm_rows_splitk_64x64 import prefill_plan

    mask = np.zeros(n_tr * n_tc, bool)
    mask[ids16] = True
    ids8 = np.flatnonzero(~mask)
    rp8 = np.r_[0, np.cumsum(np.bincount(ids8 // n_tc, minlength=n_tr))]
    rp16 = np.r_[0, np.cumsum(np.bincount(np.asarray(ids16, np.int64) // n_tc, minlength=n_tr))]
    return prefill_plan(int8_tile_ids=torch.tensor(ids8, dtype=torch.int32),
                        int8_row_ptr=torch.tensor(rp8, dtype=torch.int32),
                        fp16_row_ptr=torch.tensor(rp16, dtype=torch.int32), n_tr=n_tr, n_tc=n_tc, device="cpu")


def _covered_rows(units, n_tr):
    rows = []
    for u in units:
        r = u & ((1 << 30) - 1)
        rows += [r] if u >> 30 or r + 1 >= n_tr else [r, r + 1]
    return sorted(rows)


def test_prefill_plan_splits_the_released_heavy_row():
    """Released keep05 map, layer 7 down_proj: row tile 47 holds 127 of its
    128 tiles in 16 bits.  The plan (host code in the library) splits its pair
    into single row tiles and leaves the balanced pairs alone, in row order;
    every row tile is covered exactly once; uniform maps need no plan."""
    ids, (n_tr, n_tc) = mask_io.load_fp16_keep_ids_for_layer(GOLDEN / "llama32_3b_gi_keep05",
                                                              "model.layers.7.mlp.down_proj")
    plan = _plan_from_ids16(ids.numpy(), n_tr, n_tc)
    units = plan.units.tolist()
    i = units.index(46 | 1 << 30)
    assert units[i + 1] == 47 | 1 << 30 and plan.n_first == 0
    rows = [u & ((1 << 30) - 1) for u in units]
    assert rows == sorted(rows)
    counts = np.bincount(ids.numpy() // n_tc, minlength=n_tr)
    split = [u & ((1 << 30) - 1) for u in units if u >> 30]
    assert all(max(counts[r], counts[r ^ 1]) >= 20 for r in split)   # only 16-bit-heavy pairs split
    assert _covered_rows(units, n_tr) == list(range(n_tr))
    assert _plan_from_ids16(uniform_fp16_ids(48, 128, 0.05, seed=3), 48, 128) is None


def test_prefill_plan_rejects_inconsistent_bookkeeping():
    from tilequant_amd.gemm_rows_splitk_64x64 import prefill_plan

    rp8 = torch.tensor([0, 2, 4], dtype=torch.int32)
    ids8 = torch.tensor([0, 1, 2, 7], dtype=torch.int32)   # id 7 is not in row 1 (columns 2..3 of 2 x 2)
    with pytest.raises(ValueError, match="tq_gemm_prefill_plan"):
        prefill_plan(int8_tile_ids=ids8, int8_row_ptr=rp8, fp16_row_ptr=torch.zeros(0, dtype=torch.int32),
                     n_tr=2, n_tc=2, device="cpu")
