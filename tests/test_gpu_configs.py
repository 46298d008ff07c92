"""GPU parity at the benchmark workloads' real shapes.

* whole Llama-3.2-3B projections at 8192 tokens (keep05), through
  MixedLinear with the reference's 4096-row chunks (two chunks, whole-input
  scales) and with one chunk -- bitwise equal -- and against the oracle on
  sampled rows.
  The stacked Q/K/V (5120 x 3072) and Gate/Up (16384 x 3072) groups at 8192
  tokens, with the automatic schedule and with an explicit work plan.
* every projection of Qwen2.5-7B (stacked Q/K/V 4608 x 3584, O,
  stacked Gate/Up 37888 x 3584, Down) and Qwen2.5-14B (stacked Q/K/V
  7168 x 5120, O, stacked Gate/Up 27648 x 5120, Down 5120 x 13824) at its
  real output width, clustered keep10 / keep20 masks, 4 and 8192 tokens,
  against the oracle on sampled rows (the oracle's cost does not grow with the
  token count).
* the 28-layer Llama-3.2-3B with a vocabulary of 128256 at batch 4,
  a 2048-token prompt and 256 new tokens: the fused HIP-graph decode step
  against the model's own modules replayed in the same decoder and against the
  eager Hugging Face forward (teacher-forced on the fused run's tokens), over
  every one of the 255 decode steps; seeded uniform keep01 and the released
  Llama-3.2-3B gi keep01 map.

Bars: packed tiles and scales bit-exact; GEMM outputs within 2 bf16 ulp + the
fp32 accumulation bound of the float64 oracle (helpers.assert_gemm_close);
generated ids exactly the argmax of their step's logits; logits against the
two reference-style paths within the noise floor those two paths show against
each other at 28 layers, and within 3e-2 / 5e-2 of the largest logit (argmax
equal where the margin is clear) for one layer at the same widths.
"""
from __future__ import annotations

from pathlib import Path
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from helpers import assert_gemm_close, bits, clustered_weight, complement, make_w, make_x, oracle_pack, \
    uniform_fp16_ids, values
from oracle import native as onat
from oracle import numerics as nm
from oracle import packing as opk
from tilequant_amd.gemm_rows_splitk_64x64 import PrefillPlan, gemm_mixed_rows_splitk
from tilequant_amd.mixed_linear import MixedLinear
from tilequant_amd.pack import concat_packs_along_rows, pack_weight_from_tile_ids
from tilequant_amd.quant_utils import quantize_activation_tile_absmax

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
GOLDEN = Path(__file__).resolve().parent / "golden"
CFG = SimpleNamespace(quant_style="gi", dtype_out="bf16")


def _pack(W, ids16):
    n_tr, n_tc = -(-W.shape[0] // 64), -(-W.shape[1] // 64)
    ids8 = complement(ids16, n_tr * n_tc)
    return pack_weight_from_tile_ids(W.to(DEV), n_tr=n_tr, n_tc=n_tc, int8_tile_ids=torch.from_numpy(ids8),
                                     fp16_tile_ids=torch.from_numpy(np.asarray(ids16, np.int64)), cfg=CFG,
                                     tile_layout="mfma")


def _check_pack(pack, op):
    assert np.array_equal(pack.int8_scales.cpu().numpy().view(np.uint32), op.int8_scales.view(np.uint32))
    assert np.array_equal(opk.from_mfma_int8(pack.int8_tiles.cpu().numpy()), op.int8_tiles)
    assert np.array_equal(opk.from_mfma_16bit(bits(pack.fp16_tiles.cpu())), op.fp16_tiles)
    for f in ("int8_tile_ids", "int8_row_ptr", "fp16_tile_ids", "fp16_row_ptr"):
        assert np.array_equal(getattr(pack, f).cpu().numpy(), getattr(op, f)), f


def _sample_rows(n):
    return np.unique(np.r_[0:3, n // 2:n // 2 + 3, max(0, n - 300):max(0, n - 297), n - 3:n].clip(0, n - 1))


def _oracle_rows(op, x_cpu, rows, sx_ref):
    """float64 oracle outputs (and the sum of |terms|) of the sampled rows,
    with the activation scales of the WHOLE input."""
    xs = values(x_cpu[rows])
    xq_rows = nm.act_quant_codes(xs, sx_ref)
    w16 = nm.bf16_bits_to_f32(op.fp16_tiles)
    _, acc, sab = onat.gemm_mixed(xq_rows, sx_ref, xs, op.int8_tiles, op.int8_scales, op.int8_tile_ids,
                                  op.int8_row_ptr, w16, op.fp16_tile_ids, op.fp16_row_ptr, op.n_tr, op.n_tc,
                                  op.M_orig, op.K_orig, want_f64=True)
    return xq_rows, acc, sab


def _gemm(pack, xd, xq, sx, plan=None):
    return gemm_mixed_rows_splitk(
        x_fp=xd, x_int8=xq, sx=sx, int8_tiles=pack.int8_tiles, int8_scales=pack.int8_scales,
        int8_tile_ids=pack.int8_tile_ids, int8_row_ptr=pack.int8_row_ptr, fp16_tiles=pack.fp16_tiles,
        fp16_tile_ids=pack.fp16_tile_ids, fp16_row_ptr=pack.fp16_row_ptr, M=pack.M_orig, K=pack.K_orig,
        n_tr=pack.n_tr, n_tc=pack.n_tc, out_dtype=torch.bfloat16, tile_layout=pack.tile_layout,
        prefill_plan=plan)


def _stack(members, frac, seed, clustered):
    """Device and oracle packs of members stacked along the output rows (as
    MixedLinearGroup stacks Q/K/V and Gate/Up), packs checked bit-exact; and
    the most 16-bit tiles any row tile of a member carries."""
    packs, ops, max16 = [], [], 0
    for i, (m, kk) in enumerate(members):
        if clustered:
            W, ids16 = clustered_weight(m, kk, frac, seed=seed + i)
        else:
            W = make_w(m, kk, seed=seed + i)
            ids16 = uniform_fp16_ids(m // 64, kk // 64, frac, seed=seed + 50 + i)
        packs.append(_pack(W, ids16))
        ops.append(oracle_pack(W, ids16))
        _check_pack(packs[-1], ops[-1])
        rp = ops[-1].fp16_row_ptr
        max16 = max(max16, int((rp[1:] - rp[:-1]).max()))
        del W
    pack = packs[0] if len(packs) == 1 else concat_packs_along_rows(packs)
    op = ops[0] if len(ops) == 1 else opk.concat_rows(ops)
    return pack, op, max16


# ---- whole Llama-3.2-3B projections at 8192 tokens ------------------------------------

@pytest.mark.parametrize("m,k", [(3072, 3072), (3072, 8192)])
def test_llama_prefill_projection_8192_tokens_two_chunks(m, k):
    """q/o (3072 -> 3072) and down (8192 -> 3072) at 8192 tokens, keep05:
    the reference's two 4096-row chunks with whole-input scales equal one
    chunk bit for bit, and both meet the oracle on sampled rows of both
    chunks."""
    n = 8192
    W = make_w(m, k, seed=m + k)
    n_tr, n_tc = m // 64, k // 64
    ids16 = uniform_fp16_ids(n_tr, n_tc, 0.05, seed=k)
    pack = _pack(W, ids16)
    op = oracle_pack(W, ids16)
    _check_pack(pack, op)
    x = make_x(n, k, seed=k + 1)
    xd = x.to(DEV)
    two = MixedLinear(pack, None, dict(dtype_out="bf16", activation_row_chunk_size=4096))
    one = MixedLinear(pack, None, dict(dtype_out="bf16", activation_row_chunk_size=16384))
    y2 = two(xd.view(4, 2048, k))
    y1 = one(xd)
    assert torch.equal(y2.reshape(n, m), y1)
    sx_ref = onat.act_scales(values(x))
    _, sx_gpu = quantize_activation_tile_absmax(xd)
    assert np.array_equal(sx_gpu.cpu().numpy().view(np.uint32), sx_ref.view(np.uint32))
    rows = _sample_rows(n)
    _, acc, sab = _oracle_rows(op, x, rows, sx_ref)
    assert_gemm_close(y1[torch.from_numpy(rows).to(DEV)], acc, sab, n_tc)


@pytest.mark.parametrize("group", ["qkv", "gate_up"])
def test_llama_prefill_stacked_groups_8192_tokens(group):
    """The stacked Q/K/V (5120 x 3072) and Gate/Up (16384 x 3072) groups at
    8192 tokens, keep05 uniform, against the oracle on sampled rows: with the
    automatic schedule and with an explicit work plan of single row tiles
    (every row tile its own unit), which must give bitwise the same output."""
    members = {"qkv": [(3072, 3072), (1024, 3072), (1024, 3072)], "gate_up": [(8192, 3072), (8192, 3072)]}[group]
    pack, op, _ = _stack(members, 0.05, seed=31 + len(members), clustered=False)
    n, k = 8192, 3072
    x = make_x(n, k, seed=33)
    xd = x.to(DEV)
    xq, sx = quantize_activation_tile_absmax(xd)
    sx_ref = onat.act_scales(values(x))
    assert np.array_equal(sx.cpu().numpy().view(np.uint32), sx_ref.view(np.uint32))
    y = _gemm(pack, xd, xq, sx)
    units = torch.tensor([r | (1 << 30) for r in range(pack.n_tr)], dtype=torch.int32, device=DEV)
    y_plan = _gemm(pack, xd, xq, sx, plan=PrefillPlan(units, 0, pack.n_tr))
    assert torch.equal(y_plan, y)
    rows = _sample_rows(n)
    _, acc, sab = _oracle_rows(op, x, rows, sx_ref)
    assert_gemm_close(y[torch.from_numpy(rows).to(DEV)], acc, sab, op.n_tc)


# ---- Qwen2.5 widths with clustered masks -------------------------------------------

QWEN_SHAPES = {
    "qwen7b_qkv": [(3584, 3584), (512, 3584), (512, 3584)],        # stacked q/k/v: 4608 x 3584
    "qwen7b_o": [(3584, 3584)],
    "qwen7b_gate_up": [(18944, 3584), (18944, 3584)],              # stacked gate/up: 37888 x 3584
    "qwen7b_down": [(3584, 18944)],
    "qwen14b_qkv": [(5120, 5120), (1024, 5120), (1024, 5120)],     # stacked q/k/v: 7168 x 5120
    "qwen14b_o": [(5120, 5120)],
    "qwen14b_gate_up": [(13824, 5120), (13824, 5120)],             # stacked gate/up: 27648 x 5120
    "qwen14b_down": [(5120, 13824)],
}


@pytest.mark.parametrize("frac", [0.10, 0.20])
@pytest.mark.parametrize("proj", sorted(QWEN_SHAPES))
def test_qwen_real_widths_clustered_masks(proj, frac):
    """Every Qwen2.5-7B / 14B projection group at its real width with top-k
    clustered BF16 tiles: packs bit-exact; 4-token decode and 8192-token
    prefill outputs vs the oracle."""
    members = QWEN_SHAPES[proj]
    k = members[0][1]
    pack, op, max16 = _stack(members, frac, seed=sum(m for m, _ in members) + k + int(frac * 100), clustered=True)
    assert max16 >= 4 * frac * op.n_tc   # clustered: some row tiles carry several times the mean share
    for n in (4, 8192):
        x = make_x(n, k, seed=k + n)
        xd = x.to(DEV)
        xq, sx = quantize_activation_tile_absmax(xd)
        sx_ref = onat.act_scales(values(x))
        assert np.array_equal(sx.cpu().numpy().view(np.uint32), sx_ref.view(np.uint32))
        y = _gemm(pack, xd, xq, sx)
        rows = _sample_rows(n)
        xq_rows, acc, sab = _oracle_rows(op, x, rows, sx_ref)
        assert np.array_equal(xq[torch.from_numpy(rows).to(DEV)].cpu().numpy(), xq_rows)
        assert_gemm_close(y[torch.from_numpy(rows).to(DEV)], acc, sab, op.n_tc)
        del x, xd, xq, y


# ---- 28-layer Llama-3.2-3B end to end ----------------------------------------------

def _eager_teacher_forced(model, prompt, tokens):
    """Last-position logits of the eager forward over the prompt, then one
    token at a time fed the given tokens (DynamicCache, fused SDPA)."""
    from torch.nn.attention import SDPBackend, sdpa_kernel

    outs = []
    with torch.inference_mode(), sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        o = model(input_ids=prompt, use_cache=True, logits_to_keep=1)
        outs.append(o.logits[:, -1].float())
        cache = o.past_key_values
        for t in range(tokens.shape[1]):
            o = model(input_ids=tokens[:, t:t + 1], past_key_values=cache, use_cache=True, logits_to_keep=1)
            outs.append(o.logits[:, -1].float())
            cache = o.past_key_values
    return outs


def _rel(a, b):
    """max |a - b| relative to the largest |b|."""
    return float((a.float() - b.float()).abs().max()) / float(b.float().abs().max())


def _clear_argmax_agree(got, ref, rel):
    """Argmax equal wherever the reference's top-2 margin exceeds rel x its largest logit."""
    ref = ref.float()
    top2 = ref.topk(2, dim=-1).values
    clear = (top2[:, 0] - top2[:, 1]) > rel * float(ref.abs().max())
    return torch.equal(got.float().argmax(-1)[clear], ref.argmax(-1)[clear])


def _generate_three_ways(layers, tile_map, B=4, P=2048, O=256, prefill_ref=None):
    """Logits of every step from (1) the fused HIP-graph decode step, (2) the
    model's own modules replayed in the same decoder and (3) the eager
    Hugging Face forward, (2) and (3) teacher-forced on the tokens (1)
    generated; plus the generated ids.  Both decoders run the fused prefill;
    with ``prefill_ref`` (a dict) a third decoder prefills through the model's
    forward and the dict receives both prefills' last-token logits and
    layer-0 / last-layer caches."""
    from e2e_models import llama32_3b_config
    from tilequant_amd import api
    from tilequant_amd.graph_decode import CudaGraphGreedyDecoder
    from tilequant_amd.types import ApplyConfig

    config = llama32_3b_config()
    config.num_hidden_layers = layers
    kw = dict(keep_frac=0.01) if tile_map == "uniform_keep01" else dict(keep_dir=GOLDEN / "llama32_3b_gi_keep01")
    model, stats = api.build_mixed_precision_model(config, ApplyConfig(model_type="llama", dtype_out="bf16"), DEV,
                                                   seed=5, **kw)
    assert stats["num_targets"] == 7 * layers and stats["fused_projection_groups"] == 2 * layers
    prompt = torch.randint(0, config.vocab_size, (B, P), generator=torch.Generator().manual_seed(6))

    def caches(d):
        return [(d.cache.layers[i].keys[:, :, :P].clone(), d.cache.layers[i].values[:, :, :P].clone())
                for i in (0, layers - 1)]

    dec = CudaGraphGreedyDecoder.prepare(model, prompt_tokens=P, max_new_tokens=O, batch_size=B, device=DEV)
    assert dec._fused is not None and dec._fused_prefill is not None
    dec.prefill(prompt)
    fused = [dec.last_logits[:, -1].clone()]
    if prefill_ref is not None:
        prefill_ref["fused"] = (fused[0], caches(dec))
    for _ in range(O - 1):
        dec.decode(1)
        fused.append(dec.last_logits[:, -1].clone())
    ids = dec.decode(0).clone()
    assert ids.shape == (B, O)
    for t in range(O):   # every generated token is the device argmax of its step's logits
        assert torch.equal(ids[:, t], fused[t].float().argmax(-1)), t
    with pytest.raises(ValueError):
        dec.decode(1)    # the prepared bound is reached
    assert torch.equal(dec.generate(prompt), ids)   # a replayed request is identical
    dec.close()

    ref = CudaGraphGreedyDecoder.prepare(model, prompt_tokens=P, max_new_tokens=O, batch_size=B, device=DEV,
                                         fused_decode=False)
    assert ref._fused is None
    ref.prefill(prompt)
    module = [ref.last_logits[:, -1].clone()]
    for t in range(1, O):
        with torch.inference_mode():
            ref._token.copy_(ids[:, t - 1:t])
        ref._graph.replay()
        module.append(ref._decode_logits[:, -1].clone())
    ref.close()
    if prefill_ref is not None:
        from transformers.models.llama import modeling_llama

        def module_prefill():
            mf = CudaGraphGreedyDecoder.prepare(model, prompt_tokens=P, max_new_tokens=1, batch_size=B, device=DEV,
                                                fused_decode=False, fused_prefill=False)
            assert mf._fused_prefill is None
            mf.prefill(prompt)
            out = (mf.last_logits[:, -1].clone(), caches(mf))
            mf.close()
            return out

        prefill_ref["module"] = module_prefill()
        # the noise floor of a reordered sum: the same forward with each
        # RMSNorm's mean of squares taken in float64
        forward = modeling_llama.LlamaRMSNorm.forward

        def norm_f64(self, hidden_states):
            dt = hidden_states.dtype
            h = hidden_states.to(torch.float32)
            var = h.double().pow(2).mean(-1, keepdim=True).float()
            return self.weight * (h * torch.rsqrt(var + self.variance_epsilon)).to(dt)

        modeling_llama.LlamaRMSNorm.forward = norm_f64
        try:
            prefill_ref["module_f64"] = module_prefill()
        finally:
            modeling_llama.LlamaRMSNorm.forward = forward
    eager = _eager_teacher_forced(model, prompt.to(DEV), ids[:, :-1])
    return fused, module, eager


@pytest.mark.parametrize("tile_map", ["uniform_keep01", "released_gi_keep01"])
def test_llama32_3b_generation_real_shape(tile_map):
    """All 28 layers.  A random-initialised network this deep amplifies a
    single bf16 rounding flip to several percent of the largest logit (two
    reference-style paths -- the module step with this build's decode
    attention and the eager forward with SDPA -- differ by 12-16% at 28
    layers, 2-3% at one layer), so the per-step check is calibrated by that
    noise floor: the fused step may be no further from the module step, and
    at most 1.5x further from the eager forward, than the module step is from
    the eager forward.  A wrong position, cache layer, RoPE row, lm_head or
    greedy index gives O(1) differences, caught by the 0.3 bound.  The
    prefill logits of both decoders are bitwise equal (one prefill path).
    The fused prefill reorders each RMSNorm's fp32 sum of squares; the model's
    own forward with those sums taken in float64 moves the last token's logits
    by ~30% of the largest one at 28 layers (4.5% at one), so the fused
    prefill may be at most 1.5x as far from the model-forward prefill as that
    reordering is; layer 0's k/v for all 2048 x 4 prompt positions (RoPE rows,
    cache slots, batch rows), where nothing amplifies, must match within bf16
    rounding, and the model-forward prefill the eager forward tightly."""
    ref = {}
    fused, module, eager = _generate_three_ways(28, tile_map, prefill_ref=ref)
    assert torch.equal(module[0], fused[0])
    (lf, cf), (lm, cm), (l64, _) = ref["fused"], ref["module"], ref["module_f64"]
    assert _rel(lm, eager[0]) <= 3e-2
    for a, b in zip(cf[0], cm[0]):
        assert _rel(a, b) <= 2e-2
    floor = _rel(l64, lm)
    assert _rel(lf, lm) <= 1.5 * floor + 1e-2, (_rel(lf, lm), floor)
    for a, b in zip(cf[1], cm[1]):
        assert _rel(a, b) <= 0.3
    lead, worst = None, [0.0, 0.0, 0.0]
    for t in range(1, len(fused)):
        e_fm, e_me, e_fe = _rel(fused[t], module[t]), _rel(module[t], eager[t]), _rel(fused[t], eager[t])
        if lead is None and e_fm > 0:
            lead = t - 1
        worst = [max(w, e) for w, e in zip(worst, (e_fm, e_me, e_fe))]
        assert e_fm <= e_me + 1e-2, f"step {t}: fused-module {e_fm:.3e} > module-eager {e_me:.3e}"
        assert e_fe <= 1.5 * e_me + 1e-2, f"step {t}: fused-eager {e_fe:.3e} vs module-eager {e_me:.3e}"
        assert max(e_fm, e_fe) <= 0.3, t
    print(f"\n{tile_map}: fused == module bitwise for the first {lead if lead is not None else len(fused) - 1} "
          f"steps; worst fused-module {worst[0]:.2e}, module-eager {worst[1]:.2e}, fused-eager {worst[2]:.2e} "
          "of the largest logit")


def test_llama32_3b_widths_one_layer_tight():
    """One decoder layer at the real widths, vocabulary 128256, batch 4, a
    2048-token prompt and 256 new tokens (2304 keys at the end): little
    amplification, so the tight bars hold -- fused vs module and vs eager
    within 3e-2 / 5e-2 of the largest logit, argmax equal where the margin is
    clear."""
    ref = {}
    fused, module, eager = _generate_three_ways(1, "uniform_keep01", prefill_ref=ref)
    assert torch.equal(module[0], fused[0])
    (lf, cf), (lm, cm), (l64, _) = ref["fused"], ref["module"], ref["module_f64"]
    floor = _rel(l64, lm)   # the model's forward with float64 RMSNorm sums
    assert _rel(lf, lm) <= 1.5 * floor + 1e-2, (_rel(lf, lm), floor)
    assert _clear_argmax_agree(lf, lm, 5e-2)
    for a, b in zip(cf[0], cm[0]):
        assert _rel(a, b) <= 2e-2
    for t in range(len(fused)):
        assert _rel(fused[t], module[t]) <= 3e-2 and _clear_argmax_agree(fused[t], module[t], 3e-2), t
        assert _rel(fused[t], eager[t]) <= 5e-2 and _clear_argmax_agree(fused[t], eager[t], 5e-2), t


def test_llama32_3b_single_steps_from_identical_state():
    """All 28 layers, batch 4, 2048-token prompt, 256 new tokens.  At decode
    positions P, P + 64 and P + 254 (the last of the 255 decode steps) the fused
    decoder's whole state (every
    layer's K/V cache, the input token, the position and the valid lengths)
    is copied into a decoder that replays the model's own modules, and each
    runs ONE step from it (reference decode body: graph_decode.py:350-385), so
    no divergence accumulates over steps.  Depth still amplifies: this
    random-initialised 28-layer network turns a single fp32 reordering in one
    RMSNorm into ~10% of the largest logit within one step.  So the floor is
    measured at every position: the same module step from the same state with
    every RMSNorm's mean of squares taken in float64.  Bars: fused-vs-module
    logits within 1.5x that floor + 1e-2 (and 0.3 absolute), argmax equal
    where the margin exceeds the floor; the K/V the step writes at layer 0,
    before anything amplifies, equal within bf16 rounding (2e-2)."""
    from transformers.models.llama import modeling_llama

    from e2e_models import llama32_3b_config
    from tilequant_amd import api
    from tilequant_amd.graph_decode import CudaGraphGreedyDecoder
    from tilequant_amd.types import ApplyConfig

    B, P, O = 4, 2048, 256
    config = llama32_3b_config()
    model, _ = api.build_mixed_precision_model(config, ApplyConfig(model_type="llama", dtype_out="bf16"), DEV,
                                               seed=5, keep_frac=0.01)
    prompt = torch.randint(0, config.vocab_size, (B, P), generator=torch.Generator().manual_seed(6))

    def load_state(dec, state):
        with torch.inference_mode():
            for layer, (k, v) in zip(dec.cache.layers, state[0]):
                layer.keys.copy_(k)
                layer.values.copy_(v)
                # the static cache layer writes at its own device counter of the
                # tokens it holds (kept equal to the position by the decoder)
                layer.cumulative_length.copy_(state[2].to(layer.cumulative_length.dtype).view_as(
                    layer.cumulative_length))
            dec._token.copy_(state[1])
            dec._position.copy_(state[2])
            dec._decode_seq_used.copy_(state[3])
            if len(state) > 4:
                dec._generated.copy_(state[4])

    def save_state(dec):
        return ([(layer.keys.clone(), layer.values.clone()) for layer in dec.cache.layers], dec._token.clone(),
                dec._position.clone(), dec._decode_seq_used.clone(), dec._generated.clone())

    def entry(dec, pos, layer):
        return dec.cache.layers[layer].keys[:, :, pos].clone(), dec.cache.layers[layer].values[:, :, pos].clone()

    forward = modeling_llama.LlamaRMSNorm.forward

    def norm_f64(self, hidden_states):
        dt = hidden_states.dtype
        h = hidden_states.to(torch.float32)
        var = h.double().pow(2).mean(-1, keepdim=True).float()
        return self.weight * (h * torch.rsqrt(var + self.variance_epsilon)).to(dt)

    fused = CudaGraphGreedyDecoder.prepare(model, prompt_tokens=P, max_new_tokens=O, batch_size=B, device=DEV)
    assert fused._fused is not None and len(fused.cache.layers) == 28
    fused.prefill(prompt)
    done, report = 0, []
    for target in (0, 64, 254):
        if target > done:
            fused.decode(target - done)
            done = target
        state = save_state(fused)
        pos = int(state[2].item())
        assert pos == P + target
        fused.decode(1)
        done += 1
        lf = fused.last_logits[:, -1].float().clone()
        kf0, vf0 = entry(fused, pos, 0)
        after = save_state(fused)
        fused.close()   # one decoder bound to the model at a time
        ref = CudaGraphGreedyDecoder.prepare(model, prompt_tokens=P, max_new_tokens=O, batch_size=B, device=DEV,
                                             fused_decode=False, fused_prefill=False)
        load_state(ref, state)
        ref._graph.replay()
        lm = ref._decode_logits[:, -1].float().clone()
        km0, vm0 = entry(ref, pos, 0)
        load_state(ref, state)
        modeling_llama.LlamaRMSNorm.forward = norm_f64
        try:
            ref._decode_body()   # the module step eagerly, float64 norm sums
        finally:
            modeling_llama.LlamaRMSNorm.forward = forward
        l64 = ref._decode_logits[:, -1].float().clone()
        ref.close()
        e, floor = _rel(lf, lm), _rel(l64, lm)
        report.append((target, e, floor))
        assert _rel(kf0, km0) <= 2e-2 and _rel(vf0, vm0) <= 2e-2, f"position P + {target}: layer-0 cache entry"
        assert e <= 1.5 * floor + 1e-2 and e <= 0.3, f"position P + {target}: {e:.3e} vs floor {floor:.3e}"
        assert _clear_argmax_agree(lf, lm, max(floor, 3e-2)), f"position P + {target}"
        if target != 254:   # back to the fused decoder, at its own state after the step
            fused = CudaGraphGreedyDecoder.prepare(model, prompt_tokens=P, max_new_tokens=O, batch_size=B,
                                                   device=DEV)
            fused.prefill(prompt)   # sets the decoder up; its state is then replaced
            load_state(fused, after)
            fused._steps_done = done
        del state, after
    print("\nsingle steps (position - P, fused-vs-module, float64-norm floor): "
          + ", ".join(f"({t}, {e:.2e}, {f:.2e})" for t, e, f in report))
