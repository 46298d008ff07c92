"""GPU: decode attention kernel, load-time packing driver and the HIP-graph
greedy decoder (mirrors of src/quantization/api.py and src/runtime/graph_decode.py).

Bars: attention output within 2 bf16 ulp of a float64 reference (fp32
accumulation); loaded models bitwise equal to models packed directly from the
same weights; decoder logits equal to the eager forward within bf16 rounding
noise, identical across replays."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from e2e_models import tiny_llama_config, tiny_qwen2_config, write_checkpoint, write_tile_maps
from tilequant_amd import api
from tilequant_amd.attention import decode_attention, decode_attention_workspace
from tilequant_amd.mixed_linear import MixedLinear
from tilequant_amd.pack import pack_weight_from_tile_ids
from tilequant_amd.rules import iter_target_linears
from tilequant_amd.types import ApplyConfig

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _attention_reference(q, k, v, lens, scale):
    """float64 softmax attention of each sequence over its first lens[b] keys."""
    q, k, v = (t.double().cpu() for t in (q, k, v))
    B, Hq, D = q.shape
    G = Hq // k.shape[1]
    out = torch.zeros((B, Hq, D), dtype=torch.float64)
    for b in range(B):
        n = int(lens[b])
        if n == 0:
            continue
        kk = k[b, :, :n].repeat_interleave(G, dim=0)      # [Hq, n, D]
        vv = v[b, :, :n].repeat_interleave(G, dim=0)
        s = torch.einsum("hd,hnd->hn", q[b], kk) * scale
        p = torch.softmax(s, dim=-1)
        out[b] = torch.einsum("hn,hnd->hd", p, vv)
    return out


@pytest.mark.parametrize("B,Hq,Hkv,L", [(4, 24, 8, 2304), (2, 7, 1, 300), (1, 8, 1, 64), (3, 40, 8, 513),
                                          (2, 8, 2, 8400), (3, 6, 3, 500), (2, 6, 1, 700), (1, 4, 4, 1000)])
@pytest.mark.parametrize("token_major", [False, True])
def test_decode_attention_matches_reference(B, Hq, Hkv, L, token_major):
    g = torch.Generator().manual_seed(B * 1000 + L)
    D = 128
    q = torch.randn((B, Hq, D), generator=g).to(torch.bfloat16)
    if token_major:   # [B, L, Hkv, D] storage viewed as [B, Hkv, L, D]
        k = torch.randn((B, L, Hkv, D), generator=g).to(torch.bfloat16).transpose(1, 2)
        v = torch.randn((B, L, Hkv, D), generator=g).to(torch.bfloat16).transpose(1, 2)
    else:
        k = torch.randn((B, Hkv, L, D), generator=g).to(torch.bfloat16)
        v = torch.randn((B, Hkv, L, D), generator=g).to(torch.bfloat16)
    lens = [L, 1, 256, 257][:B] if B > 1 else [L // 2 + 3]
    lens = [min(x, L) for x in lens]
    scale = D ** -0.5
    kd, vd = k.to(DEV), v.to(DEV)
    out = decode_attention(q.to(DEV), kd, vd, torch.tensor(lens, dtype=torch.int32, device=DEV), scale=scale)
    ref = _attention_reference(q, k, v, lens, scale)
    got = out.double().cpu()
    ulp = torch.exp2(torch.floor(torch.log2(ref.abs().clamp_min(2.0 ** -126))) - 7)
    assert bool(((got - ref).abs() <= 2 * ulp + 1e-6).all()), float(((got - ref).abs() / ulp).max())
    # bitwise reproducible
    assert torch.equal(decode_attention(q.to(DEV), kd, vd, torch.tensor(lens, dtype=torch.int32, device=DEV),
                                        scale=scale), out)


@pytest.mark.parametrize("q_scale", [1.0, 4.0])
def test_decode_attention_fp32_accuracy_near_uniform(q_scale):
    """Near-uniform attention over long sequences (random q, k, v; 2304 keys)
    gives outputs that cancel to a small fraction of sum_t p_t |v_t|, where an
    error of the probabilities' precision shows in ulps: with fp32-accurate
    products and sums at most 0.1% of the bf16 outputs may differ from the
    correctly rounded float64 result (fp32 probabilities: 0.02-0.07%;
    probabilities carried to 16 significant bits: 0.12-0.26%), and each output
    stays within 2 ulp plus 2^-18 of sum_t p_t |v_t|."""
    B, Hq, Hkv, L, D = 4, 24, 8, 2304, 128
    lens = [2304, 2049, 1000, 77]
    for seed in range(3):
        g = torch.Generator().manual_seed(100 + seed)
        q = (torch.randn((B, Hq, D), generator=g) * q_scale).to(torch.bfloat16)
        k = torch.randn((B, Hkv, L, D), generator=g).to(torch.bfloat16)
        v = torch.randn((B, Hkv, L, D), generator=g).to(torch.bfloat16)
        out = decode_attention(q.to(DEV), k.to(DEV), v.to(DEV), torch.tensor(lens, dtype=torch.int32, device=DEV),
                               scale=D ** -0.5)
        ref = _attention_reference(q, k, v, lens, D ** -0.5)
        mag = _attention_reference(q, k, v.abs(), lens, D ** -0.5)   # sum_t p_t |v_t|
        got = out.double().cpu()
        mismatch = float((got != ref.to(torch.bfloat16).double()).double().mean())
        assert mismatch <= 1e-3, (seed, mismatch)
        ulp = torch.exp2(torch.floor(torch.log2(ref.abs().clamp_min(2.0 ** -126))) - 7)
        assert bool(((got - ref).abs() <= 2 * ulp + mag * 2.0 ** -18).all()), seed


def test_decode_attention_graph_replays_follow_device_length():
    B, Hq, Hkv, L, D = 2, 24, 8, 600, 128
    g = torch.Generator().manual_seed(5)
    q = torch.randn((B, Hq, D), generator=g).to(torch.bfloat16).to(DEV)
    k = torch.randn((B, Hkv, L, D), generator=g).to(torch.bfloat16).to(DEV)
    v = torch.randn((B, Hkv, L, D), generator=g).to(torch.bfloat16).to(DEV)
    seq = torch.ones((B,), dtype=torch.int32, device=DEV)
    ws = decode_attention_workspace(B, Hq, L, DEV)
    out = torch.empty((B, Hq, D), dtype=torch.bfloat16, device=DEV)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        decode_attention(q, k, v, seq, scale=D ** -0.5, out=out, workspace=ws)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        decode_attention(q, k, v, seq, scale=D ** -0.5, out=out, workspace=ws)
    for n in (1, 255, 256, 257, 599, 600, 17):
        seq.fill_(n)
        graph.replay()
        torch.cuda.synchronize()
        want = decode_attention(q, k, v, torch.full((B,), n, dtype=torch.int32, device=DEV), scale=D ** -0.5)
        assert torch.equal(out, want), n


def test_decode_attention_argument_errors():
    q = torch.zeros((1, 4, 64), dtype=torch.bfloat16, device=DEV)
    k = torch.zeros((1, 2, 8, 64), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):   # head_dim 64 is not served
        decode_attention(q, k, k, torch.ones(1, dtype=torch.int32, device=DEV), scale=1.0)
    q = torch.zeros((1, 4, 128), dtype=torch.bfloat16, device=DEV)
    k = torch.zeros((1, 2, 8, 128), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):
        decode_attention(q, k, k, torch.ones(1, dtype=torch.int64, device=DEV), scale=1.0)


def _direct_model(model_dir, keep_dir, apply_cfg):
    """Dense checkpoint model with every target swapped for a directly packed MixedLinear (no groups)."""
    from transformers import AutoModelForCausalLM

    model = AutoModelForCausalLM.from_pretrained(model_dir, dtype=torch.bfloat16, attn_implementation="sdpa").to(DEV)
    cfg = api._make_cfg(apply_cfg)
    maps = api.validate_fp16_ids_coverage_and_shapes(model, keep_dir, apply_cfg)
    for parent, attr, name, lin in iter_target_linears(model, cfg, apply_cfg.model_type):
        f16, i8, n_tr, n_tc = maps[name]
        pack = pack_weight_from_tile_ids(lin.weight.detach(), n_tr=n_tr, n_tc=n_tc, int8_tile_ids=i8,
                                         fp16_tile_ids=f16, cfg=cfg)
        bias = lin.bias.detach() if lin.bias is not None else None
        setattr(parent, attr, MixedLinear(pack, bias, cfg).to(DEV))
    return model.eval()


@pytest.mark.parametrize("family", ["llama", "qwen"])
def test_loader_equals_direct_packing_bitwise(tmp_path, family):
    config = tiny_llama_config() if family == "llama" else tiny_qwen2_config()
    sd = write_checkpoint(config, tmp_path / "ckpt", seed=11, shards=2)
    write_tile_maps(config, tmp_path / "keep10", frac=0.1, seed=12, model_type=family)
    apply_cfg = ApplyConfig(model_type=family, dtype_out="bf16")
    model, stats = api.load_mixed_precision_model_from_masks(tmp_path / "ckpt", tmp_path / "keep10", apply_cfg,
                                                             torch.bfloat16, DEV, attn_implementation="sdpa")
    assert stats["num_targets"] == 14 and stats["num_replaced_during_load"] == 14
    assert stats["fused_projection_groups"] == 4          # QKV and Gate/Up per layer
    emb = model.get_input_embeddings().weight
    assert torch.equal(emb.cpu(), sd["model.embed_tokens.weight"])
    ref = _direct_model(tmp_path / "ckpt", tmp_path / "keep10", apply_cfg)
    ids = torch.randint(0, config.vocab_size, (2, 40), generator=torch.Generator().manual_seed(1)).to(DEV)
    with torch.inference_mode():
        a = model(input_ids=ids).logits
        b = ref(input_ids=ids).logits
    assert torch.equal(a, b)   # stacked groups == members, same packing, same kernels


def test_random_init_builder_packs_every_target():
    config = tiny_llama_config()
    apply_cfg = ApplyConfig(model_type="llama", dtype_out="bf16")
    model, stats = api.build_mixed_precision_model(config, apply_cfg, DEV, keep_frac=0.05, seed=3)
    assert stats["num_targets"] == 14 and stats["fused_projection_groups"] == 4
    assert all(p.device.type == "cuda" for p in model.parameters())
    ids = torch.randint(0, config.vocab_size, (1, 8)).to(DEV)
    with torch.inference_mode():
        logits = model(input_ids=ids).logits
    assert logits.shape == (1, 8, config.vocab_size) and bool(torch.isfinite(logits).all())


def _eager_teacher_forced(model, prompt, tokens):
    """Eager forward with a DynamicCache on fused SDPA, fed the given tokens:
    last-position logits of the prompt and of every following step."""
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


def test_graph_decoder_matches_eager_and_replays_independently():
    from tilequant_amd.graph_decode import CudaGraphGreedyDecoder

    config = tiny_llama_config(layers=2)
    model, _ = api.build_mixed_precision_model(config, ApplyConfig(model_type="llama", dtype_out="bf16"), DEV,
                                               keep_frac=0.05, seed=21)
    B, P, O = 2, 96, 12
    g = torch.Generator().manual_seed(22)
    prompt = torch.randint(0, config.vocab_size, (B, P), generator=g)
    dec = CudaGraphGreedyDecoder.prepare(model, prompt_tokens=P, max_new_tokens=O, batch_size=B, device=DEV)
    assert dec.prefill_captured
    first = dec.prefill(prompt).clone()   # the returned token buffer is reused by decode
    prefill_logits = dec.last_logits[:, -1].float().clone()
    ids = dec.decode(O - 1).clone()
    assert ids.shape == (B, O) and torch.equal(ids[:, :1], first)
    # every generated token is the argmax of the decoder's own logits; compare with
    # the eager model fed the same tokens
    other = torch.randint(0, config.vocab_size, (B, P), generator=g)
    ids_other = dec.generate(other).clone()
    again = dec.generate(prompt).clone()
    assert torch.equal(again, ids)                 # reset-and-prefill makes replays independent
    dec.close()
    ref = _eager_teacher_forced(model, prompt.to(DEV), ids[:, :-1])
    scale = max(float(r.abs().max()) for r in ref)
    assert float((prefill_logits - ref[0]).abs().max()) <= 2e-2 * scale
    # the decode graph's argmax agrees with the eager logits wherever the eager
    # margin between the best two logits exceeds the rounding noise
    for t in range(1, O):
        r = ref[t]
        top2 = r.topk(2, dim=-1).values
        clear = (top2[:, 0] - top2[:, 1]) > 2e-2 * scale
        assert torch.equal(r.argmax(-1)[clear], ids[:, t][clear]), t
    assert not torch.equal(ids_other, ids)


def test_decoder_argument_errors():
    from tilequant_amd.graph_decode import CudaGraphGreedyDecoder

    config = tiny_llama_config(layers=1)
    model, _ = api.build_mixed_precision_model(config, ApplyConfig(model_type="llama", dtype_out="bf16"), DEV,
                                               keep_frac=0.05, seed=1)
    with pytest.raises(ValueError):
        CudaGraphGreedyDecoder(model, prompt_tokens=0, max_new_tokens=4, device=DEV)
    dec = CudaGraphGreedyDecoder.prepare(model, prompt_tokens=8, max_new_tokens=3, batch_size=1, device=DEV)
    with pytest.raises(ValueError):
        dec.prefill(torch.zeros((1, 9), dtype=torch.long))
    with pytest.raises(ValueError):
        dec.decode(5)
    dec.prefill(torch.zeros((1, 8), dtype=torch.long))
    assert dec.decode(1).shape == (1, 2)
    with pytest.raises(ValueError, match="prepared bound"):
        dec.decode(2)                  # 1 + 2 steps would pass the cache end (3 new tokens)
    assert dec.decode(1).shape == (1, 3)
    dec.prefill(torch.zeros((1, 8), dtype=torch.long))
    assert dec.decode(2).shape == (1, 3)
    with pytest.raises(RuntimeError, match="already has"):
        CudaGraphGreedyDecoder(model, prompt_tokens=8, max_new_tokens=3, device=DEV)
    dec.close()


# ---- fused decode-step kernels -------------------------------------------------------------------
from tilequant_amd import _native as nat                               # noqa: E402
from tilequant_amd.quant_utils import quantize_activation_tile_absmax   # noqa: E402


def _ulp_close(a: torch.Tensor, b: torch.Tensor, ulps: float = 1.0) -> bool:
    """|a - b| within `ulps` units in the last place of b in b's 16-bit type
    (7 fraction bits for bf16, 10 for fp16; fp16's subnormal spacing below 2^-14)."""
    frac, low = (10, -14) if b.dtype == torch.float16 else (7, -126)
    a, b = a.float(), b.float()
    ulp = torch.exp2(torch.floor(torch.log2(b.abs().clamp_min(2.0 ** low))) - frac)
    return bool(((a - b).abs() <= ulps * ulp).all())


@pytest.mark.parametrize("n,k,with_delta,dtype", [(4, 3072, True, torch.bfloat16), (1, 3072, False, torch.bfloat16),
                                                  (16, 512, True, torch.bfloat16), (3, 8192, True, torch.bfloat16),
                                                  (7, 3072, True, torch.bfloat16), (40, 1024, True, torch.bfloat16),
                                                  (64, 512, False, torch.bfloat16), (13, 3072, False, torch.bfloat16),
                                                  (4, 3584, True, torch.float16), (20, 1024, False, torch.float16)])
def test_add_rmsnorm_quant_matches_module_and_quantizer(n, k, with_delta, dtype):
    from transformers.models.llama.modeling_llama import LlamaRMSNorm

    g = torch.Generator().manual_seed(n * 7 + k)
    x = (torch.randn((n, k), generator=g) * 3).to(dtype).to(DEV)
    d = (torch.randn((n, k), generator=g) * 2).to(dtype).to(DEV)
    norm = LlamaRMSNorm(k, eps=1e-5).to(DEV).to(dtype)
    norm.weight.data = (1 + 0.1 * torch.randn(k, generator=g)).to(dtype).to(DEV)
    h_ref = (x + d) if with_delta else x
    with torch.inference_mode():
        y_ref = norm(h_ref)
    h = torch.empty_like(x)
    y = torch.empty_like(x)
    q = torch.empty((n, k), dtype=torch.int8, device=DEV)
    sx = torch.empty((k // 64,), dtype=torch.float32, device=DEV)
    rc = nat.lib().tq_add_rmsnorm_quant(x.data_ptr(), k, d.data_ptr() if with_delta else None, k,
                                        norm.weight.data_ptr(), 1e-5, h.data_ptr(), k, y.data_ptr(), k,
                                        q.data_ptr(), k, sx.data_ptr(), nat.dtype_code(dtype), n, k, None,
                                        torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    if with_delta:
        assert torch.equal(h, h_ref)                       # the residual add rounds exactly like torch
    assert _ulp_close(y, y_ref, 1.0)                        # only the sum-of-squares order differs
    q_ref, sx_ref = quantize_activation_tile_absmax(y)
    assert torch.equal(q, q_ref) and torch.equal(sx, sx_ref)   # same closed form as the quantizer, bitwise


@pytest.mark.parametrize("n,inter,dtype", [(4, 8192, torch.bfloat16), (1, 1024, torch.bfloat16),
                                           (16, 512, torch.bfloat16), (7, 8192, torch.bfloat16),
                                           (33, 1024, torch.bfloat16), (64, 512, torch.bfloat16),
                                           (4, 18944, torch.float16), (9, 1024, torch.float16)])
def test_silu_mul_quant_matches_module_and_quantizer(n, inter, dtype):
    g = torch.Generator().manual_seed(n + inter)
    gu = (torch.randn((n, 2 * inter), generator=g) * 2).to(dtype).to(DEV)
    with torch.inference_mode():
        y_ref = torch.nn.functional.silu(gu[:, :inter]) * gu[:, inter:]
    y = torch.empty((n, inter), dtype=dtype, device=DEV)
    q = torch.empty((n, inter), dtype=torch.int8, device=DEV)
    sx = torch.empty((inter // 64,), dtype=torch.float32, device=DEV)
    rc = nat.lib().tq_silu_mul_quant(gu.data_ptr(), 2 * inter, y.data_ptr(), inter, q.data_ptr(), inter,
                                     sx.data_ptr(), nat.dtype_code(dtype), n, inter, None,
                                     torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    assert _ulp_close(y, y_ref, 1.0)
    q_ref, sx_ref = quantize_activation_tile_absmax(y)
    assert torch.equal(q, q_ref) and torch.equal(sx, sx_ref)


@pytest.mark.parametrize("n,k,with_delta,dtype", [(1000, 3072, True, torch.bfloat16), (37, 3072, False, torch.bfloat16),
                                                   (513, 5120, True, torch.bfloat16), (64, 8192, True, torch.float16),
                                                   (8, 200, True, torch.bfloat16)])
def test_add_rmsnorm_rows_matches_module(n, k, with_delta, dtype):
    """Prefill form: h bitwise torch's add, y within 1 ulp of LlamaRMSNorm (sum-of-squares order only)."""
    from transformers.models.llama.modeling_llama import LlamaRMSNorm

    g = torch.Generator().manual_seed(n * 3 + k)
    x = (torch.randn((n, k), generator=g) * 3).to(dtype).to(DEV)
    d = (torch.randn((n, k), generator=g) * 2).to(dtype).to(DEV)
    norm = LlamaRMSNorm(k, eps=1e-6).to(DEV).to(dtype)
    norm.weight.data = (1 + 0.1 * torch.randn(k, generator=g)).to(dtype).to(DEV)
    h_ref = (x + d) if with_delta else x
    with torch.inference_mode():
        y_ref = norm(h_ref)
    h = torch.full_like(x, 7.0)
    y = torch.empty_like(x)
    rc = nat.lib().tq_add_rmsnorm_rows(x.data_ptr(), k, d.data_ptr() if with_delta else None, k, norm.weight.data_ptr(),
                                       1e-6, h.data_ptr() if with_delta else None, k, y.data_ptr(), k,
                                       nat.dtype_code(dtype), n, k, torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    if with_delta:
        assert torch.equal(h, h_ref)
    else:
        assert bool((h == 7.0).all())                       # no h without a delta
    # the fp32 sum of squares is ordered differently from torch's mean: where
    # that moves h * rsqrt across a rounding boundary, round(h * r) moves one
    # ulp and weight * it up to two; such elements are rare
    assert _ulp_close(y, y_ref, 2.0)
    assert float((y != y_ref).float().mean()) < 1e-3


@pytest.mark.parametrize("n,inter,dtype", [(4096, 8192, torch.bfloat16), (333, 1024, torch.bfloat16),
                                           (17, 136, torch.float16), (9, 192, torch.float16)])
def test_silu_mul_rows_matches_module(n, inter, dtype):
    g = torch.Generator().manual_seed(n + inter)
    gu = (torch.randn((n, 2 * inter), generator=g) * 2).to(dtype).to(DEV)
    with torch.inference_mode():
        y_ref = torch.nn.functional.silu(gu[:, :inter]) * gu[:, inter:]
    y = torch.empty((n, inter), dtype=dtype, device=DEV)
    rc = nat.lib().tq_silu_mul_rows(gu.data_ptr(), 2 * inter, y.data_ptr(), inter, nat.dtype_code(dtype), n, inter,
                                    torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    assert _ulp_close(y, y_ref, 1.0)
    # the decode form on the same rows gives the same values
    if n <= 64 and inter % 64 == 0:
        y2 = torch.empty_like(y)
        rc = nat.lib().tq_silu_mul_quant(gu.data_ptr(), 2 * inter, y2.data_ptr(), inter, None, inter, None,
                                         nat.dtype_code(dtype), n, inter, None, torch.cuda.current_stream().cuda_stream)
        assert rc == 0
        torch.cuda.synchronize()
        assert torch.equal(y, y2)


@pytest.mark.parametrize("B,P,hq,hkv,L", [(2, 37, 24, 8, 64), (1, 300, 8, 2, 300), (3, 5, 28, 4, 9)])
def test_rope_prefill_matches_module_ops(B, P, hq, hkv, L):
    """Every prompt position rotated with its own table row, bitwise the modules' RoPE;
    k / v land at cache index p, nothing past P is written."""
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb

    D = 128
    g = torch.Generator().manual_seed(B * 100 + P)
    qkv = torch.randn((B * P, (hq + 2 * hkv) * D), generator=g).to(torch.bfloat16).to(DEV)
    ang = torch.randn((L, D), generator=g)
    cos, sin = ang.cos().to(torch.bfloat16).to(DEV), ang.sin().to(torch.bfloat16).to(DEV)
    kc = torch.zeros((B, hkv, L, D), dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    q_out = torch.empty((B, hq, P, D), dtype=torch.bfloat16, device=DEV)
    rc = nat.lib().tq_rope_prefill(qkv.data_ptr(), qkv.stride(0), cos.data_ptr(), sin.data_ptr(), cos.stride(0),
                                   q_out.data_ptr(), q_out.stride(0), q_out.stride(1), q_out.stride(2), kc.data_ptr(),
                                   vc.data_ptr(), kc.stride(0), kc.stride(1), kc.stride(2), 0, B, P, hq, hkv, D, L,
                                   torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    q = qkv[:, :hq * D].view(B, P, hq, D).transpose(1, 2)
    k = qkv[:, hq * D:(hq + hkv) * D].view(B, P, hkv, D).transpose(1, 2)
    v = qkv[:, (hq + hkv) * D:].view(B, P, hkv, D).transpose(1, 2)
    q_ref, k_ref = apply_rotary_pos_emb(q, k, cos[:P].view(1, P, D), sin[:P].view(1, P, D))
    torch.cuda.synchronize()
    assert torch.equal(q_out, q_ref)
    assert torch.equal(kc[:, :, :P], k_ref) and torch.equal(vc[:, :, :P], v)
    assert int(kc[:, :, P:].abs().sum()) == 0 and int(vc[:, :, P:].abs().sum()) == 0


def test_rope_cache_matches_module_ops():
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb

    B, hq, hkv, D, L, pos = 4, 24, 8, 128, 300, 137
    g = torch.Generator().manual_seed(3)
    qkv = torch.randn((B, (hq + 2 * hkv) * D), generator=g).to(torch.bfloat16).to(DEV)
    ang = torch.randn(D, generator=g)
    cos, sin = ang.cos().to(torch.bfloat16).to(DEV), ang.sin().to(torch.bfloat16).to(DEV)
    kc = torch.zeros((B, hkv, L, D), dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    q_out = torch.empty((B, hq, D), dtype=torch.bfloat16, device=DEV)
    position = torch.tensor([pos], dtype=torch.int64, device=DEV)
    rc = nat.lib().tq_rope_cache(qkv.data_ptr(), qkv.stride(0), cos.data_ptr(), sin.data_ptr(), position.data_ptr(),
                                 q_out.data_ptr(), q_out.stride(0), q_out.stride(1), kc.data_ptr(), vc.data_ptr(),
                                 kc.stride(0), kc.stride(1), kc.stride(2), 0, B, hq, hkv, D, L,
                                 torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    q = qkv[:, :hq * D].view(B, 1, hq, D).transpose(1, 2)
    k = qkv[:, hq * D:(hq + hkv) * D].view(B, 1, hkv, D).transpose(1, 2)
    v = qkv[:, (hq + hkv) * D:].view(B, 1, hkv, D).transpose(1, 2)
    q_ref, k_ref = apply_rotary_pos_emb(q, k, cos.view(1, 1, D), sin.view(1, 1, D))
    torch.cuda.synchronize()
    assert torch.equal(q_out, q_ref[:, :, 0])
    assert torch.equal(kc[:, :, pos], k_ref[:, :, 0]) and torch.equal(vc[:, :, pos], v[:, :, 0])
    assert int(kc[:, :, :pos].abs().sum()) == 0 and int(vc[:, :, pos + 1:].abs().sum()) == 0


@pytest.mark.parametrize("B,L", [(4, 700), (7, 700), (13, 300), (16, 9000)])
def test_attention_quant_equals_attention_then_quantizer(B, L):
    Hq, Hkv, D = 24, 8, 128
    g = torch.Generator().manual_seed(9 + B)
    q = torch.randn((B, Hq, D), generator=g).to(torch.bfloat16).to(DEV)
    k = torch.randn((B, Hkv, L, D), generator=g).to(torch.bfloat16).to(DEV)
    v = torch.randn((B, Hkv, L, D), generator=g).to(torch.bfloat16).to(DEV)
    seq = torch.tensor(([L, 1, 129, 400] * 4)[:B], dtype=torch.int32, device=DEV)
    ref = decode_attention(q, k, v, seq, scale=D ** -0.5)
    out = torch.empty((B, Hq * D), dtype=torch.bfloat16, device=DEV)
    qo = torch.empty((B, Hq * D), dtype=torch.int8, device=DEV)
    sx = torch.empty((Hq * D // 64,), dtype=torch.float32, device=DEV)
    ws = decode_attention_workspace(B, Hq, L, DEV)
    rc = nat.lib().tq_decode_attention_quant(q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), v.data_ptr(),
                                             k.stride(0), k.stride(2), k.stride(1), seq.data_ptr(), out.data_ptr(),
                                             out.stride(0), D, qo.data_ptr(), qo.stride(0), sx.data_ptr(), 0, B, Hq,
                                             Hkv, D, L, D ** -0.5, ws.data_ptr(), ws.numel(),
                                             torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    assert torch.equal(out.view(B, Hq, D), ref)
    q_ref, sx_ref = quantize_activation_tile_absmax(out)
    assert torch.equal(qo, q_ref) and torch.equal(sx, sx_ref)


@pytest.mark.parametrize("B,hq,hkv,L,pos,quant", [(4, 24, 8, 2304, 2047, True), (4, 24, 8, 700, 128, False),
                                                    (2, 7, 1, 300, 0, True), (3, 40, 8, 513, 127, True),
                                                    (1, 8, 2, 256, 255, False), (2, 24, 8, 300, 300, True),
                                                    (3, 6, 3, 500, 411, True), (2, 6, 1, 700, 650, False),
                                                    (5, 4, 4, 1000, 999, True)])
def test_attention_rope_equals_rope_cache_then_attention(B, hq, hkv, L, pos, quant):
    """tq_decode_attention_rope against tq_rope_cache followed by
    tq_decode_attention(_quant): outputs, codes, scales and both caches
    bitwise equal.  Positions at chunk edges (0, 127, 128, 255) and in the
    middle; seq_used = position + 1 except one row whose length stops short of
    the new key (it must not be read); pos == L writes nothing.  The fused
    entry reads cos / sin from [L, 128] tables at the device position (the
    row index clamped into the table)."""
    D = 128
    g = torch.Generator().manual_seed(B * 31 + pos)
    qkv = torch.randn((B, (hq + 2 * hkv) * D), generator=g).to(torch.bfloat16).to(DEV)
    ang = torch.randn(D, generator=g) * 3
    cos, sin = ang.cos().to(torch.bfloat16).to(DEV), ang.sin().to(torch.bfloat16).to(DEV)
    cos_t = torch.randn((L, D), generator=g).to(torch.bfloat16).to(DEV)
    sin_t = torch.randn((L, D), generator=g).to(torch.bfloat16).to(DEV)
    cos_t[min(pos, L - 1)] = cos
    sin_t[min(pos, L - 1)] = sin
    kc0 = torch.randn((B, hkv, L, D), generator=g).to(torch.bfloat16).to(DEV)
    vc0 = torch.randn((B, hkv, L, D), generator=g).to(torch.bfloat16).to(DEV)
    position = torch.tensor([pos], dtype=torch.int64, device=DEV)
    seq = torch.full((B,), min(pos + 1, L), dtype=torch.int32, device=DEV)
    if B > 1:
        seq[1] = max(pos - 5, 1)
    ws = decode_attention_workspace(B, hq, L, DEV)
    stream = torch.cuda.current_stream().cuda_stream
    code = 0

    def outputs():
        return (torch.full((B, hq * D), 7.0, dtype=torch.bfloat16, device=DEV),
                torch.zeros((B, hq * D), dtype=torch.int8, device=DEV),
                torch.zeros((hq * D // 64,), dtype=torch.float32, device=DEV))

    # two launches
    kc1, vc1 = kc0.clone(), vc0.clone()
    q_rot = torch.empty((B, hq, D), dtype=torch.bfloat16, device=DEV)
    rc = nat.lib().tq_rope_cache(qkv.data_ptr(), qkv.stride(0), cos.data_ptr(), sin.data_ptr(), position.data_ptr(),
                                 q_rot.data_ptr(), q_rot.stride(0), q_rot.stride(1), kc1.data_ptr(), vc1.data_ptr(),
                                 kc1.stride(0), kc1.stride(1), kc1.stride(2), code, B, hq, hkv, D, L, stream)
    assert rc == 0
    if pos >= L:   # tq_rope_cache leaves q untouched for a position outside the cache: rotate it here
        from transformers.models.llama.modeling_llama import apply_rotary_pos_emb
        qh = qkv[:, :hq * D].view(B, 1, hq, D).transpose(1, 2)
        q_rot.copy_(apply_rotary_pos_emb(qh, qh, cos.view(1, 1, D), sin.view(1, 1, D))[0][:, :, 0])
    out1, qo1, sx1 = outputs()
    args = (q_rot.data_ptr(), q_rot.stride(0), q_rot.stride(1), kc1.data_ptr(), vc1.data_ptr(), kc1.stride(0),
            kc1.stride(2), kc1.stride(1), seq.data_ptr(), out1.data_ptr(), out1.stride(0), D)
    tail = (code, B, hq, hkv, D, L, D ** -0.5, ws.data_ptr(), ws.numel(), stream)
    if quant:
        rc = nat.lib().tq_decode_attention_quant(*args, qo1.data_ptr(), qo1.stride(0), sx1.data_ptr(), *tail)
    else:
        rc = nat.lib().tq_decode_attention(*args, *tail)
    assert rc == 0
    # one split pass
    kc2, vc2 = kc0.clone(), vc0.clone()
    out2, qo2, sx2 = outputs()
    rc = nat.lib().tq_decode_attention_rope(
        qkv.data_ptr(), qkv.stride(0), cos_t.data_ptr(), sin_t.data_ptr(), position.data_ptr(), kc2.data_ptr(),
        vc2.data_ptr(), kc2.stride(0), kc2.stride(2), kc2.stride(1), seq.data_ptr(), out2.data_ptr(), out2.stride(0),
        D, qo2.data_ptr() if quant else None, qo2.stride(0), sx2.data_ptr() if quant else None, code, B, hq, hkv, D,
        L, D ** -0.5, ws.data_ptr(), ws.numel(), None, stream)
    assert rc == 0
    torch.cuda.synchronize()
    assert torch.equal(out2, out1)
    assert torch.equal(qo2, qo1) and torch.equal(sx2, sx1)
    assert torch.equal(kc2, kc1) and torch.equal(vc2, vc1)
    if pos < L:
        assert not torch.equal(kc2[:, :, pos], kc0[:, :, pos])


@pytest.mark.parametrize("B,V,dtype", [(4, 128256, torch.bfloat16), (1, 1000, torch.float16), (16, 40001, torch.bfloat16),
                                       (3, 77, torch.bfloat16)])
def test_greedy_step_matches_torch_argmax_and_bookkeeping(B, V, dtype):
    """tq_greedy_step: torch.argmax results (planted ties, a NaN row, an
    all -inf row), token feedback, the generated column, the position and
    seq_used updates; a position past the generated buffer writes no column."""
    g = torch.Generator().manual_seed(V + B)
    logits = (torch.randn((B, 1, V), generator=g) * 4).to(dtype).to(DEV)
    if B > 2:
        logits[0, 0, 5] = logits[0, 0, V - 3] = 1000.0          # tie: the lower index wins
        logits[1, 0, V // 2] = float("nan")                       # NaN beats every number
        logits[1, 0, V // 3] = float("nan")
        logits[2] = float("-inf")                                 # all -inf: index 0
    prompt, gen_len = 50, 8
    ws = torch.empty((nat.lib().tq_greedy_step_workspace_elems(B),), dtype=torch.int32, device=DEV)
    for step, pos0 in enumerate([prompt, prompt + 3, prompt + gen_len + 2]):
        nxt = torch.full((B, 1), -1, dtype=torch.long, device=DEV)
        tok = torch.full((B, 1), -1, dtype=torch.long, device=DEV)
        gen = torch.zeros((B, gen_len), dtype=torch.long, device=DEV)
        position = torch.tensor([pos0], dtype=torch.long, device=DEV)
        seq = torch.zeros((B,), dtype=torch.int32, device=DEV)
        lg = logits.view(B, V)
        rc = nat.lib().tq_greedy_step(lg.data_ptr(), lg.stride(0), nat.dtype_code(dtype), B, V, ws.data_ptr(),
                                      ws.numel(), nxt.data_ptr(), tok.data_ptr(), gen.data_ptr(), gen.stride(0),
                                      gen_len, position.data_ptr(), prompt, seq.data_ptr(),
                                      torch.cuda.current_stream().cuda_stream)
        assert rc == 0
        torch.cuda.synchronize()
        ref = logits.argmax(dim=-1)
        assert torch.equal(nxt, ref) and torch.equal(tok, ref)
        col = pos0 - prompt + 1
        exp_gen = torch.zeros_like(gen)
        if 0 <= col < gen_len:
            exp_gen[:, col] = ref[:, 0]
        assert torch.equal(gen, exp_gen)
        assert int(position) == pos0 + 1 and torch.all(seq == pos0 + 2)
    if B > 2:
        assert int(nxt[0, 0]) == 5 and int(nxt[2, 0]) == 0 and int(nxt[1, 0]) == V // 3


def test_rotary_tables_equal_per_position_values():
    """The fused step's RoPE tables (the model's rotary module over all cache
    positions at once) equal its one-position outputs bit for bit."""
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding
    from transformers import LlamaConfig

    cfg = LlamaConfig(hidden_size=3072, num_attention_heads=24, num_key_value_heads=8, max_position_embeddings=131072,
                      rope_theta=500000.0, rope_scaling={"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0,
                                                         "high_freq_factor": 4.0,
                                                         "original_max_position_embeddings": 8192})
    rot = LlamaRotaryEmbedding(cfg).to(DEV)
    L = 2304
    x = torch.empty((1, 1, 1), dtype=torch.bfloat16, device=DEV)
    cos_t, sin_t = rot(x, torch.arange(L, device=DEV).view(1, -1))
    for p in (0, 1, 127, 2047, 2303):
        c, s_ = rot(x, torch.tensor([[p]], device=DEV))
        assert torch.equal(c.reshape(-1), cos_t[0, p]) and torch.equal(s_.reshape(-1), sin_t[0, p]), p


@pytest.mark.parametrize("family,dtype", [("llama", torch.bfloat16), ("qwen", torch.bfloat16),
                                          ("llama", torch.float16), ("qwen", torch.float16)])
def test_fused_decode_step_matches_module_forward(family, dtype):
    """The fused one-token step against the model's own forward in the same
    captured decoder (fused_decode=False): same tokens fed, logits within
    16-bit rounding noise, argmax equal wherever the margin is clear; bf16 and
    fp16 models (every fused kernel's fp16 instantiation end to end)."""
    from tilequant_amd.graph_decode import CudaGraphGreedyDecoder

    config = tiny_llama_config(layers=2) if family == "llama" else tiny_qwen2_config(layers=2)
    out = "bf16" if dtype == torch.bfloat16 else "fp16"
    model, _ = api.build_mixed_precision_model(config, ApplyConfig(model_type=family, dtype_out=out), DEV,
                                               torch_dtype=dtype, keep_frac=0.05, seed=31)
    B, P, O = 4, 80, 10
    prompt = torch.randint(0, config.vocab_size, (B, P), generator=torch.Generator().manual_seed(32))
    dec = CudaGraphGreedyDecoder.prepare(model, prompt_tokens=P, max_new_tokens=O, batch_size=B, device=DEV)
    assert dec._fused is not None
    dec.prefill(prompt)
    steps = []
    for _ in range(O - 1):
        dec._graph.replay()
        steps.append((dec._decode_logits[:, -1].float().clone(), dec._token.clone()))
    ids_fused = dec._generated.clone()
    dec.close()
    ref = CudaGraphGreedyDecoder.prepare(model, prompt_tokens=P, max_new_tokens=O, batch_size=B, device=DEV,
                                         fused_decode=False)
    assert ref._fused is None
    ref.prefill(prompt)
    # feed the fused run's tokens to the module path and compare logits step by step
    for t in range(O - 1):
        with torch.inference_mode():
            ref._token.copy_(ids_fused[:, t:t + 1])
        ref._graph.replay()
        r = ref._decode_logits[:, -1].float()
        f = steps[t][0]
        scale = float(r.abs().max())
        assert float((f - r).abs().max()) <= 3e-2 * scale, t
        top2 = r.topk(2, dim=-1).values
        clear = (top2[:, 0] - top2[:, 1]) > 3e-2 * scale
        assert torch.equal(f.argmax(-1)[clear], r.argmax(-1)[clear]), t
    ref.close()


@pytest.mark.parametrize("family,dtype", [("llama", torch.bfloat16), ("qwen", torch.bfloat16),
                                          ("llama", torch.float16)])
def test_fused_prefill_matches_module_prefill(family, dtype):
    """The decoder's fused prompt forward against the model's own forward
    (fused_prefill=False): last-token logits within 16-bit rounding noise,
    argmax equal where the margin is clear, the caches' prompt k/v close, and
    the tokens decoded after either prefill agree where the margins are clear;
    bf16 models and an fp16 one."""
    from tilequant_amd.graph_decode import CudaGraphGreedyDecoder

    config = tiny_llama_config(layers=2) if family == "llama" else tiny_qwen2_config(layers=2)
    out = "bf16" if dtype == torch.bfloat16 else "fp16"
    model, _ = api.build_mixed_precision_model(config, ApplyConfig(model_type=family, dtype_out=out), DEV,
                                               torch_dtype=dtype, keep_frac=0.05, seed=41)
    B, P, O = 3, 100, 6
    prompt = torch.randint(0, config.vocab_size, (B, P), generator=torch.Generator().manual_seed(42))
    runs = {}
    for fused in (True, False):
        dec = CudaGraphGreedyDecoder.prepare(model, prompt_tokens=P, max_new_tokens=O, batch_size=B, device=DEV,
                                             fused_prefill=fused)
        assert (dec._fused_prefill is not None) == fused
        dec.prefill(prompt)
        logits = dec.last_logits[:, -1].float().clone()
        kv = [(l.keys[:, :, :P].float().clone(), l.values[:, :, :P].float().clone()) for l in dec.cache.layers]
        assert all(int(l.cumulative_length) == P for l in dec.cache.layers)
        replay = dec.prefill(prompt).clone()                 # the captured prefill replays the same
        ids = dec.decode(O - 1).clone()
        dec.close()
        runs[fused] = (logits, kv, ids, replay)
    (lf, kvf, idf, rf), (lm, kvm, idm, rm) = runs[True], runs[False]
    scale = float(lm.abs().max())
    assert float((lf - lm).abs().max()) <= 3e-2 * scale
    top2 = lm.topk(2, dim=-1).values
    clear = (top2[:, 0] - top2[:, 1]) > 3e-2 * scale
    assert torch.equal(lf.argmax(-1)[clear], lm.argmax(-1)[clear])
    for (kf, vf), (km, vm) in zip(kvf, kvm):
        for a, b in ((kf, km), (vf, vm)):
            assert float((a - b).abs().max()) <= 3e-2 * float(b.abs().max())
    assert torch.equal(rf, idf[:, :1]) and torch.equal(rm, idm[:, :1])


@pytest.mark.parametrize("keep,blocks", [(0.05, 8), (0.05, 1024), (0.0, 64)])
def test_l2_warm_leaves_producers_bitwise_unchanged(keep, blocks):
    """The warm-up workgroups a producer runs for the next GEMM (tq_l2_warm)
    only read that GEMM's tiles: the norm, SiLU * up and attention outputs,
    codes, scales and cache contents are bitwise those of the launch without
    them; the fewest (8) and the most (1024) warm-up workgroups, with and
    without 16-bit tiles."""
    import ctypes

    from tilequant_amd.fused_decode import l2_warm_descriptor
    from tilequant_amd.mixed_linear import MixedLinear
    from tilequant_amd.pack import pack_weight_from_tile_ids
    from types import SimpleNamespace

    n_tr, n_tc = 80, 48
    g = torch.Generator().manual_seed(71)
    W = (torch.randn((n_tr * 64, n_tc * 64), generator=g) * 0.02).to(torch.bfloat16)
    ids16 = torch.randperm(n_tr * n_tc, generator=g)[:int(keep * n_tr * n_tc)].sort().values
    mask = torch.zeros(n_tr * n_tc, dtype=torch.bool)
    mask[ids16] = True
    pack = pack_weight_from_tile_ids(W.to(DEV), n_tr=n_tr, n_tc=n_tc, int8_tile_ids=torch.nonzero(~mask).flatten(),
                                     fp16_tile_ids=ids16, cfg=SimpleNamespace(quant_style="gi", dtype_out="bf16"))
    lin = MixedLinear(pack, None, SimpleNamespace(quant_style="gi", dtype_out="bf16"))
    warm = l2_warm_descriptor(lin, 4)
    assert warm is not None and (warm.fp16_tiles is None) == (keep == 0.0)
    warm.blocks = blocks
    stream = torch.cuda.current_stream().cuda_stream
    n, k, inter = 4, 3072, 8192
    x = (torch.randn((n, k), generator=g) * 3).to(torch.bfloat16).to(DEV)
    d = (torch.randn((n, k), generator=g) * 2).to(torch.bfloat16).to(DEV)
    wn = (1 + 0.1 * torch.randn(k, generator=g)).to(torch.bfloat16).to(DEV)
    gu = (torch.randn((n, 2 * inter), generator=g) * 2).to(torch.bfloat16).to(DEV)

    def norm(wd):
        h, y = torch.empty_like(x), torch.empty_like(x)
        q, sx = torch.empty((n, k), dtype=torch.int8, device=DEV), torch.empty((k // 64,), device=DEV)
        assert nat.lib().tq_add_rmsnorm_quant(x.data_ptr(), k, d.data_ptr(), k, wn.data_ptr(), 1e-5, h.data_ptr(), k,
                                              y.data_ptr(), k, q.data_ptr(), k, sx.data_ptr(), 0, n, k, wd,
                                              stream) == 0
        return h, y, q, sx

    def silu(wd):
        y = torch.empty((n, inter), dtype=torch.bfloat16, device=DEV)
        q, sx = torch.empty((n, inter), dtype=torch.int8, device=DEV), torch.empty((inter // 64,), device=DEV)
        assert nat.lib().tq_silu_mul_quant(gu.data_ptr(), 2 * inter, y.data_ptr(), inter, q.data_ptr(), inter,
                                           sx.data_ptr(), 0, n, inter, wd, stream) == 0
        return y, q, sx

    B, hq, hkv, D, L = 4, 24, 8, 128, 700
    qkv = torch.randn((B, (hq + 2 * hkv) * D), generator=g).to(torch.bfloat16).to(DEV)
    kc0 = torch.randn((B, hkv, L, D), generator=g).to(torch.bfloat16).to(DEV)
    vc0 = torch.randn((B, hkv, L, D), generator=g).to(torch.bfloat16).to(DEV)
    cos_t = torch.randn((L, D), generator=g).to(torch.bfloat16).to(DEV)
    sin_t = torch.randn((L, D), generator=g).to(torch.bfloat16).to(DEV)
    position = torch.tensor([411], dtype=torch.int64, device=DEV)
    seq = torch.full((B,), 412, dtype=torch.int32, device=DEV)
    ws = decode_attention_workspace(B, hq, L, DEV)

    def attention(wd, quant):
        kc, vc = kc0.clone(), vc0.clone()
        out = torch.empty((B, hq * D), dtype=torch.bfloat16, device=DEV)
        qo = torch.empty((B, hq * D), dtype=torch.int8, device=DEV)
        sx = torch.empty((hq * D // 64,), device=DEV)
        assert nat.lib().tq_decode_attention_rope(
            qkv.data_ptr(), qkv.stride(0), cos_t.data_ptr(), sin_t.data_ptr(), position.data_ptr(), kc.data_ptr(),
            vc.data_ptr(), kc.stride(0), kc.stride(2), kc.stride(1), seq.data_ptr(), out.data_ptr(), out.stride(0), D,
            qo.data_ptr() if quant else None, qo.stride(0), sx.data_ptr() if quant else None, 0, B, hq, hkv, D, L,
            D ** -0.5, ws.data_ptr(), ws.numel(), wd, stream) == 0
        return (out, qo, sx, kc, vc) if quant else (out, kc, vc)

    for fn in (norm, silu, lambda wd: attention(wd, True), lambda wd: attention(wd, False)):
        plain = fn(None)
        warmed = fn(ctypes.byref(warm))
        torch.cuda.synchronize()
        for a, b in zip(plain, warmed):
            assert torch.equal(a, b)


def test_fused_decode_step_with_every_gemm_warmed_gives_the_same_logits(monkeypatch):
    """Every producer warming its GEMM's weights (not only the default QKV)
    leaves each decode step's logits and tokens bitwise unchanged."""
    import tilequant_amd.fused_decode as fd
    from tilequant_amd.graph_decode import CudaGraphGreedyDecoder

    monkeypatch.setattr(fd, "WARM_GEMMS", ("qkv", "o", "gate_up", "down"))
    config = tiny_llama_config(layers=2)
    model, _ = api.build_mixed_precision_model(config, ApplyConfig(model_type="llama", dtype_out="bf16"), DEV,
                                               keep_frac=0.05, seed=41)
    B, P, O = 4, 64, 8
    prompt = torch.randint(0, config.vocab_size, (B, P), generator=torch.Generator().manual_seed(42))
    runs = {}
    for warm in (False, True):
        dec = CudaGraphGreedyDecoder.prepare(model, prompt_tokens=P, max_new_tokens=O, batch_size=B, device=DEV,
                                             l2_warm=warm)
        n_desc = sum(v is not None for ly in dec._fused.layers for v in ly.warm.values())
        assert n_desc == (8 if warm else 0)
        dec.prefill(prompt)
        logits = []
        for _ in range(O - 1):
            dec._graph.replay()
            logits.append(dec._decode_logits.clone())
        runs[warm] = (torch.stack(logits), dec._generated.clone())
        dec.close()
    assert torch.equal(runs[False][0], runs[True][0])
    assert torch.equal(runs[False][1], runs[True][1])
