"""Cooperative quantize + GEMM launches (linear_mixed_fused on shapes the
LDS-staged quantizing decode kernel cannot take): 8 producer workgroups
quantize the activation once into the per-stream workspace while the GEMM
workgroups' weight loads are in flight.  The codes are the closed form of the separate quantizer, so every
output must equal the two-launch sequence (quantize_activation_tile_absmax +
gemm_mixed_rows_splitk) bit for bit -- also when the GEMM workgroups are made
to quantize by themselves (poll budget 0), across back-to-back calls (the
counters reset themselves) and HIP-graph replays; and the INT32 tile products
of the cooperative kernel equal the oracle's."""
from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from helpers import make_w, make_x, oracle_pack, uniform_fp16_ids, values
from oracle import native as onat
from oracle import numerics as nm
from tilequant_amd import _native as nat
from tilequant_amd.gemm_rows_splitk_64x64 import (gemm_mixed_rows_products_i32, gemm_mixed_rows_splitk,
                                                  linear_mixed_fused)
from tilequant_amd.pack import pack_weight_from_tile_ids
from tilequant_amd.quant_utils import quantize_activation_tile_absmax

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
CFG = SimpleNamespace(quant_style="gi", dtype_out="bf16")


def _pack(n_tr, n_tc, frac, seed, dtype=torch.bfloat16):
    W = make_w(n_tr * 64, n_tc * 64, seed=seed).to(dtype)
    ids16 = uniform_fp16_ids(n_tr, n_tc, frac, seed=seed + 1)
    mask = np.zeros(n_tr * n_tc, bool)
    mask[ids16] = True
    pack = pack_weight_from_tile_ids(W.to(DEV), n_tr=n_tr, n_tc=n_tc,
                                     int8_tile_ids=torch.from_numpy(np.nonzero(~mask)[0]),
                                     fp16_tile_ids=torch.from_numpy(np.asarray(ids16, np.int64)), cfg=CFG,
                                     tile_layout="mfma")
    return W, ids16, pack


def _kw(pack, x, bias=None):
    return dict(x_fp=x, int8_tiles=pack.int8_tiles, int8_scales=pack.int8_scales, int8_tile_ids=pack.int8_tile_ids,
                int8_row_ptr=pack.int8_row_ptr, fp16_tiles=pack.fp16_tiles, fp16_tile_ids=pack.fp16_tile_ids,
                fp16_row_ptr=pack.fp16_row_ptr, M=pack.M_orig, K=pack.K_orig, n_tr=pack.n_tr, n_tc=pack.n_tc,
                out_dtype=torch.bfloat16, bias=bias, tile_layout=pack.tile_layout)


def _two_launch(pack, x, bias=None):
    xq, sx = quantize_activation_tile_absmax(x)
    kw = _kw(pack, x, bias)
    return gemm_mixed_rows_splitk(x_int8=xq, sx=sx, **kw)


CASES = [
    (256, 48, 4, torch.bfloat16, 0.01),    # Llama-3.2-3B stacked Gate/Up: 1024 units, 12-tile batches
    (592, 56, 4, torch.bfloat16, 0.10),    # Qwen2.5-7B stacked Gate/Up: 16-tile batches
    (432, 80, 8, torch.bfloat16, 0.10),    # Qwen2.5-14B stacked Gate/Up: 10 waves
    (80, 48, 8, torch.bfloat16, 0.02),     # Llama-3.2-3B stacked Q/K/V: 320 units
    (80, 48, 16, torch.bfloat16, 0.02),
    (48, 48, 12, torch.float16, 0.05),     # O: 192 units
    (72, 56, 8, torch.bfloat16, 0.20),     # Qwen2.5-7B stacked Q/K/V: 288 units, 7 waves
]


@pytest.mark.parametrize("n_tr,n_tc,n,dtype,frac", CASES)
def test_coop_launch_equals_two_launches_bitwise(n_tr, n_tc, n, dtype, frac):
    W, ids16, pack = _pack(n_tr, n_tc, frac, seed=n_tr + n_tc + n, dtype=dtype)
    x = make_x(n, n_tc * 64, seed=n + 7).to(dtype).to(DEV)
    bias = (torch.randn(pack.M_orig, generator=torch.Generator().manual_seed(3)) * 0.1).to(torch.bfloat16).to(DEV)
    ref = _two_launch(pack, x, bias)
    kw = _kw(pack, x, bias)
    if dtype == torch.bfloat16:
        y, prod, fam = gemm_mixed_rows_products_i32(fused=True, **kw)
        assert fam == "decode_coop"
        assert torch.equal(y, ref)
        # the INT32 products of the cooperative kernel: those of the two-launch kernel, bit for bit
        _, prod_ref, fam_ref = gemm_mixed_rows_products_i32(x_int8=quantize_activation_tile_absmax(x)[0],
                                                            sx=quantize_activation_tile_absmax(x)[1], **kw)
        assert fam_ref == "decode"
        assert torch.equal(prod, prod_ref)
    for _ in range(3):   # the counters reset themselves between calls
        assert torch.equal(linear_mixed_fused(**kw), ref)
    try:
        nat.lib().tq_test_set_coop_spin(0)    # no polling: every GEMM workgroup quantizes by itself
        assert torch.equal(linear_mixed_fused(**kw), ref)
    finally:
        nat.lib().tq_test_set_coop_spin(-1)
    assert torch.equal(linear_mixed_fused(**kw), ref)


def test_coop_products_against_the_oracle():
    """The cooperative kernel's INT32 products vs the oracle's exact integer
    products (Llama Q/K/V shape, 8 tokens)."""
    W, ids16, pack = _pack(80, 48, 0.02, seed=5)
    x_cpu = make_x(8, 3072, seed=6)
    x = x_cpu.to(DEV)
    _, prod, fam = gemm_mixed_rows_products_i32(fused=True, **_kw(pack, x))
    assert fam == "decode_coop"
    op = oracle_pack(W, ids16)
    xv = values(x_cpu)
    xq, sx = nm.act_quant(xv)
    ref = onat.tile_products_i32(xq, op.int8_tiles, op.int8_tile_ids, op.n_tc)
    assert np.array_equal(prod.cpu().numpy(), ref)


def test_coop_graph_replays_with_eager_work_between():
    W, ids16, pack = _pack(256, 48, 0.01, seed=9)
    x = make_x(4, 3072, seed=10).to(DEV)
    ref = _two_launch(pack, x)
    kw = _kw(pack, x)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        linear_mixed_fused(**kw)   # workspace allocated before capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        yg = linear_mixed_fused(**kw)
    for _ in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(yg, ref)
        assert torch.equal(linear_mixed_fused(**kw), ref)   # eager calls between replays


@pytest.mark.parametrize("n_tr,n,family", [(48, 4, "decode_quant"), (80, 4, "decode_quant"),
                                           (48, 1, "decode_quant_help"), (256, 2, "decode_quant")])
def test_shapes_the_quantizing_kernel_takes_keep_it(n_tr, n, family):
    """Where the LDS-staged quantizing kernel fits (O and Q/K/V up to 4 rows,
    Gate/Up up to 2), it runs -- with helper waves at 1-2 rows of 6-wave
    workgroups: no producers, no hand-off round trips."""
    _, _, pack = _pack(n_tr, 48, 0.02, seed=11 + n)
    x = make_x(n, 3072, seed=12 + n).to(DEV)
    y, _, fam = gemm_mixed_rows_products_i32(fused=True, **_kw(pack, x))
    assert fam == family
    assert torch.equal(y, _two_launch(pack, x))


def test_coop_and_split_k_launches_share_one_stream_workspace():
    """The cooperative launch's flags and counts sit in the split-K counter
    region of the same per-stream workspace; each kind of launch leaves that
    region zero, so alternating them on one stream changes no output."""
    _, _, pack_c = _pack(256, 48, 0.01, seed=61)        # Gate/Up shape: cooperative at 4 rows
    _, _, pack_s = _pack(48, 48, 0.02, seed=62)         # O shape: explicit split_k = 4
    x_c = make_x(4, 3072, seed=63).to(DEV)
    x_s = make_x(4, 3072, seed=64).to(DEV)
    ref_c = _two_launch(pack_c, x_c)
    xq, sx = quantize_activation_tile_absmax(x_s)
    ref_s = gemm_mixed_rows_splitk(x_int8=xq, sx=sx, split_k=4, **_kw(pack_s, x_s))
    kw_c = _kw(pack_c, x_c)
    for _ in range(3):
        _, _, fam = gemm_mixed_rows_products_i32(fused=True, **kw_c)
        assert fam == "decode_coop"
        assert torch.equal(linear_mixed_fused(**kw_c), ref_c)
        assert torch.equal(gemm_mixed_rows_splitk(x_int8=xq, sx=sx, split_k=4, **_kw(pack_s, x_s)), ref_s)
        assert torch.equal(linear_mixed_fused(split_k=4, **_kw(pack_s, x_s)), ref_s)
