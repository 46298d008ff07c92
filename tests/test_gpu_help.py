"""The one-launch quantize + GEMM with helper waves (linear_mixed_fused at 1-2
rows on 6- or 7-wave decode workgroups, and where neither the plain
quantizing kernel nor a cooperative launch applies): k / 512 extra waves
quantize by lanes while the tile waves issue their weights.  The tile waves
are the plain decode plan's, in the same order, so every output must equal
the two-launch sequence (quantize_activation_tile_absmax +
gemm_mixed_rows_splitk) bit for bit, and the INT32 tile products must equal
the oracle's."""
from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from helpers import make_w, make_x, oracle_pack, uniform_fp16_ids, values
from oracle import native as onat
from oracle import numerics as nm
from tilequant_amd import gemm_rows_splitk_64x64 as gm
from tilequant_amd.gemm_rows_splitk_64x64 import gemm_mixed_rows_products_i32, gemm_mixed_rows_splitk, linear_mixed_fused
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
    return gemm_mixed_rows_splitk(x_int8=xq, sx=sx, **_kw(pack, x, bias))


CASES = [
    (80, 48, 1, torch.bfloat16, 0.02),     # Llama-3.2-3B stacked Q/K/V: 6 tile + 6 helper waves
    (48, 48, 1, torch.bfloat16, 0.02),     # O
    (48, 48, 2, torch.float16, 0.05),
    (80, 48, 2, torch.bfloat16, 0.30),     # many 16-bit tiles
    (56, 56, 1, torch.bfloat16, 0.10),     # Qwen2.5-7B O: 7 + 7 waves
]


@pytest.mark.parametrize("n_tr,n_tc,n,dtype,frac", CASES)
def test_helper_waves_equal_two_launches_bitwise(n_tr, n_tc, n, dtype, frac):
    W, ids16, pack = _pack(n_tr, n_tc, frac, seed=n_tr + n_tc + n, dtype=dtype)
    x = make_x(n, n_tc * 64, seed=n + 3).to(dtype).to(DEV)
    bias = (torch.randn(pack.M_orig, generator=torch.Generator().manual_seed(4)) * 0.1).to(torch.bfloat16).to(DEV)
    ref = _two_launch(pack, x, bias)
    kw = _kw(pack, x, bias)
    if dtype == torch.bfloat16:
        # the DUMP instantiation needs more registers: on grids beyond one
        # workgroup per CU (Q/K/V) it may fall back to the plain kernel
        y, _, fam = gemm_mixed_rows_products_i32(fused=True, **kw)
        assert fam == "decode_quant_help" or (4 * n_tr > 256 and fam == "decode_quant")
        assert torch.equal(y, ref)
    for _ in range(3):   # repeated calls: nothing carried over between launches
        assert torch.equal(linear_mixed_fused(**kw), ref)


def test_helper_waves_products_against_the_oracle():
    """The helper-wave kernel's INT32 products vs the oracle's exact integer
    products (Llama O shape, one token)."""
    W, ids16, pack = _pack(48, 48, 0.02, seed=21)
    x_cpu = make_x(1, 3072, seed=22)
    _, prod, fam = gemm_mixed_rows_products_i32(fused=True, **_kw(pack, x_cpu.to(DEV)))
    assert fam == "decode_quant_help"
    op = oracle_pack(W, ids16)
    xq, _ = nm.act_quant(values(x_cpu))
    assert np.array_equal(prod.cpu().numpy(), onat.tile_products_i32(xq, op.int8_tiles, op.int8_tile_ids, op.n_tc))


@pytest.mark.parametrize("n_tr,n", [(80, 8), (48, 8)])
def test_without_a_workspace_oversized_shapes_take_the_helpers(monkeypatch, n_tr, n):
    """8 rows of a 3072-wide input do not fit the plain quantizing kernel; with
    no workspace for a cooperative launch the helper waves take them (instead
    of the quantizing split-K kernel), bitwise the two launches."""
    W, ids16, pack = _pack(n_tr, 48, 0.02, seed=31 + n_tr)
    x = make_x(n, 3072, seed=32).to(DEV)
    ref = _two_launch(pack, x)
    monkeypatch.setattr(gm, "_fused_workspace", lambda *a: (None, 0))
    y, _, fam = gemm_mixed_rows_products_i32(fused=True, **_kw(pack, x))
    assert fam == "decode_quant_help" or (4 * n_tr > 256 and fam == "splitk_quant")
    assert torch.equal(y, ref)
    assert torch.equal(linear_mixed_fused(**_kw(pack, x)), ref)


def test_four_rows_keep_the_plain_quantizing_kernel():
    _, _, pack = _pack(48, 48, 0.02, seed=41)
    x = make_x(4, 3072, seed=42).to(DEV)
    y, _, fam = gemm_mixed_rows_products_i32(fused=True, **_kw(pack, x))
    assert fam == "decode_quant"
    assert torch.equal(y, _two_launch(pack, x))


def test_grids_that_need_two_rounds_fall_back_to_the_plain_kernel():
    """Qwen2.5-7B stacked Q/K/V at one row: 288 workgroups of 7 + 7 waves need
    two per CU on some CUs; where the registers do not allow that the launch
    takes the plain quantizing kernel.  Either way the outputs are the two
    launches', bit for bit."""
    _, _, pack = _pack(72, 56, 0.10, seed=51)
    x = make_x(1, 3584, seed=52).to(DEV)
    y, _, fam = gemm_mixed_rows_products_i32(fused=True, **_kw(pack, x))
    assert fam in ("decode_quant_help", "decode_quant")
    assert torch.equal(y, _two_launch(pack, x))
