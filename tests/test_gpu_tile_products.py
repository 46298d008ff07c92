"""GPU parity of the exact INT32 tile products from EVERY production GEMM kernel.

The north_star's bit-exact contract is on the INT32 tile partial sums
P_t[n, j] = sum_k q[n, 64c + k] * wq_t[j, k] (the reference's tl.dot of the
int8 operands, src/kernels/triton/gemm_rows_splitk_64x64.py:125-137).  Each
test below runs the DUMP instantiation of the very kernel the automatic
schedule picks for its arguments (gemm_mixed_rows_products_i32, which reports
the kernel family that ran): the raw v_mfma_i32_16x16x64_i8 result of every
INT8 tile, before its scale FMA, is compared with the oracle's integer
products of the oracle's codes (oracle/tq_oracle.c: int64-free int32 sums,
pinned by brute force and linearity in test_oracle.py).  Positions the kernel
never reached keep the fill value -2^31 and fail the comparison, so a dropped
tile is caught as well as a wrong one.  The DUMP launch's outputs must equal
the production launch's outputs bitwise (same instruction stream plus stores).

Coverage:
* 3072 x 3072, 16 tokens, keep01 -- LDS-staged decode kernel,
  split-K kernel (explicit split_k, row-major and token-blocked codes), and
  both one-launch quantize+GEMM kernels (codes computed in the kernel).
* the Llama-3.2-3B stacked Q/K/V, O, stacked Gate/Up and Down at
  1 / 4 / 16 / 64 tokens, row-major and token-blocked codes, one-launch where
  it applies.
* the same projections at 8192 tokens, keep05 (prefill v5), three
  16-row windows, with and without a work plan (released keep05 Down map).
* Qwen2.5-7B Down and Qwen2.5-14B stacked Q/K/V with clustered
  keep10 / keep20 masks, 4 and 8192 tokens.
* the wide-K prefill kernels (v3 for K > 19456, the async ring for
  K > 32768) and the register prefill kernel (K % 64 != 0).
"""
from __future__ import annotations

from pathlib import Path
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from helpers import clustered_weight, complement, make_w, make_x, oracle_pack, uniform_fp16_ids, values
from oracle import native as onat
from oracle import numerics as nm
from oracle import packing as opk
from tilequant_amd.gemm_rows_splitk_64x64 import (fused_max_tokens, gemm_mixed_rows_products_i32,
                                                 gemm_mixed_rows_splitk, linear_mixed_fused, prefill_plan)
from tilequant_amd.mask_io import load_fp16_keep_ids_for_layer
from tilequant_amd.pack import concat_packs_along_rows, pack_weight_from_tile_ids
from tilequant_amd.quant_utils import quantize_activation_tile_absmax
from tilequant_amd.quantize_activation import quantize_activation_token_blocked

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
CFG = SimpleNamespace(quant_style="gi", dtype_out="bf16")
GOLDEN = Path(__file__).resolve().parent / "golden"

LLAMA = {
    "qkv": [(3072, 3072), (1024, 3072), (1024, 3072)],
    "o": [(3072, 3072)],
    "gate_up": [(8192, 3072), (8192, 3072)],
    "down": [(3072, 8192)],
}


def _pack_one(W, ids16):
    n_tr, n_tc = -(-W.shape[0] // 64), -(-W.shape[1] // 64)
    ids8 = complement(ids16, n_tr * n_tc)
    return pack_weight_from_tile_ids(W.to(DEV), n_tr=n_tr, n_tc=n_tc, int8_tile_ids=torch.from_numpy(ids8),
                                     fp16_tile_ids=torch.from_numpy(np.asarray(ids16, np.int64)), cfg=CFG,
                                     tile_layout="mfma")


def _stacked(members, frac, seed, clustered=False):
    """Device pack and oracle pack of members stacked along the output rows
    (as MixedLinearGroup stacks Q/K/V and Gate/Up)."""
    packs, ops = [], []
    for i, (m, k) in enumerate(members):
        if clustered:
            W, ids16 = clustered_weight(m, k, frac, seed=seed + i)
        else:
            W = make_w(m, k, seed=seed + i)
            ids16 = uniform_fp16_ids(m // 64, -(-k // 64), frac, seed=seed + 100 + i)
        packs.append(_pack_one(W, ids16))
        ops.append(oracle_pack(W, ids16))
    if len(packs) == 1:
        return packs[0], ops[0]
    return concat_packs_along_rows(packs), opk.concat_rows(ops)


def _wkw(pack):
    return dict(int8_tiles=pack.int8_tiles, int8_scales=pack.int8_scales, int8_tile_ids=pack.int8_tile_ids,
                int8_row_ptr=pack.int8_row_ptr, fp16_tiles=pack.fp16_tiles, fp16_tile_ids=pack.fp16_tile_ids,
                fp16_row_ptr=pack.fp16_row_ptr, M=pack.M_orig, K=pack.K_orig, n_tr=pack.n_tr, n_tc=pack.n_tc,
                out_dtype=torch.bfloat16, tile_layout=pack.tile_layout)


def _oracle_products(op, xq_rows):
    return onat.tile_products_i32(xq_rows, op.int8_tiles, op.int8_tile_ids, op.n_tc, K=op.K_orig)


def _assert_products(P, ref, what):
    got = P.cpu().numpy()
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    bad = got != ref
    assert not bad.any(), (f"{what}: {int(bad.any(axis=(1, 2)).sum())} of {ref.shape[0]} INT8 tiles differ "
                           f"(first at position {int(np.argmax(bad.any(axis=(1, 2))))})")


def _run_codes(pack, xd, xq, sx, rows=None, layout="row_major", **extra):
    """DUMP launch on given codes + the production launch; outputs bitwise equal."""
    kw = dict(_wkw(pack), x_fp=xd, x_int8=xq, sx=sx, x_int8_layout=layout, **extra)
    y_dump, P, kern = gemm_mixed_rows_products_i32(rows=rows, **kw)
    y = gemm_mixed_rows_splitk(**kw)
    assert torch.equal(y_dump, y), f"{kern}: the DUMP launch changed the outputs"
    return P, kern


def _run_fused(pack, xd, rows=None, **extra):
    kw = dict(_wkw(pack), x_fp=xd, **extra)
    y_dump, P, kern = gemm_mixed_rows_products_i32(rows=rows, fused=True, **kw)
    y = linear_mixed_fused(**kw)
    assert torch.equal(y_dump, y), f"{kern}: the DUMP launch changed the outputs"
    return P, kern


# ---- configs[0] -------------------------------------------------------------------------------

def test_config0_products_every_decode_kernel():
    """3072 -> 3072, 16 tokens, keep01 uniform, outlier activations: every
    decode-size kernel family writes the oracle's products."""
    pack, op = _stacked([(3072, 3072)], 0.01, seed=100)
    x = make_x(16, 3072, seed=101)
    xd = x.to(DEV)
    xq, sx = quantize_activation_tile_absmax(xd)
    xq_ref, sx_ref = nm.act_quant(values(x))
    assert np.array_equal(xq.cpu().numpy(), xq_ref)
    ref = _oracle_products(op, xq_ref)
    seen = set()
    P, kern = _run_codes(pack, xd, xq, sx)
    _assert_products(P, ref, kern)
    seen.add(kern)
    for sk in (2, 3):
        P, kern = _run_codes(pack, xd, xq, sx, split_k=sk)
        _assert_products(P, ref, f"{kern} split_k={sk}")
        seen.add(kern)
    xqb, sxb = quantize_activation_token_blocked(xd)
    P, kern = _run_codes(pack, xd, xqb, sxb, layout="token_blocked")
    _assert_products(P, ref, kern)
    seen.add(kern)
    P, kern = _run_fused(pack, xd)
    _assert_products(P, ref, kern)
    seen.add(kern)
    P, kern = _run_fused(pack, xd, split_k=2)
    _assert_products(P, ref, f"{kern} split_k=2")
    seen.add(kern)
    # at 16 rows the one-launch path is the cooperative kernel (16 rows x 3072
    # columns exceed the LDS-staged kernel's 4 chunks per thread, so producer
    # workgroups quantize into the workspace); 4 rows take the LDS-staged
    # quantizing kernel, with scales over those 4 rows
    x4 = x[:4].contiguous()
    xq4_ref, _ = nm.act_quant(values(x4))
    P, kern = _run_fused(pack, x4.to(DEV))
    _assert_products(P, _oracle_products(op, xq4_ref), f"{kern} n=4")
    seen.add(kern)
    # a window of rows: only those rows are written
    P, kern = _run_codes(pack, xd, xq, sx, rows=(5, 7))
    _assert_products(P, ref[:, 5:12], f"{kern} rows 5..11")
    assert seen == {"decode", "splitk", "splitk_token_blocked", "decode_quant", "splitk_quant",
                    "decode_coop"}, seen


# ---- configs[1] -------------------------------------------------------------------------------

@pytest.mark.parametrize("proj", sorted(LLAMA))
def test_llama_decode_products_all_token_counts(proj):
    """Each Llama-3.2-3B projection group at 1 / 4 / 16 / 24 / 64 tokens,
    keep01: the kernel the schedule picks on row-major codes, on token-blocked
    codes, and the one-launch kernel where the row count allows it (24 rows:
    the stacked Gate/Up runs half-tile split-K workgroups)."""
    members = LLAMA[proj]
    k = members[0][1]
    pack, op = _stacked(members, 0.01, seed=sum(m for m, _ in members) + k)
    seen = set()
    for n in (1, 4, 16, 24, 64):
        x = make_x(n, k, seed=k + n)
        xd = x.to(DEV)
        xq_ref, _ = nm.act_quant(values(x))
        ref = _oracle_products(op, xq_ref)
        xq, sx = quantize_activation_tile_absmax(xd)
        P, kern = _run_codes(pack, xd, xq, sx)
        _assert_products(P, ref, f"{proj} n={n} {kern}")
        seen.add(kern)
        if n == 64:
            assert kern == "splitk"
        xqb, sxb = quantize_activation_token_blocked(xd)
        P, kern = _run_codes(pack, xd, xqb, sxb, layout="token_blocked")
        assert kern == "splitk_token_blocked"
        _assert_products(P, ref, f"{proj} n={n} {kern}")
        if n <= fused_max_tokens(k):
            P, kern = _run_fused(pack, xd)
            _assert_products(P, ref, f"{proj} n={n} {kern}")
            seen.add(kern)
    assert "splitk" in seen and seen & {"decode", "decode_quant"}, seen


# ---- configs[2] -------------------------------------------------------------------------------

def _windows(n):
    return [(0, 16), (n // 2 + 100, 16), (n - 16, 16)]


def _prefill_products(pack, op, x, plan=None):
    xd = x.to(DEV)
    xq, sx = quantize_activation_tile_absmax(xd)
    sx_ref = onat.act_scales(values(x))
    assert np.array_equal(sx.cpu().numpy().view(np.uint32), sx_ref.view(np.uint32))
    kinds = set()
    for r0, cnt in _windows(x.shape[0]):
        xq_rows = nm.act_quant_codes(values(x[r0:r0 + cnt]), sx_ref)
        P, kern = _run_codes(pack, xd, xq, sx, rows=(r0, cnt), prefill_plan=plan)
        _assert_products(P, _oracle_products(op, xq_rows), f"{kern} rows {r0}..{r0 + cnt - 1}")
        kinds.add(kern)
    return kinds


@pytest.mark.parametrize("proj", sorted(LLAMA))
def test_llama_prefill_products_8192_tokens(proj):
    """Each Llama-3.2-3B projection group at 8192 tokens, keep05 uniform,
    scales over the whole input: prefill v5 products on three row windows."""
    members = LLAMA[proj]
    k = members[0][1]
    pack, op = _stacked(members, 0.05, seed=7 * k + len(members))
    x = make_x(8192, k, seed=k + 3)
    assert _prefill_products(pack, op, x) == {"prefill_v5"}


def test_prefill_products_with_work_plan_released_keep05_down():
    """Released Llama-3.2-3B gi keep05 map of layer 7's Down projection
    (row tile 47 holds 127 of 128 tiles in 16 bits): the work plan splits
    heavy pairs into single row tiles; products identical to the oracle with
    and without the plan."""
    keep = GOLDEN / "llama32_3b_gi_keep05"
    ids, shape = load_fp16_keep_ids_for_layer(keep, "model.layers.7.mlp.down_proj")
    assert tuple(shape) == (48, 128)
    ids16 = ids.numpy().astype(np.int64)
    assert np.bincount(ids16 // 128, minlength=48)[47] == 127
    W = make_w(3072, 8192, seed=5)
    pack, op = _pack_one(W, ids16), oracle_pack(W, ids16)
    plan = prefill_plan(int8_tile_ids=pack.int8_tile_ids, int8_row_ptr=pack.int8_row_ptr,
                        fp16_row_ptr=pack.fp16_row_ptr, n_tr=pack.n_tr, n_tc=pack.n_tc)
    assert plan is not None and plan.units.numel() > (pack.n_tr + 1) // 2
    x = make_x(8192, 8192, seed=6)
    assert _prefill_products(pack, op, x, plan=plan) == {"prefill_v5"}
    assert _prefill_products(pack, op, x) == {"prefill_v5"}


# ---- configs[3] -------------------------------------------------------------------------------

QWEN = {
    "qwen7b_down": [(3584, 18944)],
    "qwen14b_qkv": [(5120, 5120), (1024, 5120), (1024, 5120)],
}


@pytest.mark.parametrize("frac", [0.10, 0.20])
@pytest.mark.parametrize("proj", sorted(QWEN))
def test_qwen_clustered_products(proj, frac):
    """Qwen2.5-7B Down (3584 x 18944) and Qwen2.5-14B stacked Q/K/V
    (7168 x 5120) with top-k clustered BF16 tiles: products at 4 tokens (all
    rows) and at 8192 tokens (three windows)."""
    members = QWEN[proj]
    k = members[0][1]
    pack, op = _stacked(members, frac, seed=k + int(frac * 100), clustered=True)
    x = make_x(4, k, seed=k + 4)
    xd = x.to(DEV)
    xq, sx = quantize_activation_tile_absmax(xd)
    xq_ref, _ = nm.act_quant(values(x))
    P, kern = _run_codes(pack, xd, xq, sx)
    _assert_products(P, _oracle_products(op, xq_ref), f"{proj} n=4 {kern}")
    # the split-K kernel on token-blocked codes too: MixedLinear's choice for
    # rows of 256+ column tiles (Qwen2.5-7B Down) at every decode row count
    xqb, sxb = quantize_activation_token_blocked(xd)
    P, kern = _run_codes(pack, xd, xqb, sxb, layout="token_blocked")
    assert kern == "splitk_token_blocked"
    _assert_products(P, _oracle_products(op, xq_ref), f"{proj} n=4 {kern}")
    del x, xd, xq, xqb
    assert _prefill_products(pack, op, make_x(8192, k, seed=k + 8192)) == {"prefill_v5"}


# ---- the other prefill kernels ----------------------------------------------------------------

@pytest.mark.parametrize("k,family", [(20480, "prefill_v3"), (33280, "prefill_async")])
def test_wide_k_prefill_products(k, family):
    """K beyond the v5 kernel's column map: the v3 (K > 19456) and async
    (K > 32768) DMA-ring kernels, 300 tokens, 10% 16-bit tiles."""
    pack, op = _stacked([(192, k)], 0.10, seed=k)
    x = make_x(300, k, seed=k + 1)
    xd = x.to(DEV)
    xq, sx = quantize_activation_tile_absmax(xd)
    xq_ref, _ = nm.act_quant(values(x))
    P, kern = _run_codes(pack, xd, xq, sx)
    assert kern == family
    _assert_products(P, _oracle_products(op, xq_ref), kern)
    P, kern = _run_codes(pack, xd, xq, sx, rows=(256, 44))   # the second token block only
    _assert_products(P, _oracle_products(op, xq_ref[256:]), f"{kern} rows 256..299")


def test_dump_entry_rejects_bad_windows_and_fp16():
    pack, _ = _stacked([(128, 128)], 0.0, seed=3)
    x = make_x(8, 128, seed=4).to(DEV)
    xq, sx = quantize_activation_tile_absmax(x)
    kw = dict(_wkw(pack), x_fp=x, x_int8=xq, sx=sx)
    for rows in ((0, 0), (4, 5), (-1, 2)):
        with pytest.raises(ValueError):
            gemm_mixed_rows_products_i32(rows=rows, **kw)
    xh = x.to(torch.float16)
    packh = pack_weight_from_tile_ids(make_w(128, 128, seed=3, dtype=torch.float16).to(DEV), n_tr=2, n_tc=2,
                                      int8_tile_ids=torch.arange(4), fp16_tile_ids=torch.zeros(0, dtype=torch.long),
                                      cfg=CFG, tile_layout="mfma")
    xqh, sxh = quantize_activation_tile_absmax(xh)
    with pytest.raises(RuntimeError):
        gemm_mixed_rows_products_i32(**dict(_wkw(packh), x_fp=xh, x_int8=xqh, sx=sxh))
