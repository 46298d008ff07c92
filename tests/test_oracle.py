"""Pins the CPU oracle (tests only; no GPU).

Each oracle function is checked against something that does not restate it:
torch-CPU ops in the reference's own CPU branch (quant_utils.py:61-74,
103-115; pack.py:119-167), exhaustive sweeps over bf16/fp16 values, closed
forms and invariants, brute force on tiny inputs, and the reference's released
Decision/ maps.  Planted mistakes (in the oracle, on the CPU) must fail the
same checks.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from helpers import bits, complement, make_w, make_x, oracle_pack, uniform_fp16_ids, values
from oracle import masks as om
from oracle import native as onat
from oracle import numerics as nm
from oracle import packing as opk

ALL_POS_BF16 = np.arange(1, 0x7F80, dtype=np.uint16)          # every positive finite bf16
ALL_POS_FP16 = np.arange(1, 0x7C00, dtype=np.uint16)          # every positive finite fp16


def _torch_bf16(b: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(b.astype(np.uint16).view(np.int16)).view(torch.bfloat16)


# --------------------------------------------------------------------------
# activation scales
# --------------------------------------------------------------------------

def test_act_scale_exhaustive_bf16_vs_torch_cpu():
    a = nm.bf16_bits_to_f32(ALL_POS_BF16)
    # reference CPU branch: bf16 absmax / 127 in bf16, widened (quant_utils.py:68-74)
    ref = (_torch_bf16(ALL_POS_BF16) / 127.0).to(torch.float32).numpy()
    got = nm.round_to_dtype(a / np.float32(127.0), True)
    assert np.array_equal(got, ref)
    # the C restatement agrees on every value
    lib = onat.lib()
    c = np.array([lib.tqo_round_to_dtype(float(v), 1) for v in (a / np.float32(127.0))], np.float32)
    assert np.array_equal(c, ref)


def test_act_scale_exhaustive_fp16_vs_torch_cpu():
    h = ALL_POS_FP16.view(np.float16)
    ref = (torch.from_numpy(h.copy()) / 127.0).to(torch.float32).numpy()
    got = nm.round_to_dtype(h.astype(np.float32) / np.float32(127.0), False)
    assert np.array_equal(got, ref)
    lib = onat.lib()
    c = np.array([lib.tqo_round_to_dtype(float(v), 0) for v in (h.astype(np.float32) / np.float32(127.0))], np.float32)
    assert np.array_equal(c, ref)


def test_absmax_element_maps_to_127_when_scale_is_normal():
    # closed-form invariant: for every bf16 absmax whose scale is a normal
    # number, the absmax element itself quantizes to exactly 127
    a = nm.bf16_bits_to_f32(ALL_POS_BF16)
    s = nm.round_to_dtype(a / np.float32(127.0), True)
    normal = s >= np.float32(2.0 ** -126)
    q = nm.quant_codes(a, s)
    assert np.all(q[normal] == 127)
    quot = (a[normal].astype(np.float64) / s[normal])
    assert quot.min() > 126.5 and quot.max() < 127.5


def test_zero_scale_region_matches_reference_kernel_clamp_order():
    # absmax below 127 * 2^-134 rounds to a zero bf16 scale; codes then come
    # from x/0: +x -> 127, -x -> -127 and 0/0 = NaN -> 127 through the
    # reference kernel's NaN-ignoring min-then-max (quantize_activation.py:71)
    tiny = np.float32(2.0 ** -133)
    x = np.zeros((2, 64), np.float32)
    x[0, 0], x[1, 1] = tiny, -tiny
    q, sx = nm.act_quant(x)
    assert sx[0] == 0.0
    assert q[0, 0] == 127 and q[1, 1] == -127 and q[0, 5] == 127
    sx_c = onat.act_scales(x)
    assert np.array_equal(sx_c, sx) and np.array_equal(onat.act_quant(x, sx_c), q)


def test_zero_tile_scale_one_codes_zero():
    x = np.zeros((3, 130), np.float32)
    x[:, 64:128] = 1.5
    q, sx = nm.act_quant(x)
    assert sx[0] == 1.0 and sx[2] == 1.0
    assert np.all(q[:, :64] == 0) and np.all(q[:, 128:] == 0)
    assert np.all(q[:, 64:128] == 127)


@pytest.mark.parametrize("n,k,dtype", [(16, 3072, torch.bfloat16), (4, 100, torch.bfloat16),
                                       (37, 8192, torch.bfloat16), (8, 640, torch.float16), (1, 64, torch.bfloat16)])
def test_act_quant_numpy_c_torch_agree(n, k, dtype):
    x = make_x(n, k, seed=n * 7 + k, dtype=dtype)
    xv = values(x)
    q, sx = nm.act_quant(xv, dtype == torch.bfloat16)
    # torch-CPU statement of the reference CPU branch (quant_utils.py:61-74, 103-115):
    # oracle.torch_ref, also the quantization leg of bench.py's CPU baseline
    from oracle import torch_ref

    q_t, sx_t = torch_ref.act_quant(x)
    assert np.array_equal(sx, sx_t.numpy())
    assert np.array_equal(q, q_t.numpy())
    sx_c = onat.act_scales(xv, dtype == torch.bfloat16)
    assert np.array_equal(sx_c, sx)
    assert np.array_equal(onat.act_quant(xv, sx_c), q)


def test_planted_scale_mistakes():
    a = nm.bf16_bits_to_f32(ALL_POS_BF16)
    good = nm.round_to_dtype(a / np.float32(127.0), True)
    # a fact, not a mistake: no bf16 absmax puts a/127 on a bf16 rounding
    # boundary, so a reciprocal multiply gives the same bf16 scale everywhere
    assert np.array_equal(good, nm.round_to_dtype(a * np.float32(1.0 / 127.0), True))
    # planted: skipping the rounding of the scale to bf16 is caught
    assert not np.array_equal(good, a / np.float32(127.0))
    # planted: rounding toward zero instead of to nearest-even is caught
    trunc = (np.asarray(a / np.float32(127.0)).view(np.uint32) & 0xFFFF0000).view(np.float32)
    assert not np.array_equal(good, trunc)


# --------------------------------------------------------------------------
# weight tiles
# --------------------------------------------------------------------------

def test_weight_scale_exhaustive_vs_torch_cpu_and_not_reciprocal():
    a = nm.bf16_bits_to_f32(ALL_POS_BF16)
    tiles = np.zeros((a.size, 64, 64), np.float32)
    tiles[:, 3, 5] = a
    sw = nm.weight_tile_scales(tiles)
    # reference packer: amax in bf16 -> float32 -> / 127.0 (pack.py:125-130)
    ref = (_torch_bf16(ALL_POS_BF16).to(torch.float32) / 127.0).numpy()
    assert np.array_equal(sw, ref)
    assert np.count_nonzero(sw != (a * np.float32(1.0 / 127.0))) > 0   # planted variant differs
    assert np.count_nonzero(sw != nm.round_bf16(sw)) > 0                 # scales are NOT bf16


def test_weight_codes_vs_torch_cpu():
    W = make_w(128, 192, seed=5)
    ids = np.arange(6)
    tiles = nm.tiles_of(values(W), ids, 3)
    q, sw = nm.weight_tile_quant(tiles)
    t = torch.from_numpy(tiles).to(torch.bfloat16)
    ma = t.abs().amax(dim=(1, 2)).to(torch.float32)
    sw_t = torch.where(ma == 0, torch.ones_like(ma), (ma / 127.0).to(torch.float32))
    q_t = torch.clamp(torch.round(t / sw_t[:, None, None]), -127, 127).to(torch.int8)
    assert np.array_equal(sw, sw_t.numpy()) and np.array_equal(q, q_t.numpy())
    qc, swc = onat.weight_tiles_quant(tiles)
    assert np.array_equal(qc, q) and np.array_equal(swc, sw)
    # dequantization error bound of round-to-nearest: half a step, plus one
    # ulp of the fp32 quotient (|w/sw| <= 127 < 128, ulp 2^-17) because the
    # quotient is rounded to fp32 before rint (it can land on k + 0.5)
    err = np.abs(q.astype(np.float64) * sw[:, None, None].astype(np.float64) - tiles.astype(np.float64))
    assert np.all(err <= sw[:, None, None].astype(np.float64) * (0.5 + 2.0 ** -17))


# --------------------------------------------------------------------------
# INT32 tile products and the tile GEMM
# --------------------------------------------------------------------------

def test_tile_products_brute_force_tiny():
    rng = np.random.default_rng(3)
    xq = rng.integers(-127, 128, size=(3, 130), dtype=np.int8)
    w8 = rng.integers(-127, 128, size=(4, 64, 64), dtype=np.int8)
    ids = np.array([0, 2, 4, 5])    # n_tc = 3 -> columns 0, 2, 1, 2
    p = nm.tile_products_i32(xq, w8, ids, 3)
    for t, tid in enumerate(ids):
        c = tid % 3
        for n in range(3):
            for j in (0, 17, 63):
                want = sum(int(xq[n, c * 64 + kk]) * int(w8[t, j, kk]) for kk in range(64) if c * 64 + kk < 130)
                assert p[t, n, j] == want
    assert np.array_equal(onat.tile_products_i32(xq, w8, ids, 3), p)


def test_tile_products_linearity_and_sign():
    rng = np.random.default_rng(4)
    x1 = rng.integers(-60, 61, size=(5, 256), dtype=np.int8)
    x2 = rng.integers(-60, 61, size=(5, 256), dtype=np.int8)
    w8 = rng.integers(-127, 128, size=(8, 64, 64), dtype=np.int8)
    ids = np.arange(8)
    p1, p2 = nm.tile_products_i32(x1, w8, ids, 4), nm.tile_products_i32(x2, w8, ids, 4)
    assert np.array_equal(nm.tile_products_i32((x1 + x2).astype(np.int8), w8, ids, 4), p1 + p2)
    assert np.array_equal(nm.tile_products_i32((-x1).astype(np.int8), w8, ids, 4), -p1)
    assert np.abs(nm.tile_products_i32(np.full((1, 64), 127, np.int8), np.full((1, 64, 64), -127, np.int8),
                                       [0], 1)).max() == 64 * 127 * 127


def _config(n=16, m=3072, k=3072, frac=0.01, seed=0):
    W = make_w(m, k, seed=seed + 1)
    n_tr, n_tc = -(-m // 64), -(-k // 64)
    ids16 = uniform_fp16_ids(n_tr, n_tc, frac, seed=seed + 2)
    p = oracle_pack(W, ids16)
    x = make_x(n, k, seed=seed + 3)
    xv = values(x)
    xq, sx = nm.act_quant(xv)
    return p, xv, xq, sx


def test_gemm_f64_numpy_c_dense_agree():
    p, xv, xq, sx = _config(n=5, m=320, k=448, frac=0.1)
    args = (xq, sx, xv, p.int8_tiles, p.int8_scales, p.int8_tile_ids, p.int8_row_ptr,
            nm.bf16_bits_to_f32(p.fp16_tiles), p.fp16_tile_ids, p.fp16_row_ptr, p.n_tr, p.n_tc, p.M_orig, p.K_orig)
    acc_np, sab_np = nm.gemm_mixed_f64(*args)
    y32, acc_c, sab_c = onat.gemm_mixed(*args, want_f64=True)
    dense = nm.dense_dequant_reference(xq, sx, xv, p.int8_tiles, p.int8_scales, p.int8_tile_ids,
                                       nm.bf16_bits_to_f32(p.fp16_tiles), p.fp16_tile_ids, p.n_tr, p.n_tc,
                                       p.M_orig, p.K_orig)
    scale = np.abs(acc_np).max()
    assert np.abs(acc_np - acc_c).max() <= 1e-12 * scale
    assert np.abs(acc_np - dense).max() <= 1e-12 * scale
    assert np.allclose(sab_np, sab_c, rtol=1e-12, atol=0)
    # the reference-order fp32 result sits inside the tolerance used for the GPU
    tol = nm.gemm_tolerance(acc_c, sab_c, p.n_tc)
    assert np.all(np.abs(y32 - acc_c) <= tol)


def test_gemm_known_answer():
    # one row tile, two column tiles: tile (0,0) INT8 all-ones codes with scale
    # 0.5, tile (0,1) bf16 all 0.25; x codes all 2 with sx = 0.1, x values 1.0
    xq = np.full((2, 128), 2, np.int8)
    sx = np.array([0.1, 0.1], np.float32)
    xv = np.ones((2, 128), np.float32)
    w8 = np.ones((1, 64, 64), np.int8)
    w16 = np.full((1, 64, 64), 0.25, np.float32)
    y, acc, sab = onat.gemm_mixed(xq, sx, xv, w8, np.array([0.5], np.float32), np.array([0], np.int32),
                                  np.array([0, 1], np.int32), w16, np.array([1], np.int32),
                                  np.array([0, 1], np.int32), 1, 2, 64, 128, want_f64=True)
    want = 64 * 2 * float(np.float32(0.1)) * 0.5 + 64 * 0.25
    assert np.allclose(acc, want, rtol=1e-12)
    assert np.all(y == nm.round_bf16(np.float32(np.float32(128.0) * (np.float32(0.1) * np.float32(0.5)) + np.float32(16.0))))


def test_planted_dropped_tile_fails_tolerance():
    p, xv, xq, sx = _config(n=4, m=256, k=1024, frac=0.05, seed=9)
    args = [xq, sx, xv, p.int8_tiles, p.int8_scales, p.int8_tile_ids, p.int8_row_ptr,
            nm.bf16_bits_to_f32(p.fp16_tiles), p.fp16_tile_ids, p.fp16_row_ptr, p.n_tr, p.n_tc, p.M_orig, p.K_orig]
    y32, acc, sab = onat.gemm_mixed(*args, want_f64=True)
    tol = nm.gemm_tolerance(acc, sab, p.n_tc)
    # plant: zero the scale of one INT8 tile (drops its term)
    sw_bad = p.int8_scales.copy()
    sw_bad[5] = 0.0
    args[4] = sw_bad
    y_bad = onat.gemm_mixed(*args)
    assert np.any(np.abs(y_bad - acc) > tol)
    # plant: transposed INT8 tile
    w_bad = p.int8_tiles.copy()
    w_bad[7] = w_bad[7].T
    args[4], args[3] = p.int8_scales, w_bad
    y_bad = onat.gemm_mixed(*args)
    assert np.any(np.abs(y_bad - acc) > tol)


# --------------------------------------------------------------------------
# packing bookkeeping and tile layouts
# --------------------------------------------------------------------------

def test_pack_bookkeeping_invariants():
    W = make_w(200, 300, seed=11)              # ragged: pads to 256 x 320
    ids16 = uniform_fp16_ids(4, 5, 0.2, seed=12)
    p = oracle_pack(W, ids16)
    assert (p.M, p.K, p.n_tr, p.n_tc) == (256, 320, 4, 5)
    assert p.int8_tile_ids.size + p.fp16_tile_ids.size == 20
    assert np.all(np.diff(p.int8_tile_ids) > 0) and np.all(np.diff(p.fp16_tile_ids) > 0)
    assert p.int8_row_ptr[-1] == p.int8_tile_ids.size and p.fp16_row_ptr[-1] == p.fp16_tile_ids.size
    for r in range(4):
        sl = p.int8_tile_ids[p.int8_row_ptr[r]:p.int8_row_ptr[r + 1]]
        assert np.all(sl // 5 == r)
    # padding reads as zeros: the last row tile's padded rows quantize to 0
    last = [t for t, i in enumerate(p.int8_tile_ids) if i // 5 == 3]
    assert np.all(p.int8_tiles[last][:, 8:, :] == 0)


def test_concat_rows_matches_single_pack_of_stacked_weight():
    Wq, Wk = make_w(128, 192, seed=21), make_w(64, 192, seed=22)
    iq, ik = uniform_fp16_ids(2, 3, 0.3, seed=23), uniform_fp16_ids(1, 3, 0.4, seed=24)
    cat = opk.concat_rows([oracle_pack(Wq, iq), oracle_pack(Wk, ik)])
    whole = oracle_pack(torch.cat([Wq, Wk]), np.concatenate([iq, ik + 2 * 3]))
    for f in ("int8_tiles", "int8_scales", "int8_tile_ids", "int8_row_ptr", "fp16_tiles", "fp16_tile_ids", "fp16_row_ptr"):
        assert np.array_equal(getattr(cat, f), getattr(whole, f)), f


def test_mfma_layouts_roundtrip_and_chunk_maps():
    rng = np.random.default_rng(5)
    t8 = rng.integers(-127, 128, size=(3, 64, 64), dtype=np.int8)
    t16 = rng.integers(0, 65535, size=(2, 64, 64), dtype=np.uint16)
    assert np.array_equal(opk.from_mfma_int8(opk.to_mfma_int8(t8)), t8)
    assert np.array_equal(opk.from_mfma_16bit(opk.to_mfma_16bit(t16)), t16)
    m8 = opk.to_mfma_int8(t8).reshape(3, 256, 16)
    for j, kq in [(0, 0), (17, 2), (63, 3), (40, 1)]:
        chunk = (j // 16) * 64 + kq * 16 + j % 16       # chunk map used by tq_pack.hip / tq_gemm.hip
        assert np.array_equal(m8[1, chunk], t8[1, j, kq * 16:(kq + 1) * 16])
    m16 = opk.to_mfma_16bit(t16).reshape(2, 512, 8)
    for j, k8 in [(0, 0), (19, 5), (63, 7), (33, 3)]:
        chunk = ((j // 16) * 2 + k8 // 4) * 64 + (k8 % 4) * 16 + j % 16
        assert np.array_equal(m16[0, chunk], t16[0, j, k8 * 8:(k8 + 1) * 8])


# --------------------------------------------------------------------------
# Decision/ maps: format and the top-k rule (golden fixtures)
# --------------------------------------------------------------------------

KAT = np.load(__import__("pathlib").Path(__file__).parent / "golden" / "decision_topk_kat.npz")
KAT_CASES = sorted({k.rsplit("__", 1)[0] for k in KAT.files})


@pytest.mark.parametrize("case", KAT_CASES)
@pytest.mark.parametrize("keep,frac", [("keep01", 0.01), ("keep05", 0.05), ("keep20", 0.20)])
def test_topk_rule_reproduces_released_maps(case, keep, frac):
    scores = KAT[f"{case}__scores"]
    released = np.sort(KAT[f"{case}__{keep}"].astype(np.int64))
    n_tr, n_tc = (int(v) for v in KAT[f"{case}__shape"])
    assert scores.shape == (n_tr, n_tc)
    assert released.size == om.keep_count(n_tr * n_tc, frac)
    ours = om.topk_ids(scores, frac)
    flat = scores.reshape(-1)
    kth = np.sort(flat)[-released.size]
    if np.count_nonzero(flat == kth) == 1:
        assert np.array_equal(ours, released)
    else:   # an exact tie at the k-th score: any tied choice is valid
        assert np.array_equal(np.sort(flat[ours]), np.sort(flat[released]))


def test_released_archive_format():
    arch = om.read_archive(__import__("pathlib").Path(__file__).parent / "golden" / "llama32_3b_gi_keep01" /
                           "fp16_keep_ids_tile64x64.npz")
    assert len(arch) == 196
    shapes = {s.rsplit("_", 2)[-2] + "_" + s.rsplit("_", 2)[-1]: shp for s, (shp, _) in arch.items()}
    assert shapes["q_proj"] == (48, 48) and shapes["k_proj"] == (16, 48)
    assert shapes["gate_proj"] == (128, 48) and shapes["down_proj"] == (48, 128)
    for stem, ((n_tr, n_tc), ids) in arch.items():
        assert ids.dtype == np.uint16 and np.all(np.diff(ids.astype(np.int64)) > 0)
        assert ids.size == om.keep_count(n_tr * n_tc, 0.01)


def _all_bf16_in(lo, hi):
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    v = nm.bf16_bits_to_f32(bits)
    return np.unique(v[np.isfinite(v) & (v >= lo) & (v <= hi)])


@pytest.mark.parametrize("dtype,amax", [("bf16", 127.0), ("bf16", 100.0), ("bf16", 3.0e-3), ("fp16", 1000.0),
                                        ("fp16", 0.37), ("fp32", 5.0)])
def test_tensor_quant_matches_reference_torch_expressions(dtype, amax):
    """oracle.numerics.tensor_quant against the reference's own torch
    expressions (quant_utils.py:17-32, on CPU tensors) over every value of the
    dtype in [-amax, amax] (fp32: a dense grid with exact half-integer
    quotients), plus all-zero and empty tensors."""
    from oracle import torch_ref

    tdt = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}[dtype]
    if dtype == "bf16":
        v = _all_bf16_in(-amax, amax)
    elif dtype == "fp16":
        h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
        v = np.unique(h[np.isfinite(h) & (np.abs(h) <= amax)])
    else:
        s = np.float32(amax) / np.float32(127.0)
        v = np.concatenate([np.arange(-1270, 1271, dtype=np.float32) / np.float32(10) * s,
                            (np.arange(-127, 127, dtype=np.float32) + np.float32(0.5)) * s, [np.float32(amax)]])
    x = torch.from_numpy(np.asarray(v, np.float32)).to(tdt)
    q_t, s_t = torch_ref.tensor_quant(x)
    q, s = nm.tensor_quant(x.float().numpy(), dtype)
    assert np.float32(s) == np.float32(s_t.item())
    assert np.array_equal(q, q_t.numpy())
    assert q.min() >= -127 and q.max() <= 127 and np.abs(q).max() >= 126
    for special in (torch.zeros((3, 5), dtype=tdt), torch.zeros((0, 64), dtype=tdt)):
        q0, s0 = nm.tensor_quant(special.float().numpy(), dtype)
        q0t, s0t = torch_ref.tensor_quant(special)
        assert q0.shape == tuple(special.shape) and np.array_equal(q0, q0t.numpy()) and s0 == s0t.item() == 1.0


def test_tensor_quant_planted_mistake_is_caught():
    """Dropping the rounding of the quotient to bf16 (rint of the fp32 quotient,
    as the tile kernels do) disagrees with the reference's expressions."""
    from oracle import torch_ref

    x = torch.from_numpy(_all_bf16_in(-100.0, 100.0)).to(torch.bfloat16)
    q_t, s_t = torch_ref.tensor_quant(x)
    wrong = nm.quant_codes(x.float().numpy(), np.float32(s_t.item()))
    assert not np.array_equal(wrong, q_t.numpy())


def _iaa_case(m, k, seed, dtype=torch.bfloat16):
    from oracle import packing as opk

    g = torch.Generator().manual_seed(seed)
    W = (torch.randn((m, k), generator=g) * 0.02).to(dtype)
    W[:64, :64] = 0                       # an all-zero tile: the three candidates tie exactly
    imp = torch.rand(k, generator=g) * 3
    imp[64:128] = 0                       # importance clamped to 1e-8
    n_tr, n_tc = m // 64, k // 64
    src = W.view(n_tr, 64, n_tc, 64).permute(0, 2, 1, 3).reshape(-1, 64, 64)
    cols = torch.arange(n_tr * n_tc) % n_tc
    return src, imp.view(n_tc, 64)[cols], opk


def test_iaa_oracle_matches_reference_torch_expressions():
    """oracle.packing.iaa_scales (float64 error sums) against the reference's
    torch expressions (pack.py:132-159 on CPU tensors, fp32 means): the same
    choice on every tile whose two best errors differ by more than an fp32
    summation bound, and few tiles inside it; the all-zero tile takes the
    first candidate (0.75 x 1)."""
    from oracle import torch_ref

    src, col_imp, opk = _iaa_case(512, 2048, seed=5)
    s_ref, e_ref = torch_ref.iaa_scales(src, col_imp)
    s_or, e_or = opk.iaa_scales(src.float().numpy(), col_imp.numpy())
    srt = np.sort(e_or, axis=0)
    near = (srt[1] - srt[0]) <= 1e-4 * srt[1]
    assert np.array_equal(s_or[~near], s_ref.numpy()[~near])
    assert near.sum() <= 3 and s_or[0] == np.float32(0.75)
    # the fp32 means agree with the float64 ones to fp32 summation accuracy
    assert np.allclose(e_ref.double().numpy(), e_or, rtol=1e-4, atol=0)
    # planted: a last-wins tie rule (<=) changes the zero tile's choice
    best = np.zeros(e_or.shape[1], dtype=np.int64)
    for i in (1, 2):
        best = np.where(e_or[i] <= e_or[best, np.arange(e_or.shape[1])], i, best)
    assert best[0] == 2
