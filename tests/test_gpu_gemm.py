"""GPU parity: packer, INT32 tile products and the mixed tile GEMM vs the oracle.

Bars: packed tiles / scales and INT32 tile products bit-exact; outputs within
2 bf16 ulp + the fp32 accumulation bound of the float64 oracle
(helpers.assert_gemm_close); bitwise run-to-run reproducibility.
"""
from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from helpers import assert_gemm_close, bits, complement, make_w, make_x, oracle_pack, uniform_fp16_ids, values
from oracle import native as onat
from oracle import numerics as nm
from oracle import packing as opk
from tilequant_amd.gemm_rows_splitk_64x64 import PrefillPlan, gemm_mixed_rows_products_i32, gemm_mixed_rows_splitk, \
    prefill_plan
from tilequant_amd.pack import pack_weight_from_tile_ids, relayout_pack
from tilequant_amd.quant_utils import quantize_activation_tile_absmax

pytestmark = pytest.mark.gpu

CFG = SimpleNamespace(quant_style="gi", dtype_out="bf16")


def _case(m, k, frac, seed, dtype=torch.bfloat16, layout="mfma"):
    W = make_w(m, k, seed=seed, dtype=dtype)
    n_tr, n_tc = -(-m // 64), -(-k // 64)
    ids16 = uniform_fp16_ids(n_tr, n_tc, frac, seed=seed + 1) if frac > 0 else np.zeros(0, np.int64)
    ids8 = complement(ids16, n_tr * n_tc)
    pack = pack_weight_from_tile_ids(W, n_tr=n_tr, n_tc=n_tc, int8_tile_ids=torch.from_numpy(ids8),
                                     fp16_tile_ids=torch.from_numpy(ids16), cfg=CFG, tile_layout=layout)
    return W, pack, ids16


def _oracle_f64(pack, op, x_cpu, xq, sx):
    w16 = (nm.bf16_bits_to_f32(op.fp16_tiles) if x_cpu.dtype == torch.bfloat16
           else op.fp16_tiles.view(np.float16).astype(np.float32))
    _, acc, sab = onat.gemm_mixed(xq, sx, values(x_cpu), op.int8_tiles, op.int8_scales, op.int8_tile_ids,
                                  op.int8_row_ptr, w16, op.fp16_tile_ids, op.fp16_row_ptr, pack.n_tr, pack.n_tc,
                                  pack.M_orig, pack.K_orig, want_f64=True)
    return acc, sab


def _oracle_pack_any(W, ids16):
    if W.dtype == torch.bfloat16:
        return oracle_pack(W, ids16)
    # fp16 weights: same numerics on fp16 values
    wv = values(W)
    p = opk.pack_weight(nm.f32_to_bf16_bits(np.zeros_like(wv)), ids16)  # bookkeeping only
    wp = opk.pad64(wv)
    ids8 = p.int8_tile_ids.astype(np.int64)
    q, sw = nm.weight_tile_quant(nm.tiles_of(wp, ids8, p.n_tc))
    p.int8_tiles, p.int8_scales = q, sw
    p.fp16_tiles = nm.tiles_of(opk.pad64(bits(W)), p.fp16_tile_ids.astype(np.int64), p.n_tc)
    return p


def _kw(pack, xd, xq, sx, bias=None, out=None, split_k=None, out_dtype=torch.bfloat16):
    return dict(
        x_fp=xd, x_int8=xq, sx=sx, int8_tiles=pack.int8_tiles, int8_scales=pack.int8_scales,
        int8_tile_ids=pack.int8_tile_ids, int8_row_ptr=pack.int8_row_ptr, fp16_tiles=pack.fp16_tiles,
        fp16_tile_ids=pack.fp16_tile_ids, fp16_row_ptr=pack.fp16_row_ptr, M=pack.M_orig, K=pack.K_orig,
        n_tr=pack.n_tr, n_tc=pack.n_tc, out_dtype=out_dtype, bias=bias, split_k=split_k, out=out,
        tile_layout=pack.tile_layout)


def _gemm(pack, xd, xq, sx, bias=None, out=None, split_k=None, out_dtype=torch.bfloat16):
    return gemm_mixed_rows_splitk(**_kw(pack, xd, xq, sx, bias, out, split_k, out_dtype))


def test_config1_packer_products_and_output():
    """3072->3072, 16 tokens, keep01 uniform, outlier activations."""
    W, pack, ids16 = _case(3072, 3072, 0.01, seed=100)
    op = oracle_pack(W, ids16)
    assert pack.int8_tiles.shape[0] == 2280 and pack.fp16_tiles.shape[0] == 24
    # packer: scales, codes and 16-bit tiles bit-exact (after undoing the MFMA layout)
    assert np.array_equal(pack.int8_scales.cpu().numpy().view(np.uint32), op.int8_scales.view(np.uint32))
    assert np.array_equal(opk.from_mfma_int8(pack.int8_tiles.cpu().numpy()), op.int8_tiles)
    assert np.array_equal(opk.from_mfma_16bit(bits(pack.fp16_tiles.cpu())), op.fp16_tiles)
    for f in ("int8_tile_ids", "int8_row_ptr", "fp16_tile_ids", "fp16_row_ptr"):
        assert np.array_equal(getattr(pack, f).cpu().numpy(), getattr(op, f)), f
    x = make_x(16, 3072, seed=101)
    xd = x.cuda()
    xq, sx = quantize_activation_tile_absmax(xd)
    xq_ref, sx_ref = nm.act_quant(values(x))
    assert np.array_equal(xq.cpu().numpy(), xq_ref) and np.array_equal(sx.cpu().numpy(), sx_ref)
    # INT32 tile products: bit-exact, from the DUMP instantiation of the kernel this shape runs
    y_dump, P, kern = gemm_mixed_rows_products_i32(**_kw(pack, xd, xq, sx))
    assert kern == "decode"
    P_ref = onat.tile_products_i32(xq_ref, op.int8_tiles, op.int8_tile_ids, 48)
    assert np.array_equal(P.cpu().numpy(), P_ref)
    # output within tolerance of the exact sum
    y = _gemm(pack, xd, xq, sx)
    assert torch.equal(y_dump, y)
    acc, sab = _oracle_f64(pack, op, x, xq_ref, sx_ref)
    worst_ulp = assert_gemm_close(y, acc, sab, 48)
    assert worst_ulp <= 2.0
    # run-to-run bitwise reproducible
    for _ in range(3):
        assert torch.equal(_gemm(pack, xd, xq, sx), y)
    # the reference's row-major tile order gives bitwise the same output
    rm = relayout_pack(pack, "row_major")
    assert np.array_equal(rm.int8_tiles.cpu().numpy(), op.int8_tiles)
    assert torch.equal(_gemm(rm, xd, xq, sx), y)
    _, P_rm, _ = gemm_mixed_rows_products_i32(**_kw(rm, xd, xq, sx))
    assert torch.equal(P_rm, P)
    back = relayout_pack(rm, "mfma")
    assert torch.equal(back.int8_tiles, pack.int8_tiles) and torch.equal(back.fp16_tiles, pack.fp16_tiles)


@pytest.mark.parametrize("m,k", [(1024, 3072), (8192, 3072), (3072, 8192), (5120, 3072), (16384, 3072)])
@pytest.mark.parametrize("n", [1, 4, 16, 24, 64])
def test_llama_decode_shapes(m, k, n):
    """BASELINE configs[1] shapes (k/v, gate/up, down, fused QKV) at decode token counts."""
    W, pack, ids16 = _case(m, k, 0.01, seed=m + k + n)
    op = oracle_pack(W, ids16)
    x = make_x(n, k, seed=7 * n + m)
    xd = x.cuda()
    xq, sx = quantize_activation_tile_absmax(xd)
    xq_ref, sx_ref = nm.act_quant(values(x))
    y = _gemm(pack, xd, xq, sx)
    acc, sab = _oracle_f64(pack, op, x, xq_ref, sx_ref)
    assert_gemm_close(y, acc, sab, pack.n_tc)


@pytest.mark.parametrize("n", [2, 33, 100, 257])
def test_token_counts_and_ragged_shapes(n):
    W, pack, ids16 = _case(200, 300, 0.2, seed=300 + n)       # pads to 256 x 320, K % 64 != 0
    op = oracle_pack(W, ids16)
    x = make_x(n, 300, seed=301 + n)
    xd = x.cuda()
    xq, sx = quantize_activation_tile_absmax(xd)
    xq_ref, sx_ref = nm.act_quant(values(x))
    assert np.array_equal(xq.cpu().numpy(), xq_ref)
    # K % 64 != 0: split-K decode kernel (<= 64 rows) or register prefill kernel, on unaligned rows
    y_dump, P, kern = gemm_mixed_rows_products_i32(**_kw(pack, xd, xq, sx))
    assert kern == ("splitk" if n <= 64 else "prefill_register")
    assert np.array_equal(P.cpu().numpy(), onat.tile_products_i32(xq_ref, op.int8_tiles, op.int8_tile_ids, 5, K=300))
    y = _gemm(pack, xd, xq, sx)
    assert torch.equal(y_dump, y)
    acc, sab = _oracle_f64(pack, op, x, xq_ref, sx_ref)
    assert_gemm_close(y, acc, sab, pack.n_tc)


@pytest.mark.parametrize("frac", [0.0, 1.0, 0.5])
def test_all_int8_all_bf16_and_half(frac):
    W, pack, ids16 = _case(256, 512, frac, seed=400)
    op = oracle_pack(W, ids16)
    x = make_x(8, 512, seed=401)
    xd = x.cuda()
    xq, sx = quantize_activation_tile_absmax(xd)
    y = _gemm(pack, xd, xq, sx)
    acc, sab = _oracle_f64(pack, op, x, *nm.act_quant(values(x)))
    assert_gemm_close(y, acc, sab, pack.n_tc)


@pytest.mark.parametrize("m,k,frac,n", [(256, 8192, 1.0, 1), (256, 8192, 1.0, 4), (320, 8192, 0.9, 16),
                                        (12288, 1024, 0.9, 12), (512, 18944, 0.97, 4)])
def test_decode_rows_with_many_16bit_tiles(m, k, frac, n):
    """Row tiles that are (almost) all 16-bit: each wave takes dozens of 16-bit
    tiles past its first ones (batched loads; one-j-block and whole-tile
    workgroups)."""
    W, pack, ids16 = _case(m, k, frac, seed=m + k + n)
    op = oracle_pack(W, ids16)
    x = make_x(n, k, seed=m + n)
    xd = x.cuda()
    xq, sx = quantize_activation_tile_absmax(xd)
    y = _gemm(pack, xd, xq, sx)
    acc, sab = _oracle_f64(pack, op, x, *nm.act_quant(values(x)))
    assert_gemm_close(y, acc, sab, pack.n_tc)


def test_bias_fp16_output_and_out_slices():
    W, pack, ids16 = _case(384, 640, 0.05, seed=500)
    op = oracle_pack(W, ids16)
    x = make_x(12, 640, seed=501)
    xd = x.cuda()
    xq, sx = quantize_activation_tile_absmax(xd)
    xq_ref, sx_ref = nm.act_quant(values(x))
    acc, sab = _oracle_f64(pack, op, x, xq_ref, sx_ref)
    bias = (torch.randn(384, generator=torch.Generator().manual_seed(5)) * 0.5).to(torch.bfloat16)
    y = _gemm(pack, xd, xq, sx, bias=bias.cuda())
    assert_gemm_close(y, acc, sab, pack.n_tc, bias=values(bias))
    # bias semantics: round(round(acc) + bias), as the reference's epilogue
    y_nb = _gemm(pack, xd, xq, sx)
    want = (y_nb.float() + bias.cuda().float()).to(torch.bfloat16)
    assert torch.equal(y, want)
    # fp16 output
    y16 = _gemm(pack, xd, xq, sx, out_dtype=torch.float16)
    assert y16.dtype == torch.float16
    assert np.all(np.abs(values(y16).astype(np.float64) - acc) <= 2 * np.abs(acc) * 2.0 ** -10 + 1e-5 * sab + 1e-7)
    # writing into a row slice of a larger output (the chunked path)
    big = torch.full((20, 384), 7.0, dtype=torch.bfloat16, device="cuda")
    _gemm(pack, xd, xq, sx, out=big[4:16])
    assert torch.equal(big[4:16], y_nb) and torch.all(big[:4] == 7) and torch.all(big[16:] == 7)
    with pytest.raises(ValueError):
        _gemm(pack, xd, xq, sx, out=torch.empty((12, 383), dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(ValueError):
        _gemm(pack, xd, xq, sx, out=torch.empty((12, 384), dtype=torch.float16, device="cuda"))


def test_fp16_activations_and_weights():
    W, pack, ids16 = _case(256, 384, 0.1, seed=600, dtype=torch.float16)
    op = _oracle_pack_any(W, ids16)
    assert np.array_equal(pack.int8_scales.cpu().numpy(), op.int8_scales)
    assert np.array_equal(opk.from_mfma_int8(pack.int8_tiles.cpu().numpy()), op.int8_tiles)
    x = make_x(6, 384, seed=601, dtype=torch.float16)
    xd = x.cuda()
    xq, sx = quantize_activation_tile_absmax(xd)
    xq_ref, sx_ref = nm.act_quant(values(x), is_bf16=False)
    assert np.array_equal(xq.cpu().numpy(), xq_ref) and np.array_equal(sx.cpu().numpy(), sx_ref)
    y = _gemm(pack, xd, xq, sx)
    acc, sab = _oracle_f64(pack, op, x, xq_ref, sx_ref)
    assert_gemm_close(y, acc, sab, pack.n_tc)


@pytest.mark.parametrize("split_k", [1, 2, 3, 8, 16])
def test_split_k_is_deterministic_and_within_tolerance(split_k):
    W, pack, ids16 = _case(512, 2048, 0.05, seed=700)
    op = oracle_pack(W, ids16)
    x = make_x(4, 2048, seed=701)
    xd = x.cuda()
    xq, sx = quantize_activation_tile_absmax(xd)
    y = _gemm(pack, xd, xq, sx, split_k=split_k)
    assert torch.equal(_gemm(pack, xd, xq, sx, split_k=split_k), y)
    acc, sab = _oracle_f64(pack, op, x, *nm.act_quant(values(x)))
    assert_gemm_close(y, acc, sab, pack.n_tc)


def test_empty_token_batch():
    W, pack, _ = _case(128, 128, 0.1, seed=800)
    xd = torch.empty((0, 128), dtype=torch.bfloat16, device="cuda")
    xq = torch.empty((0, 128), dtype=torch.int8, device="cuda")
    y = _gemm(pack, xd, xq, torch.ones(2, device="cuda"))
    assert y.shape == (0, 128)


# --------------------------------------------------------------------------
# split-K decode schedule and the fused quantize + GEMM launch
# --------------------------------------------------------------------------

from tilequant_amd.gemm_rows_splitk_64x64 import linear_mixed_fused  # noqa: E402


def _fused(pack, xd, bias=None, split_k=None, out_dtype=torch.bfloat16):
    return linear_mixed_fused(
        x_fp=xd, int8_tiles=pack.int8_tiles, int8_scales=pack.int8_scales, int8_tile_ids=pack.int8_tile_ids,
        int8_row_ptr=pack.int8_row_ptr, fp16_tiles=pack.fp16_tiles, fp16_tile_ids=pack.fp16_tile_ids,
        fp16_row_ptr=pack.fp16_row_ptr, M=pack.M_orig, K=pack.K_orig, n_tr=pack.n_tr, n_tc=pack.n_tc,
        out_dtype=out_dtype, bias=bias, split_k=split_k, tile_layout=pack.tile_layout)


@pytest.mark.parametrize("n", [1, 2, 3, 4, 7, 8, 13, 16])
def test_fused_equals_two_launch_path_bitwise(n):
    W, pack, ids16 = _case(3072, 3072, 0.01, seed=900 + n)
    x = make_x(n, 3072, seed=901 + n)
    xd = x.cuda()
    xq, sx = quantize_activation_tile_absmax(xd)
    for split_k in (None, 1, 3, 8):
        y2 = _gemm(pack, xd, xq, sx, split_k=split_k)
        y1 = _fused(pack, xd, split_k=split_k)
        assert torch.equal(y1, y2), f"split_k={split_k}"
    op = oracle_pack(W, ids16)
    acc, sab = _oracle_f64(pack, op, x, *nm.act_quant(values(x)))
    assert_gemm_close(y1, acc, sab, 48)


@pytest.mark.parametrize("m,k", [(16384, 3072), (9216, 3584)])
@pytest.mark.parametrize("n", [1, 2, 4, 16])
def test_fused_equals_two_launch_path_on_many_unit_grids(m, k, n):
    """Grids of more than 512 one-j-block workgroups (stacked gate/up widths)
    take 4-wave workgroups with 12- or 16-tile batches: the fused and the
    two-launch paths (and the split-K kernel with one split) still sum the
    same terms in the same order."""
    W, pack, ids16 = _case(m, k, 0.01, seed=950 + n + k)
    x = make_x(n, k, seed=951 + n)
    xd = x.cuda()
    xq, sx = quantize_activation_tile_absmax(xd)
    y2 = _gemm(pack, xd, xq, sx)
    for split_k in (None, 1):
        assert torch.equal(_fused(pack, xd, split_k=split_k), y2), f"split_k={split_k}"
        assert torch.equal(_gemm(pack, xd, xq, sx, split_k=split_k), y2)
    op = oracle_pack(W, ids16)
    acc, sab = _oracle_f64(pack, op, x, *nm.act_quant(values(x)))
    assert_gemm_close(y2, acc, sab, pack.n_tc)


@pytest.mark.parametrize("n", [1, 4, 8, 16])
def test_fused_equals_two_launch_path_on_whole_tile_schedule(n):
    """Stacked gate/up width (256 row tiles): whole-tile workgroups."""
    W, pack, ids16 = _case(16384, 3072, 0.01, seed=950 + n)
    x = make_x(n, 3072, seed=951 + n)
    xd = x.cuda()
    xq, sx = quantize_activation_tile_absmax(xd)
    y2 = _gemm(pack, xd, xq, sx)
    y1 = _fused(pack, xd)
    assert torch.equal(y1, y2)
    op = oracle_pack(W, ids16)
    acc, sab = _oracle_f64(pack, op, x, *nm.act_quant(values(x)))
    assert_gemm_close(y1, acc, sab, 48)


@pytest.mark.parametrize("m,k,frac", [(200, 300, 0.2), (384, 640, 0.05), (128, 64, 0.5), (1024, 8192, 0.02)])
def test_fused_ragged_bias_and_fp16(m, k, frac):
    for dtype in (torch.bfloat16, torch.float16):
        W, pack, ids16 = _case(m, k, frac, seed=m + k, dtype=dtype)
        x = make_x(5, k, seed=m - k, dtype=dtype)
        xd = x.cuda()
        bias = (torch.randn(m, generator=torch.Generator().manual_seed(3)) * 0.3).to(torch.bfloat16).cuda()
        xq, sx = quantize_activation_tile_absmax(xd)
        assert torch.equal(_fused(pack, xd, bias=bias), _gemm(pack, xd, xq, sx, bias=bias))
        assert torch.equal(_fused(pack, xd, out_dtype=torch.float16),
                           _gemm(pack, xd, xq, sx, out_dtype=torch.float16))
    # strided rows (a row slice of a wider activation)
    W, pack, _ = _case(256, 512, 0.1, seed=77)
    big = make_x(6, 1024, seed=78).cuda()
    xs = big[:, 256:768]
    xq, sx = quantize_activation_tile_absmax(xs.contiguous())
    assert torch.equal(_fused(pack, xs), _gemm(pack, xs.contiguous(), xq, sx))


def test_split_k_counters_reset_over_many_launches_and_graph_replays():
    W, pack, ids16 = _case(1024, 3072, 0.01, seed=950)
    x = make_x(4, 3072, seed=951).cuda()
    y0 = _fused(pack, x, split_k=8)
    for _ in range(50):
        assert torch.equal(_fused(pack, x, split_k=8), y0)
    # captured in a HIP graph: replays reuse the same workspace and counters
    out = torch.empty_like(y0)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _fused(pack, x, split_k=8)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):   # same stream as the warm-up: reuses its workspace
        out.copy_(_fused(pack, x, split_k=8))
    for _ in range(5):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, y0)
        assert torch.equal(_fused(pack, x, split_k=8), y0)   # eager work between replays


@pytest.mark.parametrize("m,k", [(3072, 3072), (1024, 4096), (3072, 8192), (640, 1024), (3584, 3584)])
@pytest.mark.parametrize("n", [1, 2, 3, 4])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fused_lane_quantization_equals_two_launch_path(m, k, n, dtype):
    """Fused decode workgroups with one thread per 8-column chunk of a row
    (3072, 4096, 8192 and 3584 columns on these grids) take the column-tile
    absmax from registers and DPP instead of LDS atomics from 2 rows on (from
    one row with 16 waves: 8192 columns); one row on fewer waves and 1024
    columns (4 waves, 128 chunks per row) take the general path.  Both are bitwise the
    separate quantizer + GEMM, including an all-zero column tile (scale 1), a
    tile whose absmax sits in the last row and one of signed half-integers."""
    W, pack, ids16 = _case(m, k, 0.02, seed=970 + n + k, dtype=dtype)
    x = make_x(n, k, seed=971 + n + k, dtype=dtype)
    x[:, 64:128] = 0                                  # scale 1, codes 0
    x[n - 1, 200] = -37.5                             # absmax in the last row, negative
    if k >= 320:
        x[:, 256:320] = torch.tensor([(-1) ** i * (i + 0.5) for i in range(64)], dtype=torch.float32).to(dtype)
    xd = x.cuda()
    xq, sx = quantize_activation_tile_absmax(xd)
    y2 = _gemm(pack, xd, xq, sx, out_dtype=dtype)
    yf = _fused(pack, xd, out_dtype=dtype)
    assert torch.equal(yf, y2)
    assert torch.equal(_fused(pack, xd, out_dtype=dtype), yf)


def test_fused_rejects_more_than_16_rows():
    W, pack, _ = _case(128, 128, 0.1, seed=960)
    with pytest.raises(ValueError):
        _fused(pack, make_x(17, 128).cuda())


def test_workspace_shared_by_calls_with_different_row_tile_counts():
    """Regression: a call with more row tiles must not read an earlier call's
    split partials as its arrival counters (the workspace is shared per stream)."""
    cases = [_case(m, 3072, 0.01, seed=970 + m // 64) for m in (3072, 8192, 1024, 16384, 3072)]
    x = make_x(4, 3072, seed=975)
    xd = x.cuda()
    xq, sx = quantize_activation_tile_absmax(xd)
    xq_ref, sx_ref = nm.act_quant(values(x))
    for _round in range(2):
        for W, pack, ids16 in cases:
            y = _fused(pack, xd)
            assert torch.equal(y, _gemm(pack, xd, xq, sx))
            acc, sab = _oracle_f64(pack, oracle_pack(W, ids16), x, xq_ref, sx_ref)
            assert_gemm_close(y, acc, sab, pack.n_tc)


def test_fused_quantization_handles_exact_ties():
    W, pack, ids16 = _case(256, 256, 0.1, seed=990)
    x = np.zeros((3, 256), np.float32)
    for t, (k0, sign) in enumerate([(0, 1), (0, -1), (63, 1), (40, -1)]):
        k = np.arange(k0, k0 + 63, dtype=np.float32)
        x[t % 3, 64 * t:64 * t + 63] = sign * (k + 0.5) * 0.125
        x[(t + 1) % 3, 64 * t + 63] = 15.875   # absmax -> scale 0.125 exactly
    xt = torch.from_numpy(x).to(torch.bfloat16).cuda()
    xq, sx = quantize_activation_tile_absmax(xt)
    assert torch.equal(xq.cpu(), torch.from_numpy(nm.act_quant(x)[0]))
    assert torch.equal(_fused(pack, xt), _gemm(pack, xt, xq, sx))


@pytest.mark.parametrize("n,m,k,frac", [(512, 3072, 3072, 0.05), (300, 1024, 8192, 0.05), (4096, 256, 3072, 0.2)])
def test_prefill_kernel_shapes(n, m, k, frac):
    """BASELINE configs[2]-style prefill (N > 64: LDS-staged MFMA kernel) vs the oracle."""
    W, pack, ids16 = _case(m, k, frac, seed=n + m)
    op = oracle_pack(W, ids16)
    x = make_x(n, k, seed=n - m)
    xd = x.cuda()
    xq, sx = quantize_activation_tile_absmax(xd)
    xq_ref, sx_ref = nm.act_quant(values(x))
    assert np.array_equal(xq.cpu().numpy(), xq_ref)
    y = _gemm(pack, xd, xq, sx)
    rows = np.unique(np.r_[0:5, n // 2:n // 2 + 5, n - 5:n])
    acc, sab = _oracle_f64(pack, op, x[rows], xq_ref[rows], sx_ref)
    assert_gemm_close(y[rows], acc, sab, pack.n_tc)
    assert torch.equal(_gemm(pack, xd, xq, sx), y)
    rm = relayout_pack(pack, "row_major")
    assert torch.equal(_gemm(rm, xd, xq, sx), y)


@pytest.mark.parametrize("n,m,k,frac", [(300, 512, 3072, 0.05), (257, 256, 1024, 0.0)])
def test_prefill_dma_and_register_paths_agree_bitwise(n, m, k, frac):
    """Aligned activation rows take the DMA-pipelined prefill kernel; a row
    stride that is not a multiple of 16 bytes takes the register-staged one.
    Both apply the same fp32 operations in the same tile order."""
    W, pack, _ = _case(m, k, frac, seed=n + 7)
    x = make_x(n, k, seed=n + 8)
    xd = x.cuda()
    xq, sx = quantize_activation_tile_absmax(xd)
    xq_odd = torch.zeros((n, k + 8), dtype=torch.int8, device="cuda")[:, :k]
    xq_odd.copy_(xq)
    xf_odd = torch.zeros((n, k + 4), dtype=xd.dtype, device="cuda")[:, :k]
    xf_odd.copy_(xd)
    assert torch.equal(_gemm(pack, xd, xq, sx), _gemm(pack, xf_odd, xq_odd, sx))


@pytest.mark.parametrize("n,m,k,frac", [(300, 200, 640, 0.2), (260, 320, 1024, 0.1), (513, 192, 2048, 0.5),
                                         (1000, 3000, 640, 0.2), (700, 3072, 1024, 0.5)])
def test_prefill_dma_path_ragged_outputs_bias_and_strides(n, m, k, frac):
    """The DMA kernels' edges: ragged M (partial last row tile), an odd
    row-tile count (a workgroup with one row), 16-bit tiles in both rows of
    a pair, bias, fp16 output, and an output row stride that forbids 16-byte
    stores -- bitwise equal to the register-staged kernel (unaligned
    activation rows) and within tolerance of the oracle."""
    W, pack, ids16 = _case(m, k, frac, seed=n + m + k)
    op = oracle_pack(W, ids16)
    x = make_x(n, k, seed=n + 3)
    xd = x.cuda()
    xq, sx = quantize_activation_tile_absmax(xd)
    xq_ref, sx_ref = nm.act_quant(values(x))
    xq_odd = torch.zeros((n, k + 8), dtype=torch.int8, device="cuda")[:, :k]
    xq_odd.copy_(xq)
    xf_odd = torch.zeros((n, k + 4), dtype=xd.dtype, device="cuda")[:, :k]
    xf_odd.copy_(xd)
    bias = (torch.randn(m, generator=torch.Generator().manual_seed(n)) * 0.5).to(torch.bfloat16).cuda()
    y = _gemm(pack, xd, xq, sx, bias=bias)
    assert torch.equal(y, _gemm(pack, xf_odd, xq_odd, sx, bias=bias))
    rows = np.unique(np.r_[0:4, n - 4:n])
    acc, sab = _oracle_f64(pack, op, x[rows], xq_ref[rows], sx_ref)
    assert_gemm_close(y[rows], acc, sab, pack.n_tc, bias=values(bias.cpu()))
    wide = torch.full((n, m + 3), 5.0, dtype=torch.bfloat16, device="cuda")
    _gemm(pack, xd, xq, sx, bias=bias, out=wide[:, :m])
    assert torch.equal(wide[:, :m], y) and torch.all(wide[:, m:] == 5)
    y16 = _gemm(pack, xd, xq, sx, out_dtype=torch.float16)
    assert torch.equal(y16, _gemm(pack, xf_odd, xq_odd, sx, out_dtype=torch.float16))


@pytest.mark.parametrize("n,m,k,frac", [(8192, 3072, 256, 0.25), (8192, 3000, 320, 0.1), (8192, 5120, 128, 0.3),
                                         (4096, 4096, 128, 0.3)])
def test_prefill_dma_path_full_grid_at_8192_tokens(n, m, k, frac):
    """Llama o/down and qkv widths at 8192 tokens (768 and 1280 row-pair x
    token-block workgroups, more than one round of the 512 workgroup slots
    of a 256-CU MI355X; m = 3000 leaves the last pair with one row tile; the
    last case fills the slots exactly).  Bitwise equal to the register-staged
    kernel, and within tolerance of the oracle on rows of the first, middle
    and last token blocks."""
    W, pack, ids16 = _case(m, k, frac, seed=m + k)
    op = oracle_pack(W, ids16)
    x = make_x(n, k, seed=n + k)
    xd = x.cuda()
    xq, sx = quantize_activation_tile_absmax(xd)
    xq_ref, sx_ref = nm.act_quant(values(x))
    y = _gemm(pack, xd, xq, sx)
    xq_odd = torch.zeros((n, k + 8), dtype=torch.int8, device="cuda")[:, :k]
    xq_odd.copy_(xq)
    xf_odd = torch.zeros((n, k + 4), dtype=xd.dtype, device="cuda")[:, :k]
    xf_odd.copy_(xd)
    assert torch.equal(y, _gemm(pack, xf_odd, xq_odd, sx))
    rows = np.unique(np.r_[0:3, n // 2:n // 2 + 3, n - 300:n - 297, n - 3:n])
    acc, sab = _oracle_f64(pack, op, x[rows], xq_ref[rows], sx_ref)
    assert_gemm_close(y[rows], acc, sab, pack.n_tc)


@pytest.mark.parametrize("k,frac", [(3584, 0.10), (18944, 0.20), (5120, 0.20), (13824, 0.10)])
@pytest.mark.parametrize("n", [4, 300])
def test_qwen_widths_with_clustered_masks(k, frac, n):
    """the Qwen2.5-7B / 14B K widths (hidden 3584 / 5120,
    MLP 18944 / 13824) with BF16 tiles clustered by the top-k per-tile sum|W|
    rule on a weight with heavy column and row bands, so some row tiles are
    mostly BF16 and others all INT8.  Decode (4 tokens) and prefill (300)
    kernels vs the oracle; the prefill DMA kernel bitwise vs the register one."""
    from oracle import masks as om

    m = 384
    W = make_w(m, k, seed=k + n).float()
    n_tr, n_tc = m // 64, k // 64
    g = torch.Generator().manual_seed(k)
    cb = torch.randperm(n_tc, generator=g)[: max(1, n_tc // 20)]
    W.view(n_tr, 64, n_tc, 64)[:, :, cb, :] *= 4
    W.view(n_tr, 64, n_tc, 64)[1] *= 3
    W = W.to(torch.bfloat16)
    scores = W.float().abs().view(n_tr, 64, n_tc, 64).sum(dim=(1, 3)).numpy()
    ids16 = om.topk_ids(scores, frac)
    ids8 = complement(ids16, n_tr * n_tc)
    pack = pack_weight_from_tile_ids(W, n_tr=n_tr, n_tc=n_tc, int8_tile_ids=torch.from_numpy(ids8),
                                     fp16_tile_ids=torch.from_numpy(ids16), cfg=CFG, tile_layout="mfma")
    rp = pack.fp16_row_ptr.cpu().numpy()
    per_row = rp[1:] - rp[:-1]
    assert per_row.max() > 2 * max(1, per_row.min())   # uneven mixes across row tiles
    op = oracle_pack(W, ids16)
    x = make_x(n, k, seed=k - n)
    xd = x.cuda()
    xq, sx = quantize_activation_tile_absmax(xd)
    xq_ref, sx_ref = nm.act_quant(values(x))
    assert np.array_equal(xq.cpu().numpy(), xq_ref)
    y = _gemm(pack, xd, xq, sx)
    rows = np.unique(np.r_[0:4, n - 4:n])
    acc, sab = _oracle_f64(pack, op, x[rows], xq_ref[rows], sx_ref)
    assert_gemm_close(y[rows], acc, sab, pack.n_tc)
    if n > 64:
        xq_odd = torch.zeros((n, k + 8), dtype=torch.int8, device="cuda")[:, :k]
        xq_odd.copy_(xq)
        xf_odd = torch.zeros((n, k + 4), dtype=xd.dtype, device="cuda")[:, :k]
        xf_odd.copy_(xd)
        assert torch.equal(y, _gemm(pack, xf_odd, xq_odd, sx))


def test_prefill_rows_longer_than_one_metadata_chunk():
    # 1100 tiles per row tile: the DMA kernel stages tile metadata in chunks of 512
    n, m, k = 80, 128, 64 * 1100
    W, pack, ids16 = _case(m, k, 0.01, seed=901)
    op = oracle_pack(W, ids16)
    x = make_x(n, k, seed=902)
    xd = x.cuda()
    xq, sx = quantize_activation_tile_absmax(xd)
    xq_ref, sx_ref = nm.act_quant(values(x))
    y = _gemm(pack, xd, xq, sx)
    acc, sab = _oracle_f64(pack, op, x, xq_ref, sx_ref)
    assert_gemm_close(y, acc, sab, pack.n_tc)


@pytest.mark.parametrize("n,k", [(300, 64 * 320), (130, 64 * 512)])
def test_prefill_wide_k_two_row_kernel(n, k):
    """Inputs of 305..512 column tiles (K 19,520 - 32,768) are past the
    v5 kernel's metadata capacity and take the two-row 4-stage DMA kernel
    (gemm_prefill_v3_kernel): vs the oracle, and bitwise equal to the
    register-staged kernel that unaligned rows select."""
    m = 192
    W, pack, ids16 = _case(m, k, 0.05, seed=k + 5)
    op = oracle_pack(W, ids16)
    x = make_x(n, k, seed=k + 6)
    xd = x.cuda()
    xq, sx = quantize_activation_tile_absmax(xd)
    xq_ref, sx_ref = nm.act_quant(values(x))
    y = _gemm(pack, xd, xq, sx)
    rows = np.unique(np.r_[0:3, n - 3:n])
    acc, sab = _oracle_f64(pack, op, x[rows], xq_ref[rows], sx_ref)
    assert_gemm_close(y[rows], acc, sab, pack.n_tc)
    xq_odd = torch.zeros((n, k + 8), dtype=torch.int8, device="cuda")[:, :k]
    xq_odd.copy_(xq)
    xf_odd = torch.zeros((n, k + 4), dtype=xd.dtype, device="cuda")[:, :k]
    xf_odd.copy_(xd)
    assert torch.equal(y, _gemm(pack, xf_odd, xq_odd, sx))


@pytest.mark.parametrize("split_k", [2, 8])
@pytest.mark.parametrize("n", [24, 48, 64])
def test_split_k_reduction_two_and_four_token_blocks(n, split_k):
    """The cross-workgroup split-K reduction with 32- and 64-token blocks
    (17..64 rows), including a plan whose reduction buffer is the whole 64 KiB
    of its LDS budget (n = 64, split_k = 2 at 64 column tiles): vs the oracle,
    deterministic over repeated launches."""
    m, k = 512, 4096
    W, pack, ids16 = _case(m, k, 0.02, seed=n * 10 + split_k)
    op = oracle_pack(W, ids16)
    x = make_x(n, k, seed=n + split_k)
    xd = x.cuda()
    xq, sx = quantize_activation_tile_absmax(xd)
    xq_ref, sx_ref = nm.act_quant(values(x))
    y = _gemm(pack, xd, xq, sx, split_k=split_k)
    acc, sab = _oracle_f64(pack, op, x, xq_ref, sx_ref)
    assert_gemm_close(y, acc, sab, pack.n_tc)
    for _ in range(3):
        assert torch.equal(_gemm(pack, xd, xq, sx, split_k=split_k), y)


def _banded_case(m, k, heavy_rows, seed):
    """A weight whose listed row tiles are entirely 16-bit (dict row -> 'all')
    or have the given fraction of 16-bit tiles, over a 2% uniform background:
    the row-tile pairs then differ several-fold in prefill work."""
    n_tr, n_tc = -(-m // 64), -(-k // 64)
    rng = np.random.default_rng(seed)
    mask = rng.random((n_tr, n_tc)) < 0.02
    for r, frac in heavy_rows.items():
        mask[r] = True if frac == "all" else rng.random(n_tc) < frac
    ids16 = np.flatnonzero(mask.ravel()).astype(np.int64)
    W = make_w(m, k, seed=seed)
    pack = pack_weight_from_tile_ids(W, n_tr=n_tr, n_tc=n_tc, int8_tile_ids=torch.from_numpy(complement(ids16, n_tr * n_tc)),
                                     fp16_tile_ids=torch.from_numpy(ids16), cfg=CFG, tile_layout="mfma")
    return W, pack, ids16


def _plan_of(units, n_tr, n_first=0):
    return PrefillPlan(torch.tensor(units, dtype=torch.int32, device="cuda"), n_first, n_tr)


@pytest.mark.parametrize("n,m,k,heavy", [
    (300, 768, 4096, {3: "all", 8: 0.5}),            # one whole 16-bit row tile, one half
    (513, 704, 2048, {2: "all", 3: "all", 10: 0.8}),  # a pair with no INT8 column at all; odd row-tile count
    (2048, 1024, 8192, {5: "all"}),
])
def test_prefill_plans_change_nothing_but_the_order(n, m, k, heavy):
    """The prefill kernel's work plans (row-tile pairs and single row tiles)
    give bitwise the plain launch's outputs, which match the oracle; hand-built
    plans cover every unit kind and dispatch order (units sent first too)."""
    W, pack, ids16 = _banded_case(m, k, heavy, seed=n + m)
    x = make_x(n, k, seed=n + 1)
    xd = x.cuda()
    xq, sx = quantize_activation_tile_absmax(xd)
    y = _gemm(pack, xd, xq, sx)
    plan = prefill_plan(int8_tile_ids=pack.int8_tile_ids, int8_row_ptr=pack.int8_row_ptr,
                        fp16_row_ptr=pack.fp16_row_ptr, n_tr=pack.n_tr, n_tc=pack.n_tc)
    assert plan is not None
    units = plan.units.cpu().tolist()
    n_tr = pack.n_tr
    assert any(u >> 30 for u in units)   # the heavy pair is split
    if plan.n_first:
        r = units[0] & ((1 << 30) - 1)
        first_rows = {r} if units[0] >> 30 or r + 1 >= n_tr else {r, r + 1}
        assert first_rows & set(heavy)   # a heavy row's unit goes first
    plans = [plan,
             _plan_of([r | 1 << 30 for r in range(n_tr)], n_tr),                          # all single rows
             _plan_of([r | 1 << 30 for r in reversed(range(n_tr))], n_tr, n_first=3),      # reversed, three first
             _plan_of(list(range(0, n_tr, 2))[::-1], n_tr, n_first=1)]                     # pairs, reversed
    for p in plans:
        out = torch.full_like(y, float("nan"))
        gemm_mixed_rows_splitk(
            x_fp=xd, x_int8=xq, sx=sx, int8_tiles=pack.int8_tiles, int8_scales=pack.int8_scales,
            int8_tile_ids=pack.int8_tile_ids, int8_row_ptr=pack.int8_row_ptr, fp16_tiles=pack.fp16_tiles,
            fp16_tile_ids=pack.fp16_tile_ids, fp16_row_ptr=pack.fp16_row_ptr, M=pack.M_orig, K=pack.K_orig,
            n_tr=pack.n_tr, n_tc=pack.n_tc, out_dtype=torch.bfloat16, out=out, tile_layout=pack.tile_layout,
            prefill_plan=p)
        assert torch.equal(out.view(torch.int16), y.view(torch.int16))
    with pytest.raises(ValueError, match="row tiles"):   # a plan for a smaller matrix would skip row tiles
        gemm_mixed_rows_splitk(
            x_fp=xd, x_int8=xq, sx=sx, int8_tiles=pack.int8_tiles, int8_scales=pack.int8_scales,
            int8_tile_ids=pack.int8_tile_ids, int8_row_ptr=pack.int8_row_ptr, fp16_tiles=pack.fp16_tiles,
            fp16_tile_ids=pack.fp16_tile_ids, fp16_row_ptr=pack.fp16_row_ptr, M=pack.M_orig, K=pack.K_orig,
            n_tr=pack.n_tr, n_tc=pack.n_tc, out_dtype=torch.bfloat16, tile_layout=pack.tile_layout,
            prefill_plan=_plan_of(list(range(0, n_tr - 2, 2)), n_tr - 2))
    op = oracle_pack(W, ids16)
    xq_ref, sx_ref = nm.act_quant(values(x))
    rows = np.unique(np.r_[0:3, n // 2, n - 3:n])
    acc, sab = _oracle_f64(pack, op, x[rows], xq_ref[rows], sx_ref)
    assert_gemm_close(y[rows], acc, sab, pack.n_tc)


def test_mixed_linear_builds_and_uses_the_prefill_plan():
    from tilequant_amd.mixed_linear import MixedLinear

    W, pack, _ = _banded_case(640, 3072, {4: "all"}, seed=77)
    lin = MixedLinear(pack, None, CFG)
    x = make_x(1000, 3072, seed=78).cuda()
    y = lin(x)
    assert lin._plan is not None and lin._plan[0] is not None
    xq, sx = quantize_activation_tile_absmax(x)
    assert torch.equal(y, _gemm(pack, x, xq, sx))
    assert lin(x[:4]).shape == (4, 640)   # decode sizes run without it


def test_prefill_plan_fp16_bias_and_ragged_rows():
    """A planned prefill launch on fp16 weights with a bias and M = 1000 (a
    ragged last row tile, odd row-tile count) through MixedLinear: bitwise
    equal to the plain launch, and within tolerance of the oracle."""
    from tilequant_amd.mixed_linear import MixedLinear

    m, k, n = 1000, 2048, 700
    n_tr, n_tc = -(-m // 64), k // 64
    rng = np.random.default_rng(5)
    mask = rng.random((n_tr, n_tc)) < 0.03
    mask[6] = True                        # one row tile entirely 16-bit
    mask[15, : n_tc // 2] = True          # the last (ragged, unpaired) row tile half 16-bit
    ids16 = np.flatnonzero(mask.ravel()).astype(np.int64)
    W = make_w(m, k, seed=9, dtype=torch.float16)
    pack = pack_weight_from_tile_ids(W, n_tr=n_tr, n_tc=n_tc, int8_tile_ids=torch.from_numpy(complement(ids16, n_tr * n_tc)),
                                     fp16_tile_ids=torch.from_numpy(ids16), cfg=SimpleNamespace(quant_style="gi", dtype_out="fp16"),
                                     tile_layout="mfma")
    bias = (torch.randn(m, generator=torch.Generator().manual_seed(10)) * 0.1).to(torch.float16)
    lin = MixedLinear(pack, bias.cuda(), SimpleNamespace(quant_style="gi", dtype_out="fp16"))
    x = make_x(n, k, seed=11, dtype=torch.float16)
    xd = x.cuda()
    y = lin(xd)
    plan = lin._plan[0]
    assert plan is not None and any(u >> 30 for u in plan.units.cpu().tolist())
    xq, sx = quantize_activation_tile_absmax(xd)
    y_plain = _gemm(pack, xd, xq, sx, bias=bias.cuda(), out_dtype=torch.float16)
    assert torch.equal(y.view(torch.int16), y_plain.view(torch.int16))
    op = _oracle_pack_any(W, ids16)
    xq_ref, sx_ref = nm.act_quant(values(x), False)
    rows = np.unique(np.r_[0:3, n - 3:n])
    acc, sab = _oracle_f64(pack, op, x[rows], xq_ref[rows], sx_ref)
    assert_gemm_close(y[rows], acc, sab, pack.n_tc, bias=bias.float().numpy())


def test_read_probe_reads_and_leaves_the_sink():
    """tq_read_probe (bench.py's plain-read context for the GEMM roofline):
    runs over sizes that are not a multiple of its 16 KiB block share (the
    clamped tail re-reads the last word) and, on data that does not fold to its
    constant, writes nothing."""
    from tilequant_amd import _native as nat

    for nbytes in (16, 16 * 1023, 16 * 4097, 25446144):
        buf = torch.zeros((nbytes,), dtype=torch.uint8, device="cuda")
        sink = torch.full((256,), 7, dtype=torch.int32, device="cuda")
        assert nat.lib().tq_read_probe(nat.ptr(buf), nbytes, nat.ptr(sink), nat.stream_handle(buf.device)) == 0
        torch.cuda.synchronize()
        assert bool((sink == 7).all()), nbytes
