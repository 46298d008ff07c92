"""GPU parity at the module level: MixedLinear forward (2D/3D, chunked prefill
with whole-input scales), projection groups, IAA packing."""
from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from helpers import assert_gemm_close, complement, make_w, make_x, oracle_pack, uniform_fp16_ids, values
from oracle import native as onat
from oracle import numerics as nm
from tilequant_amd.mixed_linear import MixedLinear, fuse_projection_groups
from tilequant_amd.pack import pack_weight_from_tile_ids

pytestmark = pytest.mark.gpu


def _linear(m, k, frac, seed, cfg, bias=False, layout="mfma"):
    W = make_w(m, k, seed=seed)
    n_tr, n_tc = -(-m // 64), -(-k // 64)
    ids16 = uniform_fp16_ids(n_tr, n_tc, frac, seed=seed + 1)
    pack = pack_weight_from_tile_ids(W, n_tr=n_tr, n_tc=n_tc,
                                     int8_tile_ids=torch.from_numpy(complement(ids16, n_tr * n_tc)),
                                     fp16_tile_ids=torch.from_numpy(ids16), cfg=cfg, tile_layout=layout)
    b = (torch.randn(m, generator=torch.Generator().manual_seed(seed)) * 0.1).to(torch.bfloat16) if bias else None
    return MixedLinear(pack, b.cuda() if b is not None else None, cfg), W, ids16, b


def _expected(W, ids16, x_cpu, sx_ref=None):
    op = oracle_pack(W, ids16)
    xv = values(x_cpu)
    if sx_ref is None:
        xq, sx = nm.act_quant(xv)
    else:
        sx = sx_ref
        xq = nm.act_quant_codes(xv, sx)
    _, acc, sab = onat.gemm_mixed(xq, sx, xv, op.int8_tiles, op.int8_scales, op.int8_tile_ids, op.int8_row_ptr,
                                  nm.bf16_bits_to_f32(op.fp16_tiles), op.fp16_tile_ids, op.fp16_row_ptr,
                                  op.n_tr, op.n_tc, op.M_orig, op.K_orig, want_f64=True)
    return acc, sab, op.n_tc


def test_forward_2d_and_3d():
    cfg = SimpleNamespace(quant_style="gi", dtype_out="bf16")
    lin, W, ids16, b = _linear(512, 1024, 0.02, 10, cfg, bias=True)
    x = make_x(8, 1024, seed=11)
    y2 = lin(x.cuda())
    acc, sab, n_tc = _expected(W, ids16, x)
    assert y2.dtype == torch.bfloat16 and y2.shape == (8, 512)
    assert_gemm_close(y2, acc, sab, n_tc, bias=values(b))
    y3 = lin(x.cuda().view(2, 4, 1024))
    assert y3.shape == (2, 4, 512) and torch.equal(y3.view(8, 512), y2)


def test_default_out_dtype_is_fp16_like_reference():
    lin, _, _, _ = _linear(128, 128, 0.1, 20, SimpleNamespace(quant_style="gi"))
    assert lin(make_x(2, 128).cuda()).dtype == torch.float16


def test_chunked_rows_use_whole_input_scales():
    # activation_row_chunk_size smaller than N: the scale is taken over ALL rows
    # before chunking (mixed_linear.py:240-250)
    cfg = SimpleNamespace(quant_style="gi", dtype_out="bf16", activation_row_chunk_size=64)
    lin, W, ids16, _ = _linear(256, 512, 0.05, 30, cfg)
    x = make_x(200, 512, seed=31)
    x[150:, :64] *= 50                     # the last chunk holds the first tile's absmax
    y = lin(x.cuda())
    sx_all = nm.act_tile_scales(values(x))
    acc, sab, n_tc = _expected(W, ids16, x, sx_ref=sx_all)
    assert_gemm_close(y, acc, sab, n_tc)
    # per-chunk scales would differ measurably in the first tile's rows
    acc_bad, _, _ = _expected(W, ids16, x[:64])
    assert not np.allclose(acc_bad, acc[:64], rtol=1e-3)


def test_prefill_8192_rows_two_chunks():
    cfg = SimpleNamespace(quant_style="gi", dtype_out="bf16")
    lin, W, ids16, _ = _linear(256, 3072, 0.05, 40, cfg)
    x = make_x(8192, 3072, seed=41)
    y = lin(x.cuda())
    # check a sample of rows from both chunks against the oracle with whole-input scales
    sx_all = nm.act_tile_scales(values(x))
    rows = np.r_[0:8, 4090:4100, 8184:8192]
    acc, sab, n_tc = _expected(W, ids16, x[rows], sx_ref=sx_all)
    assert_gemm_close(y[rows], acc, sab, n_tc)


def test_projection_groups_equal_members_bitwise():
    cfg = SimpleNamespace(quant_style="gi", dtype_out="bf16")

    class Attn(torch.nn.Module):
        pass

    parent = Attn()
    members = {}
    for i, (name, m) in enumerate((("q_proj", 512), ("k_proj", 128), ("v_proj", 128))):
        lin, _, _, _ = _linear(m, 768, 0.05, 50 + i, cfg)
        setattr(parent, name, lin)
        members[name] = lin
    for n in (1, 4, 40):
        x = make_x(n, 768, seed=60 + n).cuda()
        want = {name: members[name](x) for name in members}
        solo = Attn()
        for name, lin in members.items():
            setattr(solo, name, lin)
        assert fuse_projection_groups(solo) == 1
        with torch.inference_mode():
            got = {name: getattr(solo, name)(x) for name in members}
        for name in members:
            assert torch.equal(got[name], want[name]), name


@pytest.mark.parametrize("dtype,layout", [(torch.bfloat16, "row_major"), (torch.float16, "mfma")])
def test_iaa_packing_matches_oracle(dtype, layout):
    """IAA scale search (pack.py:132-159) against oracle.packing.iaa_scales
    (float64 error sums, the exact selection): the chosen scale bitwise on
    every tile whose two best candidates' errors differ by more than the
    kernel's fp32 summation bound (16 sequential terms + a 64-lane butterfly +
    4 waves: ~25 * 2^-24 of the sum; 4e-6 relative used), the codes bitwise for
    the chosen scales.  Includes an all-zero tile (exact three-way tie: first
    candidate) and zero importances (clamped to 1e-8)."""
    from oracle import numerics as nm
    from oracle import packing as opk

    m, k = 1024, 4096
    n_tr, n_tc = m // 64, k // 64
    g = torch.Generator().manual_seed(70)
    W = (torch.randn((m, k), generator=g) * 0.02).to(dtype)
    W[:64, :64] = 0
    imp = torch.rand(k, generator=g) * 3
    imp[64:128] = 0
    ids16 = uniform_fp16_ids(n_tr, n_tc, 0.1, seed=71)
    ids16 = ids16[ids16 != 0]             # keep the zero tile INT8
    ids8 = complement(ids16, n_tr * n_tc)
    cfg = SimpleNamespace(quant_style="iaa", dtype_out="bf16")
    pack = pack_weight_from_tile_ids(W, n_tr=n_tr, n_tc=n_tc, int8_tile_ids=torch.from_numpy(ids8),
                                     fp16_tile_ids=torch.from_numpy(ids16), iaa_col_importance=imp, cfg=cfg,
                                     tile_layout=layout)
    src = W.float().view(n_tr, 64, n_tc, 64).permute(0, 2, 1, 3)[torch.from_numpy(ids8 // n_tc),
                                                                   torch.from_numpy(ids8 % n_tc)].numpy()
    col_imp = imp.view(n_tc, 64)[torch.from_numpy(ids8 % n_tc)].numpy()
    want_s, errs = opk.iaa_scales(src, col_imp)
    got_s = pack.int8_scales.cpu().numpy()
    srt = np.sort(errs, axis=0)
    band = (srt[1] - srt[0]) <= 4e-6 * srt[1]
    assert np.array_equal(got_s[~band].view(np.uint32), want_s[~band].view(np.uint32))
    assert band.sum() <= len(ids8) // 100
    if band.any():   # inside the band: one of the two tied candidates
        cands = np.stack([np.maximum(nm.weight_tile_scales(src) * np.float32(mu), np.float32(1e-12))
                          for mu in opk.IAA_MULTS]).astype(np.float32)
        two = np.argsort(errs, axis=0)[:2]
        ok = (got_s == cands[two[0], np.arange(len(ids8))]) | (got_s == cands[two[1], np.arange(len(ids8))])
        assert ok[band].all()
    assert got_s[0] == np.float32(0.75)   # the zero tile
    tiles = pack.int8_tiles.cpu().numpy()
    if layout == "mfma":
        tiles = opk.from_mfma_int8(tiles)
    assert np.array_equal(tiles, nm.quant_codes(src, got_s[:, None, None]))


def test_fused_decode_option_is_bitwise_identical():
    cfg = SimpleNamespace(quant_style="gi", dtype_out="bf16", fused_decode=False)
    lin, W, ids16, _ = _linear(1024, 3072, 0.01, 80, cfg, bias=True)
    lin_f = MixedLinear(lin.to_pack(), lin.bias.detach(), SimpleNamespace(quant_style="gi", dtype_out="bf16",
                                                                           fused_decode=True))
    lin_a = MixedLinear(lin.to_pack(), lin.bias.detach(), SimpleNamespace(quant_style="gi", dtype_out="bf16"))
    for n in (1, 2, 3, 4, 16):
        x = make_x(n, 3072, seed=81 + n).cuda()
        y = lin(x)
        assert torch.equal(lin_f(x), y)
        assert torch.equal(lin_a(x), y)   # "auto": fused up to 4 rows here (narrow input, 64 workgroups)
    assert lin_a._fused_rows_for_cfg() == 4
    down, _, _, _ = _linear(256, 8192, 0.01, 82, SimpleNamespace(quant_style="gi", dtype_out="bf16"))
    assert down._fused_rows_for_cfg() == 4   # 8192 columns, 16 workgroups: fused up to 4 rows
    wide, _, _, _ = _linear(256, 12288, 0.01, 83, SimpleNamespace(quant_style="gi", dtype_out="bf16"))
    assert wide._fused_rows_for_cfg() == 2   # wider: quantization repeated per workgroup is too dear


@pytest.mark.parametrize("n", [2, 3, 4])
def test_down_width_fused_by_auto_policy_eager_and_graph(n):
    """Llama-3.2-3B Down width (3072 x 8192, 192 workgroups): the "auto" policy
    runs quantize + GEMM as one launch up to 4 rows (lane quantization, 16
    waves); eager calls, the cached descriptor, inference mode and HIP-graph
    replays are all bitwise the two-launch module's output, and within the
    oracle's tolerance."""
    off = SimpleNamespace(quant_style="gi", dtype_out="bf16", fused_decode=False)
    ref_lin, W, ids16, _ = _linear(3072, 8192, 0.01, 990 + n, off, bias=True)
    auto = MixedLinear(ref_lin.to_pack(), ref_lin.bias.detach(), SimpleNamespace(quant_style="gi", dtype_out="bf16"))
    assert auto._fused_rows_for_cfg() == 4
    x_cpu = make_x(n, 8192, seed=991 + n)
    x = x_cpu.cuda()
    ref = ref_lin(x)
    assert torch.equal(auto(x), ref)
    assert torch.equal(auto(x), ref)                      # cached descriptor
    with torch.inference_mode():
        assert torch.equal(auto(x.view(1, n, 8192)).view(n, -1), ref)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        auto(x)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        yg = auto(x)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(yg, ref)
        assert torch.equal(ref_lin(x), ref)               # eager work between replays
    acc, sab, n_tc = _expected(W, ids16, x_cpu)
    assert_gemm_close(ref, acc, sab, n_tc, bias=values(ref_lin.bias.detach().cpu()))


@pytest.mark.parametrize("fused_mode", ["auto", False, True])
@pytest.mark.parametrize("bias,dtype_out", [(False, "bf16"), (True, "fp16")])
def test_cached_launch_path_equals_uncached_calls(fused_mode, bias, dtype_out):
    """Eager decode-size forwards run through a cached tq_linear_forward
    descriptor: bitwise equal to the quantizer + GEMM entry points called
    directly, on the first call and on cache hits, after the input moves to
    another buffer, on another stream, and after .to() rebuilds the tensors."""
    from tilequant_amd.gemm_rows_splitk_64x64 import gemm_mixed_rows_splitk, linear_mixed_fused
    from tilequant_amd.quant_utils import quantize_activation_tile_absmax

    cfg = SimpleNamespace(quant_style="gi", dtype_out=dtype_out, fused_decode=fused_mode)
    lin, W, ids16, b = _linear(640, 3072, 0.02, seed=71, cfg=cfg, bias=bias)
    out_dtype = torch.float16 if dtype_out == "fp16" else torch.bfloat16

    def direct(x):
        bias_t = lin._out_bias(out_dtype)
        if 0 < x.shape[0] <= lin._fused_rows_for_cfg():
            return linear_mixed_fused(x_fp=x, int8_tiles=lin.int8_tiles, int8_scales=lin.int8_scales,
                                      int8_tile_ids=lin.int8_tile_ids, int8_row_ptr=lin.int8_row_ptr,
                                      fp16_tiles=lin.fp16_tiles, fp16_tile_ids=lin.fp16_tile_ids,
                                      fp16_row_ptr=lin.fp16_row_ptr, M=lin.M_orig, K=lin.K_orig, n_tr=lin.n_tr,
                                      n_tc=lin.n_tc, out_dtype=out_dtype, bias=bias_t, tile_layout=lin.tile_layout)
        xq, sx = quantize_activation_tile_absmax(x)
        return gemm_mixed_rows_splitk(x_fp=x, x_int8=xq, sx=sx, int8_tiles=lin.int8_tiles,
                                      int8_scales=lin.int8_scales, int8_tile_ids=lin.int8_tile_ids,
                                      int8_row_ptr=lin.int8_row_ptr, fp16_tiles=lin.fp16_tiles,
                                      fp16_tile_ids=lin.fp16_tile_ids, fp16_row_ptr=lin.fp16_row_ptr, M=lin.M_orig,
                                      K=lin.K_orig, n_tr=lin.n_tr, n_tc=lin.n_tc, out_dtype=out_dtype, bias=bias_t,
                                      tile_layout=lin.tile_layout)

    for n in (1, 2, 4, 7, 16, 31):
        for rep in range(3):
            x = make_x(n, 3072, seed=100 * n + rep).cuda()
            y = lin(x)
            assert y.dtype == out_dtype and torch.equal(y, direct(x)), (n, rep)
        assert sum(1 for key in lin._launches if key[0] == n) == 1   # one descriptor per row count
    x = make_x(4, 3072, seed=5).cuda()
    ref = direct(x)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        y_side = lin(x)
    torch.cuda.current_stream().wait_stream(side)
    assert torch.equal(y_side, ref)
    before = len(lin._launches)
    assert before > 0
    lin.to(torch.device("cuda", 0))   # _apply rebuilds nothing here, but the cache is dropped
    assert len(lin._launches) == 0
    assert torch.equal(lin(x), ref) and torch.equal(lin(x.view(1, 4, 3072)).view(4, -1), ref)


@pytest.mark.parametrize("dtype_out", ["bf16", "fp16"])
def test_cached_launch_sees_in_place_bias_updates(dtype_out):
    """An in-place bias update between two eager decode calls reaches the
    cached launch path (its descriptor may hold a converted copy of the bias:
    fp16 outputs from a bf16 bias), exactly as the uncached path sees it."""
    cfg = SimpleNamespace(quant_style="gi", dtype_out=dtype_out)
    lin, W, ids16, b = _linear(256, 512, 0.05, 60, cfg, bias=True)
    x = make_x(4, 512, seed=61).cuda()
    y0 = lin(x)
    with torch.no_grad():
        lin.bias.data.copy_(lin.bias.data * -2 + 1)
    y1 = lin(x)                       # cached path, same descriptor key but a new bias version
    out_dtype = torch.bfloat16 if dtype_out == "bf16" else torch.float16
    xq, sx = _codes(x)
    ref = lin._gemm_bias(x_fp=x, x_int8=xq, sx=sx)   # uncached quantize + GEMM with the current bias
    assert not torch.equal(y1, y0) and torch.equal(y1, ref) and y1.dtype == out_dtype
    assert len(lin._launches) <= 2


def _codes(x):
    from tilequant_amd.quant_utils import quantize_activation_tile_absmax

    return quantize_activation_tile_absmax(x)
