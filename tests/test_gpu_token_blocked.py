"""GPU parity of token-blocked activation codes (TQ_XQ_TOKEN_BLOCKED).

Bars: the token-blocked quantizer writes exactly the row-major codes of the
same input (and the oracle's), re-laid out, with zero padding rows and the
same scales; the GEMM reading token-blocked codes is bitwise equal to the GEMM
reading the same codes row-major (and within the oracle tolerance); MixedLinear
at 33..64 rows, which takes that path, is bitwise equal to its row-major
computation.
"""
from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from helpers import assert_gemm_close, complement, make_w, make_x, oracle_pack, uniform_fp16_ids, values
from oracle import native as onat
from oracle import numerics as nm
from tilequant_amd.gemm_rows_splitk_64x64 import gemm_mixed_rows_splitk
from tilequant_amd.mixed_linear import MixedLinear, MixedLinearGroup
from tilequant_amd.pack import pack_weight_from_tile_ids
from tilequant_amd.quant_utils import quantize_activation_tile_absmax
from tilequant_amd.quantize_activation import quantize_activation_token_blocked, token_blocked_elems

pytestmark = pytest.mark.gpu

CFG = SimpleNamespace(quant_style="gi", dtype_out="bf16")


def token_blocked(codes: np.ndarray) -> np.ndarray:
    """Row-major int8 codes [n, k] -> the token-blocked byte order: block
    (c, b) = rows 16 b .. 16 b + 15 of column tile c, 16-byte run 16 kq + j =
    row 16 b + j, columns 64 c + 16 kq .. + 15; rows past n zero."""
    n, k = codes.shape
    nb = -(-n // 16)
    padded = np.zeros((16 * nb, k), np.int8)
    padded[:n] = codes
    # [b, j, c, kq, byte] -> [c, b, kq, j, byte]
    return padded.reshape(nb, 16, k // 64, 4, 16).transpose(2, 0, 3, 1, 4).reshape(-1)


def test_relayout_helper_places_a_known_element():
    codes = np.zeros((20, 128), np.int8)
    codes[17, 64 + 16 * 2 + 5] = 7          # row 17 -> block b = 1, j = 1; column tile 1, kq = 2, byte 5
    flat = token_blocked(codes)
    nb = 2
    assert flat.size == 16 * nb * 128 and np.count_nonzero(flat) == 1
    assert flat[(1 * nb + 1) * 1024 + (16 * 2 + 1) * 16 + 5] == 7


@pytest.mark.parametrize("n", [1, 15, 16, 17, 33, 40, 63, 64])
@pytest.mark.parametrize("k", [64, 3072, 8192])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_token_blocked_codes_are_the_row_major_codes(n, k, dtype):
    x = make_x(n, k, seed=1000 + n + k, dtype=dtype)
    xd = x.cuda()
    qb, sb = quantize_activation_token_blocked(xd)
    q, s = quantize_activation_tile_absmax(xd)
    assert qb.numel() == token_blocked_elems(n, k) and qb.dim() == 1
    assert torch.equal(sb, s)
    assert np.array_equal(qb.cpu().numpy(), token_blocked(q.cpu().numpy()))
    q_ref, s_ref = nm.act_quant(values(x), dtype == torch.bfloat16)     # and the oracle's codes and scales
    assert np.array_equal(qb.cpu().numpy(), token_blocked(q_ref))
    assert np.array_equal(sb.cpu().numpy().view(np.uint32), np.asarray(s_ref, np.float32).view(np.uint32))


def test_token_blocked_quantizer_rejects_other_shapes():
    with pytest.raises(ValueError):
        quantize_activation_token_blocked(torch.zeros((65, 64), device="cuda", dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        quantize_activation_token_blocked(torch.zeros((4, 100), device="cuda", dtype=torch.bfloat16))


def _pack(m, k, frac, seed, dtype=torch.bfloat16, layout="mfma"):
    W = make_w(m, k, seed=seed, dtype=dtype)
    n_tr, n_tc = -(-m // 64), -(-k // 64)
    ids16 = uniform_fp16_ids(n_tr, n_tc, frac, seed=seed + 1) if frac > 0 else np.zeros(0, np.int64)
    ids8 = complement(ids16, n_tr * n_tc)
    pack = pack_weight_from_tile_ids(W, n_tr=n_tr, n_tc=n_tc, int8_tile_ids=torch.from_numpy(ids8),
                                     fp16_tile_ids=torch.from_numpy(ids16), cfg=CFG, tile_layout=layout)
    return W, pack, ids16


def _gemm(pack, xd, xq, sx, layout, bias=None, split_k=None):
    return gemm_mixed_rows_splitk(
        x_fp=xd, x_int8=xq, sx=sx, int8_tiles=pack.int8_tiles, int8_scales=pack.int8_scales,
        int8_tile_ids=pack.int8_tile_ids, int8_row_ptr=pack.int8_row_ptr, fp16_tiles=pack.fp16_tiles,
        fp16_tile_ids=pack.fp16_tile_ids, fp16_row_ptr=pack.fp16_row_ptr, M=pack.M_orig, K=pack.K_orig,
        n_tr=pack.n_tr, n_tc=pack.n_tc, out_dtype=xd.dtype, bias=bias, split_k=split_k,
        tile_layout=pack.tile_layout, x_int8_layout=layout)


@pytest.mark.parametrize("m,k,frac,n,split_k,dtype,tiles,bias", [
    (5120, 3072, 0.01, 64, None, torch.bfloat16, "mfma", False),    # Llama QKV at 64 tokens
    (3072, 8192, 0.01, 64, None, torch.bfloat16, "mfma", False),    # Down
    (16384, 3072, 0.01, 48, None, torch.bfloat16, "mfma", False),   # Gate/Up: whole-tile workgroups
    (3072, 3072, 0.05, 33, None, torch.float16, "row_major", True),
    (1024, 3072, 0.20, 17, None, torch.bfloat16, "mfma", True),     # two token blocks
    (3072, 3072, 0.01, 64, 4, torch.bfloat16, "mfma", False),       # explicit split-K
    (704, 1280, 0.30, 5, 2, torch.float16, "mfma", True),           # one block, ragged rows and outputs
    (3584, 18944, 0.10, 64, None, torch.bfloat16, "mfma", False),   # Qwen2.5-7B Down width
    # at 1-16 rows row-major codes run the LDS-staged kernel and token-blocked ones the split-K
    # kernel: the planner's choice between them must not change a bit
    (3584, 18944, 0.10, 4, None, torch.bfloat16, "mfma", False),    # Qwen2.5-7B Down, its schedule now
    (3072, 8192, 0.01, 16, None, torch.bfloat16, "mfma", False),    # Down staged up to 16 rows
    (5120, 3072, 0.01, 1, None, torch.bfloat16, "mfma", True),
    (16384, 3072, 0.01, 9, None, torch.float16, "mfma", False),     # whole-tile workgroups in both
])
def test_token_blocked_gemm_is_bitwise_the_row_major_gemm(m, k, frac, n, split_k, dtype, tiles, bias):
    W, pack, ids16 = _pack(m, k, frac, seed=m + k + n, dtype=dtype, layout=tiles)
    x = make_x(n, k, seed=n + 7, dtype=dtype)
    xd = x.cuda()
    b = (torch.randn((pack.M_orig,), generator=torch.Generator().manual_seed(3)) * 0.1).to(dtype).cuda() if bias else None
    xq, sx = quantize_activation_tile_absmax(xd)
    xb, sxb = quantize_activation_token_blocked(xd)
    y = _gemm(pack, xd, xq, sx, "row_major", b, split_k)
    yb = _gemm(pack, xd, xb, sxb, "token_blocked", b, split_k)
    assert torch.equal(yb, y)
    assert torch.equal(_gemm(pack, xd, xb, sxb, "token_blocked", b, split_k), yb)   # reproducible
    if dtype == torch.bfloat16 and not bias and m * k <= 16384 * 3072:
        op = oracle_pack(W, ids16)
        xq_ref, sx_ref = nm.act_quant(values(x))
        _, acc, sab = onat.gemm_mixed(xq_ref, sx_ref, values(x), op.int8_tiles, op.int8_scales, op.int8_tile_ids,
                                      op.int8_row_ptr, nm.bf16_bits_to_f32(op.fp16_tiles), op.fp16_tile_ids,
                                      op.fp16_row_ptr, pack.n_tr, pack.n_tc, pack.M_orig, pack.K_orig,
                                      want_f64=True)
        assert_gemm_close(yb, acc, sab, pack.n_tc)


def test_token_blocked_gemm_rejects_wrong_buffers():
    _, pack, _ = _pack(1024, 3072, 0.01, seed=5)
    xd = make_x(40, 3072, seed=9).cuda()
    xb, sxb = quantize_activation_token_blocked(xd)
    with pytest.raises(ValueError):
        _gemm(pack, xd, xb[:-16], sxb, "token_blocked")
    with pytest.raises(ValueError):
        _gemm(pack, xd, xb.view(-1, 3072), sxb, "token_blocked")
    with pytest.raises(ValueError):
        _gemm(pack, xd, xb, sxb, "column_major")
    x65 = make_x(65, 3072, seed=9).cuda()
    q65, s65 = quantize_activation_tile_absmax(x65)
    with pytest.raises(ValueError):
        _gemm(pack, x65, q65.reshape(-1), s65, "token_blocked")


@pytest.mark.parametrize("m,k,n,blocked", [
    (5120, 3072, 16, False), (5120, 3072, 17, True), (5120, 3072, 24, True), (5120, 3072, 32, True),
    (5120, 3072, 33, True), (5120, 3072, 48, True), (5120, 3072, 64, True),
    (3072, 8192, 8, False), (3072, 8192, 16, False), (3072, 8192, 17, True), (3072, 8192, 24, True),
    (3584, 18944, 4, True), (3584, 18944, 16, True)])
def test_mixed_linear_token_blocked_rows_are_bitwise_row_major(m, k, n, blocked):
    """MixedLinear quantizes token-blocked where the GEMM prefers it (17..64
    rows; fewer for rows of 256+ column tiles and for inputs whose codes do not
    fit LDS) -- through the cached eager launch below 32 rows, the
    shared-quantization path from 32 -- and its output is the row-major
    computation's bit for bit."""
    _, pack, _ = _pack(m, k, 0.01, seed=77)
    lin = MixedLinear(pack, None, CFG)
    assert lin.token_blocked_codes(n) == blocked
    x = make_x(n, k, seed=n).cuda()
    xq, sx = quantize_activation_tile_absmax(x)
    ref = _gemm(pack, x, xq, sx, "row_major")
    y = lin(x)                                    # eager: descriptor path below 32 rows
    assert torch.equal(y, ref)
    assert torch.equal(lin(x), ref)               # the cached descriptor again
    with torch.inference_mode():
        assert torch.equal(lin(x.view(1, n, k)).view(n, -1), ref)
    # captured in a HIP graph (the quantize + GEMM path), replayed
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        lin(x)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        yg = lin(x)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(yg, ref)


def test_projection_group_at_64_rows_equals_members():
    packs = [_pack(m, 3072, 0.01, seed=s)[1] for m, s in ((3072, 1), (1024, 2), (1024, 3))]
    members = [MixedLinear(p, None, CFG) for p in packs]
    group = MixedLinearGroup(members)
    x = make_x(64, 3072, seed=11).cuda()
    with torch.inference_mode():
        stacked = group.output_for(x, 0)
        outs = [m(x) for m in members]
    lo = 0
    for o in outs:
        assert torch.equal(stacked[:, lo:lo + o.shape[1]], o)
        lo += o.shape[1]
