"""GPU parity: activation quantization kernels vs the oracle (bit-exact codes and scales)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import make_x, values
from oracle import numerics as nm
from tilequant_amd import quant_utils
from tilequant_amd import _native as nat
from tilequant_amd.quantize_activation import (
    activation_tile_absmax_scales_64_fused,
    quantize_activation_tile_absmax_fused,
    quantize_activation_tile_absmax_two_level,
    quantize_activation_tile_with_scales_64_fused,
)

pytestmark = pytest.mark.gpu


def _check(x_cpu: torch.Tensor, q: torch.Tensor, sx: torch.Tensor):
    is_bf16 = x_cpu.dtype == torch.bfloat16
    q_ref, sx_ref = nm.act_quant(values(x_cpu), is_bf16)
    sx_got = sx.cpu().numpy()
    assert np.array_equal(sx_got.view(np.uint32), sx_ref.view(np.uint32)), "scales differ"
    q_got = q.cpu().numpy()
    bad = np.argwhere(q_got != q_ref)
    assert bad.size == 0, f"{len(bad)} codes differ, first at {bad[0].tolist()}"


@pytest.mark.parametrize("n", [1, 4, 16, 64, 128])
@pytest.mark.parametrize("k", [3072, 8192, 100, 64])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fused_vs_oracle(n, k, dtype):
    x = make_x(n, k, seed=1000 + n + k, dtype=dtype)
    q, sx = quantize_activation_tile_absmax_fused(x.cuda())
    _check(x, q, sx)


@pytest.mark.parametrize("n,k", [(129, 3072), (600, 1000), (4096, 3072), (8192, 3072), (4100, 8192)])
def test_scales_then_codes_vs_oracle(n, k):
    x = make_x(n, k, seed=2000 + n + k)
    xd = x.cuda()
    sx = activation_tile_absmax_scales_64_fused(xd)
    q = quantize_activation_tile_with_scales_64_fused(xd, sx)
    _check(x, q, sx)
    q2, sx2 = quant_utils.quantize_activation_tile_absmax(xd)
    assert torch.equal(q2, q) and torch.equal(sx2, sx)
    # the single-launch kernel gives the same bits at any size
    q3, sx3 = quantize_activation_tile_absmax_fused(xd)
    assert torch.equal(q3, q) and torch.equal(sx3, sx)


def test_strided_inputs():
    base = make_x(24, 3 * 512, seed=7)
    # row stride 1536 with every other row, start offset 5 (unaligned rows)
    xd = base.cuda()[::2, 5:5 + 1000]
    q, sx = quantize_activation_tile_absmax_fused(xd)
    _check(base[::2, 5:5 + 1000].contiguous(), q, sx)
    # column stride != 1
    src = make_x(300, 64, seed=8)
    xt = src.cuda().t()
    q, sx = quantize_activation_tile_absmax_fused(xt)
    _check(src.t().contiguous(), q, sx)
    sx2 = activation_tile_absmax_scales_64_fused(xt)
    assert torch.equal(sx2, sx)
    assert torch.equal(quantize_activation_tile_with_scales_64_fused(xt, sx2), q)


def test_every_bf16_absmax_gives_the_oracle_scale():
    # one 64-column tile per positive finite bf16 value: the tile's absmax is
    # that value (exhaustive over the scale's domain); other entries are
    # random fractions of it so the codes sweep the whole int8 range
    vals = np.arange(1, 0x7F80, dtype=np.uint16)
    a = nm.bf16_bits_to_f32(vals)
    rng = np.random.default_rng(0)
    frac = rng.uniform(-1, 1, size=(2, vals.size, 64)).astype(np.float32)
    x = nm.round_bf16(frac * a[None, :, None])
    x[0, :, 7] = a
    x = x.reshape(2, -1)
    xt = torch.from_numpy(nm.f32_to_bf16_bits(x).view(np.int16)).view(torch.bfloat16)
    q, sx = quantize_activation_tile_absmax_fused(xt.cuda())
    _check(xt, q, sx)
    sx2 = activation_tile_absmax_scales_64_fused(xt.cuda())
    assert torch.equal(sx2, sx)


def test_every_fp16_absmax_gives_the_oracle_scale():
    vals = np.arange(1, 0x7C00, dtype=np.uint16)
    a = vals.view(np.float16).astype(np.float32)
    rng = np.random.default_rng(1)
    x = (rng.uniform(-1, 1, size=(2, vals.size, 64)).astype(np.float32) * a[None, :, None]).astype(np.float16)
    x[0, :, 3] = a.astype(np.float16)
    xt = torch.from_numpy(x.reshape(2, -1))
    q, sx = quantize_activation_tile_absmax_fused(xt.cuda())
    _check(xt, q, sx)


def test_zero_and_tiny_tiles():
    x = torch.zeros((5, 256), dtype=torch.bfloat16)
    x[:, 64:128] = 2.5
    tiny = torch.tensor(2.0 ** -133, dtype=torch.float32).to(torch.bfloat16)
    x[0, 130] = tiny
    x[3, 140] = -tiny
    q, sx = quantize_activation_tile_absmax_fused(x.cuda())
    _check(x, q, sx)
    s = sx.cpu()
    assert s[0] == 1.0 and s[3] == 1.0 and s[2] == 0.0
    qq = q.cpu()
    assert torch.all(qq[:, :64] == 0) and qq[0, 130] == 127 and qq[3, 140] == -127 and qq[1, 131] == 127


def test_empty_inputs():
    x = torch.empty((0, 192), dtype=torch.bfloat16, device="cuda")
    q, sx = quantize_activation_tile_absmax_fused(x)
    assert q.shape == (0, 192) and torch.equal(sx.cpu(), torch.ones(3))
    q, sx = quantize_activation_tile_absmax_fused(torch.empty((4, 0), dtype=torch.bfloat16, device="cuda"))
    assert q.shape == (4, 0) and sx.numel() == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_exact_half_integer_quotients_round_half_even(dtype):
    # absmax 15.875 = 127/8 gives the scale 0.125 exactly; x = (k + 0.5) * 0.125
    # are exact in bf16 and fp16, so every x / s is an exact tie k + 0.5 that
    # must round to even (the reciprocal-multiply code path detects these)
    # each 64-column tile: 63 tie values and its own absmax 15.875
    x = np.zeros((2, 256), np.float32)
    for t, (k0, sign) in enumerate([(0, 1), (0, -1), (63, 1), (63, -1)]):
        k = np.arange(k0, k0 + 63, dtype=np.float32)
        x[0, 64 * t:64 * t + 63] = sign * (k + 0.5) * 0.125
        x[1, 64 * t + 63] = 15.875
    xt = torch.from_numpy(x).to(dtype)
    q, sx = quantize_activation_tile_absmax_fused(xt.cuda())
    _check(xt, q, sx)
    assert torch.all(sx.cpu() == 0.125)
    qq = q.cpu()
    assert int(qq[0, 0]) == 0 and int(qq[0, 1]) == 2 and int(qq[0, 2]) == 2      # 0.5->0, 1.5->2, 2.5->2
    assert int(qq[0, 64]) == 0 and int(qq[0, 65]) == -2 and int(qq[0, 128]) == 64  # -1.5->-2, 63.5->64
    sx2 = activation_tile_absmax_scales_64_fused(xt.cuda())
    assert torch.equal(quantize_activation_tile_with_scales_64_fused(xt.cuda(), sx2), q)


@pytest.mark.parametrize("n,k,dtype", [(513, 64, torch.bfloat16), (1000, 3072, torch.float16),
                                       (8192, 8192, torch.bfloat16), (4353, 1024, torch.float16),
                                       (777, 3136, torch.bfloat16), (20000, 192, torch.float16)])
def test_two_level_launch_equals_scales_then_codes(n, k, dtype):
    """tq_act_quant_two_level (the codes kernel reduces the absmax partials
    itself, two column tiles per workgroup) against the oracle and the
    two-call path, bitwise; odd tile counts (1, 3, 49) leave the last
    workgroup one tile, 20000 rows give 79 partials per column."""
    x = make_x(n, k, seed=3000 + n + k, dtype=dtype)
    xd = x.cuda()
    q, sx = quantize_activation_tile_absmax_two_level(xd)
    _check(x, q, sx)
    sx2 = activation_tile_absmax_scales_64_fused(xd)
    q2 = quantize_activation_tile_with_scales_64_fused(xd, sx2)
    assert torch.equal(q, q2) and torch.equal(sx, sx2)


def test_two_level_argument_errors():
    TQ_ERR_ALIGN, TQ_ERR_WORKSPACE = -3, -4   # include/tilequant.h
    lib = nat.lib()
    x = torch.zeros((600, 100), dtype=torch.bfloat16, device="cuda")
    q = torch.empty((600, 100), dtype=torch.int8, device="cuda")
    sx = torch.empty((2,), dtype=torch.float32, device="cuda")
    ws = torch.empty((1 << 14,), dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    # width not a multiple of 64
    assert lib.tq_act_quant_two_level(x.data_ptr(), 100, 0, 600, 100, q.data_ptr(), 100, sx.data_ptr(),
                                      ws.data_ptr(), ws.numel(), stream) == TQ_ERR_ALIGN
    x = torch.zeros((600, 128), dtype=torch.bfloat16, device="cuda")
    q = torch.empty((600, 128), dtype=torch.int8, device="cuda")
    # too small a workspace, and too few rows for the two-level scales
    assert lib.tq_act_quant_two_level(x.data_ptr(), 128, 0, 600, 128, q.data_ptr(), 128, sx.data_ptr(),
                                      ws.data_ptr(), 1, stream) == TQ_ERR_WORKSPACE
    assert lib.tq_act_quant_two_level(x.data_ptr(), 128, 0, 500, 128, q.data_ptr(), 128, sx.data_ptr(),
                                      ws.data_ptr(), ws.numel(), stream) == nat.TQ_ERR_ARG


def _tensor_case(shape, dtype, seed, scale=2.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype)


@pytest.mark.parametrize("shape,dtype", [
    ((64, 64), torch.bfloat16),        # quantize_weight_tile_absmax's tile
    ((4, 3072), torch.bfloat16),
    ((1,), torch.bfloat16),
    ((2, 3, 64), torch.float16),       # any rank
    ((1000, 1000), torch.float16),     # two-pass form (above one workgroup's 65536 elements)
    ((3000, 4096), torch.bfloat16),    # 12.3 M elements
    ((70000,), torch.float32),
])
def test_tensor_absmax_quant_matches_oracle(shape, dtype):
    """quantize_activation_absmax / _per_tensor_absmax / quantize_weight_tile_absmax
    (tq_quant_tensor_absmax) vs the oracle: codes and scale bitwise."""
    x = _tensor_case(shape, dtype, seed=sum(shape))
    name = {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}[dtype]
    q_ref, s_ref = nm.tensor_quant(x.float().numpy(), name)
    for fn in (quant_utils.quantize_activation_absmax, quant_utils.quantize_activation_per_tensor_absmax,
               quant_utils.quantize_weight_tile_absmax):
        q, s = fn(x.cuda())
        assert q.shape == x.shape and q.dtype == torch.int8 and s.dim() == 0 and s.dtype == torch.float32
        assert np.float32(s.item()).view(np.uint32) == np.float32(s_ref).view(np.uint32)
        assert np.array_equal(q.cpu().numpy(), q_ref)


@pytest.mark.parametrize("dtype,amax", [(torch.bfloat16, 100.0), (torch.bfloat16, 127.0), (torch.float16, 1000.0)])
def test_tensor_absmax_quant_every_value_of_a_range(dtype, amax):
    """Every bf16 / fp16 value in [-amax, amax] in one tensor (exact half-integer
    quotients included), contiguous and as a transposed view."""
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    v = (nm.bf16_bits_to_f32(bits) if dtype == torch.bfloat16 else bits.view(np.float16).astype(np.float32))
    v = np.unique(v[np.isfinite(v) & (np.abs(v) <= amax)])
    v = v[: (v.size // 8) * 8]
    x = torch.from_numpy(v).to(dtype)
    q_ref, s_ref = nm.tensor_quant(x.float().numpy(), "bf16" if dtype == torch.bfloat16 else "fp16")
    q, s = quant_utils.quantize_activation_absmax(x.cuda())
    assert s.item() == s_ref and np.array_equal(q.cpu().numpy(), q_ref)
    xt = x.view(8, -1).cuda().t()   # non-contiguous
    qt, st = quant_utils.quantize_activation_absmax(xt)
    assert st.item() == s_ref and np.array_equal(qt.cpu().numpy(), q_ref.reshape(8, -1).T)


def test_tensor_absmax_quant_zero_and_empty():
    for x in (torch.zeros((5, 64), dtype=torch.bfloat16), torch.zeros((0, 64), dtype=torch.bfloat16)):
        q, s = quant_utils.quantize_weight_tile_absmax(x.cuda())
        assert s.item() == 1.0 and q.shape == x.shape and int(q.abs().sum()) == 0
    with pytest.raises(ValueError):
        quant_utils.quantize_activation_absmax(torch.zeros(4, dtype=torch.int32, device="cuda"))
