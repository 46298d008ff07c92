"""Activation quantization dispatcher (mirror of src/kernels/quant_utils.py).

Same functions, arguments, return values and ``ValueError`` checks as the
reference (quant_utils.py:41-134, 152-164).  The reference computes on the CPU
with torch ops when handed a CPU tensor (quant_utils.py:64-74, 106-115); this
build has no CPU branch: the ops run the HIP kernels and raise for a tensor
that is not on a ROCm device.  Only ``tile_n == 64`` is supported (the only
value the reference's GPU kernels take).
"""
from __future__ import annotations

from typing import Tuple

import torch

from . import _native as nat
from .quantize_activation import (
    activation_tile_absmax_scales_64_fused,
    quantize_activation_tile_absmax_fused,
    quantize_activation_tile_absmax_two_level,
    quantize_activation_tile_with_scales_64_fused,
    two_level_ok,
)

INT8_MAX = 127.0
# The reference quantizes up to this many rows in one fused launch
# (quant_utils.py:127-133); larger inputs take scales + codes.
FUSED_MAX_ROWS = 128

_TENSOR_DTYPES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}   # TQ_DTYPE_*


def _quantize_tensor_absmax(x_fp: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """One absmax scale for the whole tensor (tq_quant_tensor_absmax): codes
    shaped like x_fp and a 0-dim float32 scale, both on x_fp's device."""
    nat.require_device(x_fp)
    code = _TENSOR_DTYPES.get(x_fp.dtype)
    if code is None:
        raise ValueError(f"expected a bfloat16, float16 or float32 tensor, got {x_fp.dtype}")
    q = torch.empty(x_fp.shape, device=x_fp.device, dtype=torch.int8)
    sx = torch.ones((), device=x_fp.device, dtype=torch.float32)
    n = x_fp.numel()
    if n == 0:
        return q, sx
    x = x_fp.contiguous()
    need = int(nat.lib().tq_quant_tensor_workspace_elems(n))
    ws = torch.empty(need, device=x.device, dtype=torch.float32) if need else None
    rc = nat.lib().tq_quant_tensor_absmax(nat.ptr(x), n, code, nat.ptr(q), nat.ptr(sx), nat.ptr(ws), need,
                                          nat.stream_handle(x.device))
    nat.check(rc, "tq_quant_tensor_absmax")
    return q, sx


def quantize_activation_absmax(x_fp: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """(codes, scale) with ONE scale for the whole tensor (quant_utils.py:17-32):
    scale = (max|x| / 127) in x's dtype, widened to float32 (1 for an empty or
    all-zero tensor); codes = clamp(round(x / scale), -127, 127), the quotient
    rounded to x's dtype as torch does for a 16-bit tensor."""
    return _quantize_tensor_absmax(x_fp)


def quantize_activation_per_tensor_absmax(x_fp: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Alias of quantize_activation_absmax (quant_utils.py:35-38)."""
    return quantize_activation_absmax(x_fp)


def quantize_weight_tile_absmax(w_fp_tile_64x64: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """(codes, scale) of one weight tile with one absmax scale
    (quant_utils.py:138-148): the same closed form as quantize_activation_absmax.
    (The load-time packer's per-tile scales are f32(a) / 127 unrounded,
    pack.py:125-130; this helper keeps the reference helper's own form.)"""
    return _quantize_tensor_absmax(w_fp_tile_64x64)


def _check_tile(x_fp: torch.Tensor, tile_n: int) -> None:
    if x_fp.dim() != 2:
        raise ValueError(f"Expected 2D activation tensor, got shape={tuple(x_fp.shape)}")
    if tile_n <= 0:
        raise ValueError(f"tile_n must be > 0, got {tile_n}")
    if tile_n != 64:
        raise ValueError(f"only tile_n=64 is supported by the gfx950 kernels, got {tile_n}")


def activation_tile_absmax_scales(x_fp: torch.Tensor, tile_n: int = 64) -> torch.Tensor:
    _check_tile(x_fp, tile_n)
    return activation_tile_absmax_scales_64_fused(x_fp)


def quantize_activation_tile_with_scales(x_fp: torch.Tensor, sx: torch.Tensor, tile_n: int = 64) -> torch.Tensor:
    _check_tile(x_fp, tile_n)
    n, k = x_fp.shape
    if k == 0:
        return torch.zeros_like(x_fp, dtype=torch.int8)
    n_tc = (k + tile_n - 1) // tile_n
    if sx.numel() != n_tc:
        raise ValueError(f"Scale length mismatch: got {sx.numel()}, expected {n_tc}")
    sx_work = sx.to(device=x_fp.device, dtype=torch.float32).contiguous()
    return quantize_activation_tile_with_scales_64_fused(x_fp, sx_work)


def quantize_activation_tile_absmax(x_fp: torch.Tensor, tile_n: int = 64) -> Tuple[torch.Tensor, torch.Tensor]:
    _check_tile(x_fp, tile_n)
    if int(x_fp.shape[0]) <= FUSED_MAX_ROWS:
        return quantize_activation_tile_absmax_fused(x_fp)
    if x_fp.is_cuda and two_level_ok(x_fp):
        return quantize_activation_tile_absmax_two_level(x_fp)   # the same two steps in two launches
    sx = activation_tile_absmax_scales(x_fp, tile_n=tile_n)
    return quantize_activation_tile_with_scales(x_fp, sx=sx, tile_n=tile_n), sx


def pad_to_multiple(W: torch.Tensor, multiple: int = 64) -> Tuple[torch.Tensor, int, int]:
    """Zero-pad a 2D weight to multiples of ``multiple`` (quant_utils.py:152-164)."""
    if W.dim() != 2:
        raise ValueError(f"Expected 2D weight tensor, got shape={tuple(W.shape)}")
    M, K = W.shape
    M_pad = -(-M // multiple) * multiple
    K_pad = -(-K // multiple) * multiple
    if (M_pad, K_pad) == (M, K):
        return W, M, K
    out = W.new_zeros((M_pad, K_pad))
    out[:M, :K] = W
    return out, M_pad, K_pad
