"""Activation INT8 quantization launchers (HIP, gfx950).

Same names, arguments and return values as the reference's Triton launchers
(src/kernels/triton/quantize_activation.py:118-203); the kernels behind them
are ``tq_act_*`` in ``csrc/tq_act_quant.hip``.  One scale per 64-column tile,
taken over ALL rows of the call.
"""
from __future__ import annotations

from typing import Dict, Tuple

import torch

from . import _native as nat

_WORKSPACE: Dict[Tuple[int, int], torch.Tensor] = {}


def _absmax_workspace(x: torch.Tensor, n: int, k: int) -> torch.Tensor:
    """Per (device, stream) fp32 partial-max buffer, grown only (the analogue of
    the reference's per-stream split-K workspace, gemm_rows_splitk_64x64.py:193-215)."""
    need = int(nat.lib().tq_act_absmax_workspace_elems(n, k))
    dev = x.device
    key = (dev.index if dev.index is not None else torch.cuda.current_device(), nat.stream_handle(dev))
    ws = _WORKSPACE.get(key)
    if ws is None or ws.numel() < need:
        ws = torch.empty((max(need, 1 << 14),), device=dev, dtype=torch.float32)
        _WORKSPACE[key] = ws
    return ws


def _check_x(x_fp: torch.Tensor) -> None:
    if x_fp.dim() != 2:
        raise ValueError(f"Expected 2D activation tensor, got shape={tuple(x_fp.shape)}")
    nat.require_device(x_fp)
    nat.dtype_code(x_fp.dtype)


def quantize_activation_tile_absmax_fused(x_fp: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """absmax -> scale -> codes in one launch (reference :118-155)."""
    _check_x(x_fp)
    n, k = x_fp.shape
    if k == 0:
        return torch.empty_like(x_fp, dtype=torch.int8), torch.empty((0,), device=x_fp.device, dtype=torch.float32)
    n_tc = (int(k) + 63) // 64
    x_q = torch.empty((n, k), device=x_fp.device, dtype=torch.int8)
    sx = torch.empty((n_tc,), device=x_fp.device, dtype=torch.float32)
    rc = nat.lib().tq_act_quant_fused(
        nat.ptr(x_fp), x_fp.stride(0), x_fp.stride(1), nat.dtype_code(x_fp.dtype), int(n), int(k),
        nat.ptr(x_q), x_q.stride(0), nat.ptr(sx), nat.stream_handle(x_fp.device))
    nat.check(rc, "tq_act_quant_fused")
    return x_q, sx


def token_blocked_elems(n: int, k: int) -> int:
    """Bytes of token-blocked codes of n rows and k columns: 16-row blocks."""
    return 16 * ((int(n) + 15) // 16) * int(k)


def quantize_activation_token_blocked(x_fp: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """quantize_activation_tile_absmax_fused with the codes TOKEN-BLOCKED, the
    operand format of the 17..64-token GEMM: a flat int8 tensor of
    ``token_blocked_elems(n, k)`` bytes in which block (c, b) -- rows
    16 b .. 16 b + 15 of column tile c -- is one 1 KiB MFMA A operand (16-byte
    run 16 kq + j holds row 16 b + j, columns 64 c + 16 kq .. + 15; rows past n
    are zero).  Same scales and code values.  1 <= n <= 64, k a multiple of 64,
    rows 16-byte aligned with unit column stride."""
    _check_x(x_fp)
    n, k = (int(v) for v in x_fp.shape)
    if not 1 <= n <= 64 or k == 0 or k % 64:
        raise ValueError(f"token-blocked codes take 1..64 rows and a multiple of 64 columns, got {(n, k)}")
    x_q = torch.empty((token_blocked_elems(n, k),), device=x_fp.device, dtype=torch.int8)
    sx = torch.empty((k // 64,), device=x_fp.device, dtype=torch.float32)
    rc = nat.lib().tq_act_quant_token_blocked(nat.ptr(x_fp), x_fp.stride(0), nat.dtype_code(x_fp.dtype), n, k,
                                              nat.ptr(x_q), nat.ptr(sx), nat.stream_handle(x_fp.device))
    nat.check(rc, "tq_act_quant_token_blocked")
    return x_q, sx


def activation_tile_absmax_scales_64_fused(x_fp: torch.Tensor) -> torch.Tensor:
    """Scales only, over all rows (reference :158-176)."""
    _check_x(x_fp)
    n, k = x_fp.shape
    if k == 0:
        return torch.empty((0,), device=x_fp.device, dtype=torch.float32)
    n_tc = (int(k) + 63) // 64
    sx = torch.empty((n_tc,), device=x_fp.device, dtype=torch.float32)
    ws = _absmax_workspace(x_fp, int(n), int(k))
    rc = nat.lib().tq_act_absmax_scales(
        nat.ptr(x_fp), x_fp.stride(0), x_fp.stride(1), nat.dtype_code(x_fp.dtype), int(n), int(k),
        nat.ptr(sx), nat.ptr(ws), ws.numel(), nat.stream_handle(x_fp.device))
    nat.check(rc, "tq_act_absmax_scales")
    return sx


def quantize_activation_tile_with_scales_64_fused(x_fp: torch.Tensor, sx: torch.Tensor) -> torch.Tensor:
    """Codes from given per-tile scales (reference :179-203)."""
    _check_x(x_fp)
    nat.require_device(sx)
    n, k = x_fp.shape
    if k == 0:
        return torch.empty_like(x_fp, dtype=torch.int8)
    n_tc = (int(k) + 63) // 64
    if sx.numel() != n_tc or sx.dtype != torch.float32 or not sx.is_contiguous():
        raise ValueError(f"sx must be a contiguous float32 tensor of {n_tc} scales")
    x_q = torch.empty((n, k), device=x_fp.device, dtype=torch.int8)
    rc = nat.lib().tq_act_quant_with_scales(
        nat.ptr(x_fp), x_fp.stride(0), x_fp.stride(1), nat.dtype_code(x_fp.dtype), int(n), int(k),
        nat.ptr(sx), nat.ptr(x_q), x_q.stride(0), nat.stream_handle(x_fp.device))
    nat.check(rc, "tq_act_quant_with_scales")
    return x_q


def quantize_activation_tile_absmax_two_level(x_fp: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Scales over all rows, then codes, for inputs of more than 512 rows in
    two launches (``tq_act_quant_two_level``): bitwise the result of
    ``activation_tile_absmax_scales_64_fused`` followed by
    ``quantize_activation_tile_with_scales_64_fused`` (the reference's
    two-kernel path, quant_utils.py:119-134).  Needs unit column stride,
    16-byte aligned rows and a width that is a multiple of 64
    (``two_level_ok``)."""
    _check_x(x_fp)
    n, k = x_fp.shape
    n_tc = int(k) // 64
    x_q = torch.empty((n, k), device=x_fp.device, dtype=torch.int8)
    sx = torch.empty((n_tc,), device=x_fp.device, dtype=torch.float32)
    ws = _absmax_workspace(x_fp, int(n), int(k))
    rc = nat.lib().tq_act_quant_two_level(
        nat.ptr(x_fp), x_fp.stride(0), nat.dtype_code(x_fp.dtype), int(n), int(k), nat.ptr(x_q), x_q.stride(0),
        nat.ptr(sx), nat.ptr(ws), ws.numel(), nat.stream_handle(x_fp.device))
    nat.check(rc, "tq_act_quant_two_level")
    return x_q, sx


def two_level_ok(x_fp: torch.Tensor) -> bool:
    """Whether ``quantize_activation_tile_absmax_two_level`` takes this input."""
    n, k = x_fp.shape
    return (int(n) > 512 and int(k) > 0 and int(k) % 64 == 0 and x_fp.stride(1) == 1 and x_fp.stride(0) % 8 == 0
            and x_fp.data_ptr() % 16 == 0)
