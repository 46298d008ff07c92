"""torch-CPU restatement of the reference's CPU quantization branch.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): the checker in the
tests and the quantization leg of ``bench.py``'s CPU baseline.

The reference's ``quant_utils`` computes activation scales and codes with
torch ops when the input is not a CUDA bf16/fp16 tensor
(src/kernels/quant_utils.py:61-74 for the scales, :103-115 for the codes):
zero-pad K to whole 64-column tiles, absmax per tile over all rows, scale =
absmax / 127 in the input dtype (1.0 for an all-zero tile), codes =
clamp(round(x / scale), -127, 127) with the division in fp32.  These
functions are those steps, op for op, on CPU tensors.
"""
from __future__ import annotations

from typing import Tuple

import torch

INT8_MAX = 127.0
TILE = 64


def _tiles(x: torch.Tensor) -> torch.Tensor:
    n, k = x.shape
    n_tc = (k + TILE - 1) // TILE
    if k % TILE:
        padded = x.new_zeros((n, n_tc * TILE))
        padded[:, :k] = x
        x = padded
    return x.view(n, n_tc, TILE)


def act_tile_scales(x: torch.Tensor) -> torch.Tensor:
    """quant_utils.py:61-74: one fp32 scale per 64-column tile, over all rows."""
    max_abs = _tiles(x).abs().amax(dim=(0, 2))
    return torch.where(max_abs > 0, max_abs / INT8_MAX,
                       torch.ones_like(max_abs, dtype=torch.float32)).to(torch.float32).contiguous()


def act_codes_with_scales(x: torch.Tensor, sx: torch.Tensor) -> torch.Tensor:
    """quant_utils.py:103-115: int8 codes of x under the given tile scales."""
    n, k = x.shape
    t = _tiles(x)
    q = torch.clamp(torch.round(t / sx.view(1, t.shape[1], 1)), -127, 127).to(torch.int8)
    return q.view(n, -1)[:, :k].contiguous()


def act_quant(x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    sx = act_tile_scales(x)
    return act_codes_with_scales(x, sx), sx


def tensor_quant(x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """quant_utils.py:17-32 (quantize_activation_absmax; also the body of
    quantize_weight_tile_absmax, :138-148): one scale for the whole tensor,
    the reference's torch expressions op for op on a CPU tensor."""
    if x.numel() == 0:
        return torch.zeros_like(x, dtype=torch.int8), torch.tensor(1.0, dtype=torch.float32)
    max_abs = x.abs().max()
    if float(max_abs.item()) == 0.0:
        return torch.zeros_like(x, dtype=torch.int8), torch.tensor(1.0, dtype=torch.float32)
    sx = (max_abs / INT8_MAX).to(torch.float32)
    return torch.clamp(torch.round(x / sx), -127, 127).to(torch.int8), sx


def iaa_scales(src: torch.Tensor, col_imp_tiles: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """pack.py:132-159 op for op on CPU tensors: src [T, 64, 64] 16-bit INT8
    tiles, col_imp_tiles [T, 64] their columns' importances.  Returns the
    chosen scales [T] and the candidates' fp32 mean errors [3, T]."""
    max_abs = src.abs().amax(dim=(1, 2)).to(torch.float32)
    base = torch.where(max_abs == 0, torch.ones_like(max_abs, dtype=torch.float32),
                       (max_abs / 127.0).to(torch.float32))
    wm = col_imp_tiles.to(torch.float32).clamp_min(1e-8)[:, None, :]
    src_f = src.to(torch.float32)
    best_err = best_scales = None
    errs = []
    for m in torch.tensor([0.75, 1.00, 1.25], dtype=torch.float32):
        s = (base * m).clamp_min(1e-12)
        dq = torch.clamp(torch.round(src_f / s[:, None, None]), -127, 127) * s[:, None, None]
        err = ((dq - src_f) ** 2 * wm).mean(dim=(1, 2))
        errs.append(err)
        if best_err is None:
            best_err, best_scales = err, s
        else:
            better = err < best_err
            best_err = torch.where(better, err, best_err)
            best_scales = torch.where(better, s, best_scales)
    return best_scales.to(torch.float32), torch.stack(errs)
