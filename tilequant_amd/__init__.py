"""TileQuant mixed INT8/BF16 64x64-tile linear path, native to MI355X (gfx950).

Python host code mirrors the reference's module interface; the arithmetic runs
in hand-written HIP kernels behind the C ABI in ``include/tilequant.h``
(``_lib/libtilequant_hip.so``, built by ``tilequant_amd.build.build()``).

Module map (reference file -> this package):

  src/kernels/triton/quantize_activation.py    -> quantize_activation
  src/kernels/triton/gemm_rows_splitk_64x64.py -> gemm_rows_splitk_64x64
  src/kernels/quant_utils.py                   -> quant_utils
  src/kernels/pack.py                          -> pack
  src/kernels/mask_io.py                       -> mask_io
  src/models/mixed_linear.py                   -> mixed_linear
  src/models/rules.py                          -> rules
  src/quantization/types.py                    -> types
"""
from __future__ import annotations

__all__ = [
    "Pack",
    "MixedLinear",
    "MixedLinearGroup",
    "MixedLinearSlice",
    "fuse_projection_groups",
    "gemm_mixed_rows_splitk",
    "pack_weight_from_tile_ids",
    "quantize_activation_tile_absmax",
    "activation_tile_absmax_scales",
    "quantize_activation_tile_with_scales",
]

from .gemm_rows_splitk_64x64 import gemm_mixed_rows_splitk
from .mixed_linear import MixedLinear, MixedLinearGroup, MixedLinearSlice, fuse_projection_groups
from .pack import Pack, pack_weight_from_tile_ids
from .quant_utils import (
    activation_tile_absmax_scales,
    quantize_activation_tile_absmax,
    quantize_activation_tile_with_scales,
)
