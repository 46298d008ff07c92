"""Drop-in ``MixedLinear`` module (mirror of src/models/mixed_linear.py).

Same constructor, nine persistent buffers, ``forward``/``to_pack`` semantics,
projection groups and sibling-activation cache as the reference
(mixed_linear.py:24-392):

* ``forward`` accepts [N, K] or [B, T, K]; inputs of up to
  ``activation_row_chunk_size`` rows are quantized and multiplied in one
  call, larger inputs get scales over the WHOLE input and are then quantized
  and multiplied in row chunks that write straight into one output
  (mixed_linear.py:229-250).  The default chunk is 16384 rows (the
  reference's is 4096): the INT8 copy of even a 16384 x 18944 input is 310 MB,
  small against 288 GB of HBM, and one GEMM launch over a whole 8192-token
  prefill fills the GPU better than two (measured 16% faster per layer).
  Chunking never changes the output: the scales are over the whole input
  either way and rows are independent.
* Q/K/V and Gate/Up siblings can be stacked into one ``MixedLinearGroup``
  (one quantization + one GEMM per group), each member served a column slice.

Decode-sized inputs can run quantization and GEMM as one launch
(``linear_mixed_fused``), bit-identical to the two-launch path: every GEMM
workgroup quantizes the whole activation into LDS while its weights stream
in.  That saves a launch (~2.5 us on MI355X) but repeats the quantization in
every workgroup, so it pays off only for very few rows.  ``cfg.fused_decode``
selects it: ``None`` / ``"auto"`` (default) for inputs of at most
``FUSED_AUTO_MAX_ROWS`` rows (``FUSED_AUTO_NARROW_ROWS`` for narrow inputs
whose grid fits the CUs once), ``True`` for every size the fused launch takes
(at most 16 rows, fewer for very wide inputs), ``False`` never.

The extra state records the packed tiles' storage order (``tile_layout``) so a
``state_dict`` round trip keeps it.
"""
from __future__ import annotations

import weakref
from dataclasses import dataclass
from typing import Any, Dict, Optional, Tuple

import torch
import torch.nn as nn

from .gemm_rows_splitk_64x64 import fused_max_tokens, gemm_mixed_rows_splitk, linear_mixed_fused
from .pack import Pack, concat_packs_along_rows
from .quant_utils import (
    activation_tile_absmax_scales,
    quantize_activation_tile_absmax,
    quantize_activation_tile_with_scales,
)

DEFAULT_ACTIVATION_ROW_CHUNK_SIZE = 16384
# Rows up to which cfg.fused_decode = "auto" fuses quantization into the GEMM
# (measured on MI355X: 1 row saves ~2 us per projection, 4 rows break even).
FUSED_AUTO_MAX_ROWS = 2
# ... and up to this many rows when the repeated quantization is cheap: inputs
# of at most FUSED_AUTO_NARROW_K columns whose decode grid (four workgroups
# per 64-row output tile) gives no CU a second workgroup.  At 4 rows on MI355X
# the O projection (3072 x 3072, 192 workgroups) runs fused in 7.4-7.5 us
# instead of 7.8-8.1 us for quantize + GEMM; Q/K/V (320 workgroups), Gate/Up
# (1024) and Down (8192 columns) are slower fused.
FUSED_AUTO_NARROW_ROWS = 4
FUSED_AUTO_NARROW_K = 4096


def _device_cus(device: torch.device) -> int:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    cus = _CU_COUNT.get(idx)
    if cus is None:
        cus = _CU_COUNT[idx] = int(torch.cuda.get_device_properties(idx).multi_processor_count)
    return cus


_CU_COUNT: Dict[int, int] = {}
# Sibling projections reuse one activation quantization for inputs of at least
# this many rows (mixed_linear.py:20-21).
ACTIVATION_QUANT_CACHE_MIN_ROWS = 32


@dataclass
class _ActivationQuantCacheEntry:
    source_ref: "weakref.ReferenceType[torch.Tensor]"
    signature: Tuple[Any, ...]
    consumers: set
    x_int8: torch.Tensor
    sx: torch.Tensor


# One inference-only entry per (device, stream): Q/K/V or Gate/Up siblings
# that see the same activation tensor reuse its codes and scales.
_ACTIVATION_QUANT_CACHE: Dict[Tuple[int, int], _ActivationQuantCacheEntry] = {}


def _cfg_get(cfg: Any, key: str, default=None):
    if isinstance(cfg, dict):
        return cfg.get(key, default)
    return getattr(cfg, key, default)


def _activation_version(x: torch.Tensor) -> Optional[int]:
    try:
        return int(x._version)
    except RuntimeError:  # inference tensors have no version counter
        return None


def _quantize_shared_activation(source: torch.Tensor, x_work: torch.Tensor, tile_n: int,
                                consumer_id: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Quantize ``x_work``, reusing a sibling's result for the same activation
    (mixed_linear.py:54-111)."""
    if int(x_work.shape[0]) < ACTIVATION_QUANT_CACHE_MIN_ROWS or not (
        torch.is_inference_mode_enabled() and x_work.is_cuda
    ):
        return quantize_activation_tile_absmax(x_work, tile_n=tile_n)
    slot = (int(x_work.device.index or 0), int(torch.cuda.current_stream(x_work.device).cuda_stream))
    signature = (int(x_work.data_ptr()), int(x_work.storage_offset()), tuple(x_work.shape),
                 tuple(x_work.stride()), x_work.dtype, int(tile_n), _activation_version(source))
    cached = _ACTIVATION_QUANT_CACHE.get(slot)
    if (cached is not None and cached.source_ref() is source and cached.signature == signature
            and consumer_id not in cached.consumers):
        cached.consumers.add(consumer_id)
        return cached.x_int8, cached.sx
    # drop the old entry first so an unrelated activation is not kept alive
    _ACTIVATION_QUANT_CACHE.pop(slot, None)
    x_int8, sx = quantize_activation_tile_absmax(x_work, tile_n=tile_n)
    try:
        def evict(dead):
            cur = _ACTIVATION_QUANT_CACHE.get(slot)
            if cur is not None and cur.source_ref is dead:
                _ACTIVATION_QUANT_CACHE.pop(slot, None)

        ref = weakref.ref(source, evict)
    except TypeError:
        return x_int8, sx
    _ACTIVATION_QUANT_CACHE[slot] = _ActivationQuantCacheEntry(ref, signature, {consumer_id}, x_int8, sx)
    return x_int8, sx


_BUFFERS = ("int8_tiles", "int8_scales", "int8_tile_ids", "int8_row_ptr", "int8_row_indices",
            "fp16_tiles", "fp16_tile_ids", "fp16_row_ptr", "fp16_row_indices")


class MixedLinear(nn.Module):
    def __init__(self, pack: Pack, bias: Optional[torch.Tensor], cfg: Any):
        super().__init__()
        self.cfg = cfg
        self.M_orig = int(pack.M_orig)
        self.K_orig = int(pack.K_orig)
        self.M = int(pack.M)
        self.K = int(pack.K)
        self.tile_m = int(pack.tile_m)
        self.tile_n = int(pack.tile_n)
        self.n_tr = int(pack.n_tr)
        self.n_tc = int(pack.n_tc)
        self.tile_layout = str(getattr(pack, "tile_layout", "row_major"))
        for name in _BUFFERS:
            self.register_buffer(name, getattr(pack, name), persistent=True)
        if bias is not None:
            self.bias = nn.Parameter(bias.detach().clone(), requires_grad=False)
        else:
            self.register_parameter("bias", None)

    # the tile storage order travels with the state_dict
    def get_extra_state(self):
        return {"tile_layout": self.tile_layout}

    def set_extra_state(self, state):
        if isinstance(state, dict) and "tile_layout" in state:
            self.tile_layout = str(state["tile_layout"])

    def to_pack(self) -> Pack:
        return Pack(M_orig=self.M_orig, K_orig=self.K_orig, M=self.M, K=self.K, tile_m=self.tile_m,
                    tile_n=self.tile_n, n_tr=self.n_tr, n_tc=self.n_tc,
                    **{name: getattr(self, name) for name in _BUFFERS}, tile_layout=self.tile_layout)

    def _out_dtype(self) -> torch.dtype:
        dtype_out = _cfg_get(self.cfg, "dtype_out", "fp16")
        return torch.bfloat16 if dtype_out in ("bf16", torch.bfloat16) else torch.float16

    def _activation_row_chunk_size(self) -> int:
        return max(1, int(_cfg_get(self.cfg, "activation_row_chunk_size", DEFAULT_ACTIVATION_ROW_CHUNK_SIZE)))

    def _out_bias(self, out_dtype: torch.dtype) -> Optional[torch.Tensor]:
        bias = self.bias
        if bias is None:
            return None
        if bias.dtype != out_dtype or not bias.is_contiguous():
            bias = bias.to(dtype=out_dtype).contiguous()
        return bias

    def _gemm_bias(self, x_fp: torch.Tensor, x_int8: torch.Tensor, sx: torch.Tensor,
                   out: Optional[torch.Tensor] = None) -> torch.Tensor:
        out_dtype = self._out_dtype()
        return gemm_mixed_rows_splitk(
            x_fp=x_fp, x_int8=x_int8, sx=sx,
            int8_tiles=self.int8_tiles, int8_scales=self.int8_scales, int8_tile_ids=self.int8_tile_ids,
            int8_row_ptr=self.int8_row_ptr, fp16_tiles=self.fp16_tiles, fp16_tile_ids=self.fp16_tile_ids,
            fp16_row_ptr=self.fp16_row_ptr, M=self.M_orig, K=self.K_orig, n_tr=self.n_tr, n_tc=self.n_tc,
            out_dtype=out_dtype, bias=self._out_bias(out_dtype), out=out, tile_layout=self.tile_layout,
        )

    def _fused_limit(self) -> int:
        limit = getattr(self, "_fused_rows", None)
        if limit is None:
            limit = self._fused_rows = fused_max_tokens(self.K_orig)
        return limit

    def _fused_rows_for_cfg(self) -> int:
        mode = _cfg_get(self.cfg, "fused_decode", None)
        if mode is False:
            return 0
        if mode is None or mode == "auto":
            rows = FUSED_AUTO_MAX_ROWS
            dev = self.int8_tiles.device
            if (dev.type == "cuda" and self.K_orig <= FUSED_AUTO_NARROW_K
                    and 4 * self.n_tr <= _device_cus(dev)):
                rows = FUSED_AUTO_NARROW_ROWS
            return min(rows, self._fused_limit())
        return self._fused_limit()

    def _fused_decode(self, x_fp: torch.Tensor) -> torch.Tensor:
        out_dtype = self._out_dtype()
        return linear_mixed_fused(
            x_fp=x_fp, int8_tiles=self.int8_tiles, int8_scales=self.int8_scales,
            int8_tile_ids=self.int8_tile_ids, int8_row_ptr=self.int8_row_ptr, fp16_tiles=self.fp16_tiles,
            fp16_tile_ids=self.fp16_tile_ids, fp16_row_ptr=self.fp16_row_ptr, M=self.M_orig, K=self.K_orig,
            n_tr=self.n_tr, n_tc=self.n_tc, out_dtype=out_dtype, bias=self._out_bias(out_dtype),
            tile_layout=self.tile_layout,
        )

    def _forward_chunk(self, x_chunk: torch.Tensor, sx: torch.Tensor, out: torch.Tensor) -> None:
        x_int8 = quantize_activation_tile_with_scales(x_chunk, sx=sx, tile_n=self.tile_n)
        self._gemm_bias(x_fp=x_chunk, x_int8=x_int8, sx=sx, out=out)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        in_shape = x.shape
        if x.dim() == 3:
            x2d = x.reshape(-1, x.shape[-1])
        elif x.dim() == 2:
            x2d = x
        else:
            raise ValueError(f"Expected input rank 2 or 3, got shape={tuple(x.shape)}")
        n_rows, k_in = x2d.shape
        if k_in != self.K_orig:
            raise ValueError(f"Input K mismatch: got {k_in}, expected {self.K_orig}")
        x_work = x2d.contiguous()
        chunk = self._activation_row_chunk_size()
        if 0 < n_rows <= min(self._fused_rows_for_cfg(), chunk):
            y = self._fused_decode(x_work)
        elif n_rows <= chunk:
            x_int8, sx = _quantize_shared_activation(source=x, x_work=x_work, tile_n=self.tile_n,
                                                     consumer_id=id(self))
            y = self._gemm_bias(x_fp=x_work, x_int8=x_int8, sx=sx)
        else:
            sx = activation_tile_absmax_scales(x_work, tile_n=self.tile_n)
            y = torch.empty((n_rows, self.M_orig), device=x_work.device, dtype=self._out_dtype())
            for start in range(0, n_rows, chunk):
                self._forward_chunk(x_work[start:start + chunk], sx, y[start:start + chunk])
        if x.dim() == 3:
            y = y.reshape(in_shape[0], in_shape[1], self.M_orig)
        return y


@dataclass
class _PendingGroupOutput:
    source_ref: "weakref.ReferenceType[torch.Tensor]"
    signature: Tuple[Any, ...]
    consumed: set
    output: torch.Tensor


class MixedLinearGroup(nn.Module):
    """Sibling projections of one activation executed as one stacked GEMM
    (mixed_linear.py:265-333).  Every output element comes from the same tile
    sequence and arithmetic as the member's own MixedLinear."""

    def __init__(self, members):
        super().__init__()
        if len(members) < 2:
            raise ValueError("A projection group needs at least two members")
        has_bias = [m.bias is not None for m in members]
        if any(has_bias) and not all(has_bias):
            raise ValueError("Projection group members must all have or all lack bias")
        bias = torch.cat([m.bias.detach() for m in members]) if all(has_bias) else None
        self.linear = MixedLinear(concat_packs_along_rows([m.to_pack() for m in members]), bias, members[0].cfg)
        bounds, start = [], 0
        for m in members:
            bounds.append((start, start + m.M_orig))
            start += m.M_orig
        self.bounds = tuple(bounds)
        self._pending: Optional[_PendingGroupOutput] = None

    def _signature(self, x: torch.Tensor) -> Tuple[Any, ...]:
        return (int(x.data_ptr()), int(x.storage_offset()), tuple(x.shape), tuple(x.stride()), x.dtype,
                x.device, _activation_version(x))

    def output_for(self, x: torch.Tensor, index: int) -> torch.Tensor:
        pending = self._pending
        signature = self._signature(x)
        if (pending is not None and pending.source_ref() is x and pending.signature == signature
                and index not in pending.consumed):
            pending.consumed.add(index)
            out = pending.output
            if len(pending.consumed) == len(self.bounds):
                self._pending = None
            return out
        self._pending = None
        out = self.linear(x)
        try:
            ref = weakref.ref(x)
        except TypeError:
            return out
        self._pending = _PendingGroupOutput(ref, signature, {index}, out)
        return out

    def reset_pending(self) -> None:
        self._pending = None


class MixedLinearSlice(nn.Module):
    """One member projection served from its MixedLinearGroup output."""

    def __init__(self, group: MixedLinearGroup, index: int):
        super().__init__()
        object.__setattr__(self, "group", group)  # owned (and counted) by the parent
        self.index = int(index)
        self.start, self.stop = group.bounds[self.index]
        self.out_features = self.stop - self.start
        self.in_features = group.linear.K_orig

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.group.output_for(x, self.index)[..., self.start:self.stop]


PROJECTION_GROUPS = (
    ("tilequant_qkv", ("q_proj", "k_proj", "v_proj")),
    ("tilequant_gate_up", ("gate_proj", "up_proj")),
)


def fuse_projection_groups(model: nn.Module) -> int:
    """Replace Q/K/V and Gate/Up MixedLinear siblings by stacked groups
    (mixed_linear.py:359-386).  Returns the number of groups formed."""
    fused = 0
    for parent in list(model.modules()):
        for group_name, names in PROJECTION_GROUPS:
            members = [getattr(parent, n, None) for n in names]
            if not all(isinstance(m, MixedLinear) for m in members):
                continue
            first = members[0]
            if any(m.K_orig != first.K_orig or m.M_orig % m.tile_m != 0 or m.tile_m != first.tile_m
                   or m.tile_n != first.tile_n or m.int8_tiles.device != first.int8_tiles.device
                   or m.tile_layout != first.tile_layout for m in members):
                continue
            if len({m.bias is None for m in members}) != 1:
                continue
            group = MixedLinearGroup(members)
            parent.add_module(group_name, group)
            for i, n in enumerate(names):
                setattr(parent, n, MixedLinearSlice(group, i))
            fused += 1
    return fused


def reset_projection_groups(model: nn.Module) -> None:
    for module in model.modules():
        if isinstance(module, MixedLinearGroup):
            module.reset_pending()
