"""Load-time weight packing (mirror of src/kernels/pack.py).

Same ``Pack`` fields, function names, arguments and error behaviour as the
reference (pack.py:11-29, 38-62, 65-224, 239-321).  Differences, both by
design for gfx950:

* The per-tile quantization and the 16-bit tile copy run as HIP kernels
  (``tq_pack_int8_tiles`` / ``tq_pack_16bit_tiles``), so a weight handed over
  on the CPU is copied to the current ROCm device first and the returned
  ``Pack`` lives there (callers that ``.to(device)`` it, as the reference's
  loader does at api.py:238, are unaffected).
* Tiles are written in ``tile_layout`` order: ``"mfma"`` (default; the MFMA
  operand-major order the GEMM streams with one coalesced 1 KiB load per
  16-row block) or ``"row_major"`` (the reference's order).  ``Pack`` records
  it in an extra trailing field.

Tile bookkeeping (sorted ids, CSR row pointers) is integer host logic and runs
with torch ops on the ids' device.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Dict, Optional, Sequence

import torch

from . import _native as nat
from ._config import cfg_value

TILE_LAYOUTS = ("row_major", "mfma")


@dataclass
class Pack:
    M_orig: int
    K_orig: int
    M: int
    K: int
    tile_m: int
    tile_n: int
    n_tr: int
    n_tc: int
    int8_tiles: torch.Tensor
    int8_scales: torch.Tensor
    int8_tile_ids: torch.Tensor
    int8_row_ptr: torch.Tensor
    int8_row_indices: torch.Tensor
    fp16_tiles: torch.Tensor
    fp16_tile_ids: torch.Tensor
    fp16_row_ptr: torch.Tensor
    fp16_row_indices: torch.Tensor
    tile_layout: str = "row_major"



def _order_tile_ids_row_major(tile_ids: torch.Tensor) -> torch.Tensor:
    """Ascending ids: the tiles of row tile r become contiguous, in ascending
    column order (pack.py:38-45)."""
    if tile_ids.numel() <= 1:
        return tile_ids.contiguous()
    return torch.sort(tile_ids).values.contiguous()


def _build_row_schedule(tile_ids: torch.Tensor, *, n_tr: int, n_tc: int):
    """CSR row pointer over sorted ids and the (identity) row index list (pack.py:48-62)."""
    row_ptr = torch.zeros((n_tr + 1,), device=tile_ids.device, dtype=torch.int32)
    if tile_ids.numel() == 0:
        return row_ptr, torch.empty((0,), device=tile_ids.device, dtype=torch.int32)
    rows = torch.div(tile_ids, n_tc, rounding_mode="floor")
    counts = torch.bincount(rows, minlength=n_tr).to(torch.int32)
    row_ptr[1:] = torch.cumsum(counts, dim=0)
    row_indices = torch.argsort(tile_ids).to(torch.int32).contiguous()
    return row_ptr, row_indices


def _target_device(W: torch.Tensor) -> torch.device:
    if W.is_cuda:
        return W.device
    if not torch.cuda.is_available():
        raise RuntimeError("tilequant_amd packs weights with HIP kernels and needs a ROCm device")
    return torch.device("cuda", torch.cuda.current_device())


def _pack_weight_with_tile_ids(
    W_fp: torch.Tensor,
    *,
    n_tr: int,
    n_tc: int,
    int8_tile_ids: torch.Tensor,
    fp16_tile_ids: torch.Tensor,
    iaa_col_importance: Optional[torch.Tensor],
    cfg: Any,
    tile_layout: str = "mfma",
) -> Pack:
    if W_fp.dim() != 2:
        raise ValueError(f"Expected W to be 2D, got shape={tuple(W_fp.shape)}")
    tile_m = int(cfg_value(cfg, "tile_m", 64))
    tile_n = int(cfg_value(cfg, "tile_n", 64))
    use_pad = bool(cfg_value(cfg, "pad_to_tile", True))
    quant_style = str(cfg_value(cfg, "quant_style", "gi")).lower()
    if quant_style not in ("gi", "iaa"):
        raise ValueError(f"Unsupported quant_style={quant_style}. Expected one of: gi, iaa")
    if (tile_m, tile_n) != (64, 64):
        raise ValueError(f"only 64x64 tiles are supported, got {tile_m}x{tile_n}")
    if tile_layout not in TILE_LAYOUTS:
        raise ValueError(f"tile_layout must be one of {TILE_LAYOUTS}, got {tile_layout!r}")
    M_orig, K_orig = (int(v) for v in W_fp.shape)
    if use_pad:
        M = -(-M_orig // 64) * 64
        K = -(-K_orig // 64) * 64
    else:
        if (M_orig % tile_m) or (K_orig % tile_n):
            raise ValueError("pad_to_tile=False but weight shape is not multiple of tile size")
        M, K = M_orig, K_orig
    if n_tr * tile_m != M or n_tc * tile_n != K:
        raise ValueError(
            f"PrecisionMap dimensions mismatch: map(n_tr={n_tr}, n_tc={n_tc}) "
            f"vs weight(M={M}, K={K}, tile_m={tile_m}, tile_n={tile_n})"
        )
    w_dtype = W_fp.dtype
    code = nat.dtype_code(w_dtype)
    device = _target_device(W_fp)
    # the kernels read the weight as if zero-padded to (M, K): no padded copy
    W_dev = W_fp.to(device=device)
    if W_dev.stride(1) != 1:
        W_dev = W_dev.contiguous()

    int8_ids = _order_tile_ids_row_major(int8_tile_ids.to(device="cpu", dtype=torch.int64))
    fp16_ids = _order_tile_ids_row_major(fp16_tile_ids.to(device="cpu", dtype=torch.int64))
    if int8_ids.numel() + fp16_ids.numel() != n_tr * n_tc:
        raise RuntimeError(
            "Packed tile count mismatch: "
            f"T8={int8_ids.numel()}, T16={fp16_ids.numel()}, total={n_tr * n_tc}"
        )
    int8_row_ptr, int8_row_indices = _build_row_schedule(int8_ids, n_tr=n_tr, n_tc=n_tc)
    fp16_row_ptr, fp16_row_indices = _build_row_schedule(fp16_ids, n_tr=n_tr, n_tc=n_tc)

    ids8_dev = int8_ids.to(device=device, dtype=torch.int32)
    ids16_dev = fp16_ids.to(device=device, dtype=torch.int32)
    T8, T16 = int(ids8_dev.numel()), int(ids16_dev.numel())
    int8_tiles = torch.empty((T8, 64, 64), device=device, dtype=torch.int8)
    int8_scales = torch.empty((T8,), device=device, dtype=torch.float32)
    fp16_tiles = torch.empty((T16, 64, 64), device=device, dtype=w_dtype)
    stream = nat.stream_handle(device)
    layout = nat.TQ_LAYOUT[tile_layout]

    imp = None
    if quant_style == "iaa" and iaa_col_importance is not None and T8:
        col = iaa_col_importance.to(device=device, dtype=torch.float32).reshape(-1)
        imp = torch.zeros((K,), device=device, dtype=torch.float32)
        n_copy = min(int(col.numel()), K)
        imp[:n_copy] = col[:n_copy]
    if T8:
        rc = nat.lib().tq_pack_int8_tiles(
            nat.ptr(W_dev), W_dev.stride(0), code, M_orig, K_orig, nat.ptr(ids8_dev), T8, n_tc, layout,
            nat.ptr(imp), nat.ptr(int8_tiles), nat.ptr(int8_scales), stream)
        nat.check(rc, "tq_pack_int8_tiles")
    if T16:
        rc = nat.lib().tq_pack_16bit_tiles(
            nat.ptr(W_dev), W_dev.stride(0), code, M_orig, K_orig, nat.ptr(ids16_dev), T16, n_tc, layout,
            nat.ptr(fp16_tiles), stream)
        nat.check(rc, "tq_pack_16bit_tiles")

    return Pack(
        M_orig=M_orig, K_orig=K_orig, M=M, K=K, tile_m=tile_m, tile_n=tile_n, n_tr=n_tr, n_tc=n_tc,
        int8_tiles=int8_tiles, int8_scales=int8_scales, int8_tile_ids=ids8_dev,
        int8_row_ptr=int8_row_ptr.to(device), int8_row_indices=int8_row_indices.to(device),
        fp16_tiles=fp16_tiles, fp16_tile_ids=ids16_dev,
        fp16_row_ptr=fp16_row_ptr.to(device), fp16_row_indices=fp16_row_indices.to(device),
        tile_layout=tile_layout,
    )


def pack_weight_from_tile_ids(
    W_fp: torch.Tensor,
    *,
    n_tr: int,
    n_tc: int,
    int8_tile_ids: torch.Tensor,
    fp16_tile_ids: torch.Tensor,
    iaa_col_importance: Optional[torch.Tensor] = None,
    cfg: Any,
    tile_layout: str = "mfma",
) -> Pack:
    return _pack_weight_with_tile_ids(
        W_fp=W_fp, n_tr=int(n_tr), n_tc=int(n_tc), int8_tile_ids=int8_tile_ids,
        fp16_tile_ids=fp16_tile_ids, iaa_col_importance=iaa_col_importance, cfg=cfg,
        tile_layout=tile_layout,
    )


def pack_weight(W_fp: torch.Tensor, pmap: Dict[str, Any], cfg: Any) -> Pack:
    return _pack_weight_with_tile_ids(
        W_fp=W_fp, n_tr=int(pmap["n_tr"]), n_tc=int(pmap["n_tc"]),
        int8_tile_ids=pmap["int8_tile_ids"], fp16_tile_ids=pmap["fp16_tile_ids"],
        iaa_col_importance=None, cfg=cfg,
    )


def is_row_major_pack(pack: Pack) -> bool:
    """True when tile ids are strictly ascending (row-major tile ORDER, pack.py:239-243)."""
    for ids in (pack.int8_tile_ids, pack.fp16_tile_ids):
        if ids.numel() > 1 and not bool((ids[1:] > ids[:-1]).all()):
            return False
    return True


def relayout_pack(pack: Pack, tile_layout: str) -> Pack:
    """Return ``pack`` with its tiles re-written in ``tile_layout`` (a copy, on
    the GPU); payload values and scales are unchanged."""
    if tile_layout not in TILE_LAYOUTS:
        raise ValueError(f"tile_layout must be one of {TILE_LAYOUTS}, got {tile_layout!r}")
    if pack.tile_layout == tile_layout:
        return pack
    nat.require_device(pack.int8_tiles, pack.fp16_tiles)

    def convert(tiles: torch.Tensor, elem_bytes: int) -> torch.Tensor:
        out = torch.empty_like(tiles)
        if tiles.numel():
            rc = nat.lib().tq_tiles_relayout(
                nat.ptr(tiles.contiguous()), nat.ptr(out), int(tiles.shape[0]), elem_bytes,
                nat.TQ_LAYOUT[pack.tile_layout], nat.TQ_LAYOUT[tile_layout], nat.stream_handle(tiles.device))
            nat.check(rc, "tq_tiles_relayout")
        return out

    d = dict(pack.__dict__)
    d["int8_tiles"] = convert(pack.int8_tiles, 1)
    d["fp16_tiles"] = convert(pack.fp16_tiles, 2)
    d["tile_layout"] = tile_layout
    return Pack(**d)


def concat_packs_along_rows(packs: Sequence[Pack]) -> Pack:
    """Stack packs of projections that share one input along the output rows
    (pack.py:246-321).  Members need the same input geometry, tile-aligned
    output widths, row-major tile order and the same tile layout; payloads and
    scales are copied unchanged, ids shift by the row offset and row pointers
    by the running tile count."""
    if not packs:
        raise ValueError("Expected at least one pack")
    first = packs[0]
    for pack in packs:
        if (pack.K_orig, pack.K, pack.tile_m, pack.tile_n, pack.n_tc) != (
            first.K_orig, first.K, first.tile_m, first.tile_n, first.n_tc
        ):
            raise ValueError("Packs must share input geometry to be stacked")
        if pack.M_orig != pack.M or pack.M_orig % pack.tile_m != 0:
            raise ValueError("Stacked packs require tile-aligned output widths")
        if not is_row_major_pack(pack):
            raise ValueError("Stacked packs require row-major tile order")
        if pack.tile_layout != first.tile_layout:
            raise ValueError("Stacked packs require the same tile layout")
    n_tc = first.n_tc

    def stack(kind: str):
        tiles, scales, ids, row_indices = [], [], [], []
        row_ptrs = [torch.zeros((1,), dtype=torch.int32, device=first.int8_row_ptr.device)]
        tile_base = row_base = 0
        for pack in packs:
            pid = getattr(pack, f"{kind}_tile_ids").to(torch.int64)
            tiles.append(getattr(pack, f"{kind}_tiles"))
            if kind == "int8":
                scales.append(pack.int8_scales)
            ids.append(pid + row_base * n_tc)
            row_ptrs.append(getattr(pack, f"{kind}_row_ptr")[1:].to(torch.int32) + tile_base)
            row_indices.append(getattr(pack, f"{kind}_row_indices").to(torch.int32) + tile_base)
            tile_base += int(pid.numel())
            row_base += pack.n_tr
        return (torch.cat(tiles).contiguous(), torch.cat(scales).contiguous() if scales else None,
                torch.cat(ids).to(torch.int32).contiguous(), torch.cat(row_ptrs).contiguous(),
                torch.cat(row_indices).contiguous())

    t8, s8, i8, rp8, ri8 = stack("int8")
    t16, _, i16, rp16, ri16 = stack("fp16")
    M = sum(p.M for p in packs)
    return Pack(
        M_orig=M, K_orig=first.K_orig, M=M, K=first.K, tile_m=first.tile_m, tile_n=first.tile_n,
        n_tr=sum(p.n_tr for p in packs), n_tc=n_tc,
        int8_tiles=t8, int8_scales=s8, int8_tile_ids=i8, int8_row_ptr=rp8, int8_row_indices=ri8,
        fp16_tiles=t16, fp16_tile_ids=i16, fp16_row_ptr=rp16, fp16_row_indices=ri16,
        tile_layout=first.tile_layout,
    )
