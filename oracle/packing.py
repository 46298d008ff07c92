"""numpy restatement of the load-time packer's bookkeeping and tile layouts.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Follows src/kernels/pack.py:38-62 (id order, CSR row pointers), 65-203
(tile gather and per-tile INT8 quantization, "gi" style; the "iaa" scale
search of :132-159 in ``iaa_scales``), 246-321 (row
stacking of packs that share one input) and src/quantization/api.py:112-117
(INT8 ids are the complement of the BF16 ids).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import numerics as nm

TILE = 64


@dataclass
class OraclePack:
    M_orig: int
    K_orig: int
    M: int
    K: int
    n_tr: int
    n_tc: int
    int8_tiles: np.ndarray      # [T8, 64, 64] int8, row-major tiles
    int8_scales: np.ndarray     # [T8] f32
    int8_tile_ids: np.ndarray   # [T8] int32 ascending
    int8_row_ptr: np.ndarray    # [n_tr+1] int32
    fp16_tiles: np.ndarray      # [T16, 64, 64] uint16 bf16 bit patterns, row-major
    fp16_tile_ids: np.ndarray   # [T16] int32 ascending
    fp16_row_ptr: np.ndarray    # [n_tr+1] int32


def row_ptr_of(ids: np.ndarray, n_tr: int, n_tc: int) -> np.ndarray:
    """CSR row pointer: row_ptr[r+1]-row_ptr[r] = number of ids in row tile r."""
    ids = np.asarray(ids, dtype=np.int64)
    counts = np.bincount(ids // n_tc, minlength=n_tr) if ids.size else np.zeros(n_tr, np.int64)
    return np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)


def int8_ids_complement(fp16_ids: np.ndarray, n_tiles: int) -> np.ndarray:
    mask = np.zeros(n_tiles, dtype=bool)
    mask[np.asarray(fp16_ids, dtype=np.int64)] = True
    return np.flatnonzero(~mask).astype(np.int32)


def pad64(w: np.ndarray) -> np.ndarray:
    m, k = w.shape
    mp, kp = -(-m // TILE) * TILE, -(-k // TILE) * TILE
    if (mp, kp) == (m, k):
        return w
    out = np.zeros((mp, kp), dtype=w.dtype)
    out[:m, :k] = w
    return out


def pack_weight(w_bits: np.ndarray, fp16_ids: np.ndarray) -> OraclePack:
    """Pack a bf16 weight [M, K] (uint16 bit patterns) given its BF16 tile ids."""
    w_bits = np.asarray(w_bits, dtype=np.uint16)
    m0, k0 = w_bits.shape
    wp = pad64(w_bits)
    m, k = wp.shape
    n_tr, n_tc = m // TILE, k // TILE
    fp16_ids = np.sort(np.asarray(fp16_ids, dtype=np.int64))
    int8_ids = int8_ids_complement(fp16_ids, n_tr * n_tc).astype(np.int64)
    w8src = nm.bf16_bits_to_f32(nm.tiles_of(wp, int8_ids, n_tc)) if int8_ids.size else np.zeros((0, 64, 64), np.float32)
    q8, sw = nm.weight_tile_quant(w8src) if int8_ids.size else (np.zeros((0, 64, 64), np.int8), np.zeros(0, np.float32))
    w16 = nm.tiles_of(wp, fp16_ids, n_tc) if fp16_ids.size else np.zeros((0, 64, 64), np.uint16)
    return OraclePack(
        M_orig=m0, K_orig=k0, M=m, K=k, n_tr=n_tr, n_tc=n_tc,
        int8_tiles=q8, int8_scales=sw, int8_tile_ids=int8_ids.astype(np.int32),
        int8_row_ptr=row_ptr_of(int8_ids, n_tr, n_tc),
        fp16_tiles=np.ascontiguousarray(w16), fp16_tile_ids=fp16_ids.astype(np.int32),
        fp16_row_ptr=row_ptr_of(fp16_ids, n_tr, n_tc),
    )


def concat_rows(packs):
    """Stack packs along output rows: ids shift by row_base*n_tc, row pointers
    by the running tile count, payloads copied unchanged (pack.py:274-298)."""
    n_tc = packs[0].n_tc
    out = {}
    for kind in ("int8", "fp16"):
        ids, rps, tiles = [], [np.zeros(1, np.int32)], []
        tile_base = row_base = 0
        for p in packs:
            pid = getattr(p, f"{kind}_tile_ids").astype(np.int64)
            ids.append(pid + row_base * n_tc)
            rps.append(getattr(p, f"{kind}_row_ptr")[1:].astype(np.int64) + tile_base)
            tiles.append(getattr(p, f"{kind}_tiles"))
            tile_base += pid.size
            row_base += p.n_tr
        out[kind] = (np.concatenate(tiles), np.concatenate(ids).astype(np.int32),
                     np.concatenate(rps).astype(np.int32))
    M = sum(p.M for p in packs)
    return OraclePack(
        M_orig=M, K_orig=packs[0].K_orig, M=M, K=packs[0].K, n_tr=sum(p.n_tr for p in packs),
        n_tc=n_tc, int8_tiles=out["int8"][0], int8_scales=np.concatenate([p.int8_scales for p in packs]),
        int8_tile_ids=out["int8"][1], int8_row_ptr=out["int8"][2],
        fp16_tiles=out["fp16"][0], fp16_tile_ids=out["fp16"][1], fp16_row_ptr=out["fp16"][2],
    )


# ---------------------------------------------------------------------------
# IAA scale search (pack.py:132-159)
# ---------------------------------------------------------------------------

IAA_MULTS = (0.75, 1.00, 1.25)


def iaa_scales(tiles: np.ndarray, col_imp: np.ndarray):
    """IAA per-tile scale choice for INT8 tiles [T, 64, 64] (float values) whose
    64 columns have importances col_imp [T, 64] (the tile's slice of the input-
    column importance vector).

    pack.py:132-159: base = 1 if a == 0 else f32(a) / 127; candidates
    s = max(base * m, 1e-12) for m in (0.75, 1, 1.25); the fp32 terms
    ((clamp(rint(w / s), -127, 127) * s - w)^2 * max(imp, 1e-8)) are formed op
    by op in fp32 as the reference's torch expressions do; their mean over the
    tile decides, the first candidate with a strictly lower error winning.
    The reference's fp32 mean has its own summation order; here the terms are
    summed in float64 (relative error ~2^-40), so the selection is the exact
    one.  Returns (scales f32 [T], errors f64 [3, T]) -- the errors let a
    caller see which tiles are near-ties within an fp32 summation bound.
    """
    t = np.asarray(tiles, dtype=np.float32)
    wm = np.maximum(np.asarray(col_imp, dtype=np.float32), np.float32(1e-8))[:, None, :]
    base = nm.weight_tile_scales(t)
    errs, cands = [], []
    for m in IAA_MULTS:
        sc = np.maximum(base * np.float32(m), np.float32(1e-12)).astype(np.float32)
        with np.errstate(divide="ignore", invalid="ignore"):
            q = np.clip(np.rint(t / sc[:, None, None]), -127, 127).astype(np.float32)
        d = (q * sc[:, None, None] - t).astype(np.float32)
        terms = ((d * d).astype(np.float32) * wm).astype(np.float32)
        errs.append(terms.astype(np.float64).sum(axis=(1, 2)) / 4096.0)
        cands.append(sc)
    errs = np.stack(errs)
    best = np.zeros(t.shape[0], dtype=np.int64)
    for i in (1, 2):
        best = np.where(errs[i] < errs[best, np.arange(t.shape[0])], i, best)
    return np.stack(cands)[best, np.arange(t.shape[0])].astype(np.float32), errs


# ---------------------------------------------------------------------------
# MFMA operand-major tile layout (the HIP kernels' storage order)
# ---------------------------------------------------------------------------
#
# INT8 tile t[j, k] (j = output feature, k = input column within the tile)
# is the B operand of v_mfma_i32_16x16x64_i8: for 16-row block jb, lane
# l = kq*16 + (j % 16) holds the 16 bytes t[j, 16kq:16kq+16].  Storing
# [jb][kq][j%16][16 bytes] makes one coalesced 1 KiB load per block.
#
# BF16 tile t[j, k] is the B operand of v_mfma_f32_16x16x32_bf16 twice per
# 16-row block (k halves h = 0, 1): lane l = kq*16 + (j % 16) holds the 8
# values t[j, 32h + 8kq : 32h + 8kq + 8].  Storage [jb][h][kq][j%16][8].

def to_mfma_int8(tiles: np.ndarray) -> np.ndarray:
    t = np.asarray(tiles).reshape(-1, 4, 16, 4, 16)          # [T, jb, jl, kq, e]
    return np.ascontiguousarray(t.transpose(0, 1, 3, 2, 4)).reshape(-1, 64, 64)


def from_mfma_int8(tiles: np.ndarray) -> np.ndarray:
    t = np.asarray(tiles).reshape(-1, 4, 4, 16, 16)          # [T, jb, kq, jl, e]
    return np.ascontiguousarray(t.transpose(0, 1, 3, 2, 4)).reshape(-1, 64, 64)


def to_mfma_16bit(tiles: np.ndarray) -> np.ndarray:
    t = np.asarray(tiles).reshape(-1, 4, 16, 2, 4, 8)        # [T, jb, jl, h, kq, e]
    return np.ascontiguousarray(t.transpose(0, 1, 3, 4, 2, 5)).reshape(-1, 64, 64)


def from_mfma_16bit(tiles: np.ndarray) -> np.ndarray:
    t = np.asarray(tiles).reshape(-1, 4, 2, 4, 16, 8)        # [T, jb, h, kq, jl, e]
    return np.ascontiguousarray(t.transpose(0, 1, 4, 2, 3, 5)).reshape(-1, 64, 64)
