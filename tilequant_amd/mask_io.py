"""Decision/ tile-map archives (mirror of src/kernels/mask_io.py).

Format (mask_io.py:36-68): ``<keep_dir>/fp16_keep_ids_tile{tm}x{tn}.npz`` with
``stems`` (sorted unicode stems, module name with '.' -> '_'), and per stem
index i ``shape_i`` (int32 [n_tr, n_tc]) and ``ids_i`` (ascending flat ids
r * n_tc + c of the tiles kept in 16-bit; uint16 when n_tr * n_tc <= 65535,
else uint32).  Readers validate shapes and id bounds and cache one parsed
archive per path per process (mask_io.py:71-95).
"""
from __future__ import annotations

from pathlib import Path
from typing import Dict, Tuple

import numpy as np
import torch

_ARCHIVE_BASENAME = "fp16_keep_ids"
_ARCHIVE_CACHE: Dict[str, Dict[str, Tuple[Tuple[int, int], np.ndarray]]] = {}


def layer_name_to_stem(layer_name: str) -> str:
    return layer_name.replace(".", "_")


def _as_binary_mask(mask_keep) -> np.ndarray:
    arr = np.asarray(mask_keep)
    if arr.ndim != 2:
        raise ValueError(f"mask_keep must be 2D, got shape={tuple(arr.shape)}")
    u8 = arr.astype(np.uint8, copy=False)
    values = set(int(v) for v in np.unique(u8).tolist())
    if not values.issubset({0, 1}):
        raise ValueError(f"mask_keep must be binary {{0,1}}, got values={sorted(values)}")
    return u8


def _archive_path(keep_dir, tile_m: int, tile_n: int) -> Path:
    return Path(keep_dir) / f"{_ARCHIVE_BASENAME}_tile{tile_m}x{tile_n}.npz"


def _ids_of_mask(mask_u8: np.ndarray) -> np.ndarray:
    flat = mask_u8.reshape(-1)
    ids = np.flatnonzero(flat == 1)
    small = flat.size <= np.iinfo(np.uint16).max
    return ids.astype(np.uint16 if small else np.uint32, copy=False)


def save_mask_keep_archive(keep_dir, masks_by_stem: Dict[str, np.ndarray], tile_m: int = 64,
                           tile_n: int = 64) -> Path:
    keep_dir = Path(keep_dir)
    keep_dir.mkdir(parents=True, exist_ok=True)
    if not masks_by_stem:
        raise ValueError("masks_by_stem is empty")
    stems = sorted(str(k) for k in masks_by_stem)
    payload = {"stems": np.asarray(stems, dtype=np.str_)}
    for i, stem in enumerate(stems):
        mask = _as_binary_mask(masks_by_stem[stem])
        payload[f"shape_{i}"] = np.asarray(mask.shape, dtype=np.int32)
        payload[f"ids_{i}"] = _ids_of_mask(mask)
    path = _archive_path(keep_dir, tile_m, tile_n)
    np.savez_compressed(path, **payload)
    _ARCHIVE_CACHE.pop(str(path.resolve()), None)
    return path


def _load_archive_map(keep_dir, tile_m: int, tile_n: int) -> Dict[str, Tuple[Tuple[int, int], np.ndarray]]:
    path = _archive_path(keep_dir, tile_m, tile_n)
    if not path.exists():
        raise FileNotFoundError(f"FP16 keep-id archive not found: {path}")
    key = str(path.resolve())
    cached = _ARCHIVE_CACHE.get(key)
    if cached is not None:
        return cached
    out: Dict[str, Tuple[Tuple[int, int], np.ndarray]] = {}
    with np.load(path, allow_pickle=False) as data:
        for i, stem in enumerate(str(s) for s in np.asarray(data["stems"]).tolist()):
            shape = np.asarray(data[f"shape_{i}"], dtype=np.int64)
            if shape.shape != (2,):
                raise RuntimeError(f"Invalid shape metadata for stem={stem} in {path}")
            n_tr, n_tc = int(shape[0]), int(shape[1])
            ids = np.asarray(data[f"ids_{i}"])
            if ids.dtype not in (np.uint16, np.uint32):
                ids = ids.astype(np.uint32, copy=False)
            if ids.size and int(ids.max()) >= n_tr * n_tc:
                raise RuntimeError(f"Out-of-bound fp16 tile id for stem={stem} in {path}")
            out[stem] = ((n_tr, n_tc), ids)
    _ARCHIVE_CACHE[key] = out
    return out


def _lookup(keep_dir, layer_name: str, tile_m: int, tile_n: int):
    stem = layer_name_to_stem(layer_name)
    amap = _load_archive_map(keep_dir, tile_m, tile_n)
    if stem not in amap:
        raise FileNotFoundError(f"Layer stem not found in archive for layer '{layer_name}': stem={stem}")
    return amap[stem]


def _mask_of(shape: Tuple[int, int], ids: np.ndarray) -> torch.Tensor:
    n_tr, n_tc = shape
    flat = np.zeros((n_tr * n_tc,), dtype=np.uint8)
    flat[ids.astype(np.int64, copy=False)] = 1
    return torch.from_numpy(flat.reshape(n_tr, n_tc)).contiguous()


def load_mask_keep_for_layer(keep_dir, layer_name: str, tile_m: int = 64, tile_n: int = 64) -> torch.Tensor:
    shape, ids = _lookup(keep_dir, layer_name, tile_m, tile_n)
    return _mask_of(shape, ids)


def load_fp16_keep_ids_for_layer(keep_dir, layer_name: str, tile_m: int = 64,
                                 tile_n: int = 64) -> Tuple[torch.Tensor, Tuple[int, int]]:
    shape, ids = _lookup(keep_dir, layer_name, tile_m, tile_n)
    return torch.from_numpy(ids.astype(np.int64, copy=False)).to(torch.int32).contiguous(), shape


def load_mask_keep_stem_dict(keep_dir, tile_m: int = 64, tile_n: int = 64) -> Dict[str, torch.Tensor]:
    amap = _load_archive_map(keep_dir, tile_m, tile_n)
    return {stem: _mask_of(shape, ids) for stem, (shape, ids) in amap.items()}
