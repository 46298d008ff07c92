"""Decision/ tile maps: reader and writer of the released archive format.

The format is the contract shared with the released maps (written by the
reference at src/kernels/mask_io.py:45-68, read at :71-142):

* one file per keep level and tile size, ``<keep_dir>/fp16_keep_ids_tile{TM}x{TN}.npz``
  (numpy's npz container; pickled objects are never read);
* ``stems``: unicode array of module stems (the module name with every ``.``
  replaced by ``_``), sorted lexicographically;
* for the stem at index ``i``: ``shape_i``, int32 ``(n_tr, n_tc)``, the tile
  grid, and ``ids_i``, the ascending flat ids ``r * n_tc + c`` of the tiles
  kept in 16 bits -- uint16 for grids of at most 65535 tiles, else uint32.

Here an archive is parsed and validated once into a ``TileMapArchive``; the
parsed form is shared per file and re-read when the file changes on disk.
The public functions keep the reference's names, arguments, return values,
exception types and messages (the drop-in boundary).
"""
from __future__ import annotations

import threading
from dataclasses import dataclass
from pathlib import Path
from typing import Dict, Iterator, Mapping, Tuple

import numpy as np
import torch

# ids of grids up to this many tiles are stored as uint16, larger grids as uint32
_UINT16_GRID_LIMIT = int(np.iinfo(np.uint16).max)


def archive_path(keep_dir, tile_m: int = 64, tile_n: int = 64) -> Path:
    """Location of the archive of one keep level for tile_m x tile_n tiles."""
    return Path(keep_dir) / f"fp16_keep_ids_tile{int(tile_m)}x{int(tile_n)}.npz"


def layer_name_to_stem(layer_name: str) -> str:
    """``model.layers.0.mlp.up_proj`` -> ``model_layers_0_mlp_up_proj``."""
    return "_".join(layer_name.split("."))


@dataclass(frozen=True)
class TileMap:
    """One layer's entry: its tile grid and the ascending flat ids of the
    tiles kept in 16 bits (uint16 or uint32, bounds-checked)."""

    grid: Tuple[int, int]
    ids: np.ndarray

    def ids_tensor(self) -> torch.Tensor:
        """The 16-bit tile ids as a contiguous int32 tensor."""
        return torch.from_numpy(self.ids.astype(np.int32))

    def mask_tensor(self) -> torch.Tensor:
        """The keep mask as a contiguous uint8 [n_tr, n_tc] tensor (1 = 16-bit tile)."""
        n_tr, n_tc = self.grid
        keep = np.zeros(n_tr * n_tc, dtype=np.uint8)
        keep[self.ids.astype(np.int64)] = 1
        return torch.from_numpy(keep).view(n_tr, n_tc)


class TileMapArchive(Mapping[str, TileMap]):
    """A parsed archive: a read-only mapping stem -> TileMap, every entry
    validated when the file is opened."""

    def __init__(self, path: Path):
        self.path = Path(path)
        self._maps: Dict[str, TileMap] = {}
        with np.load(self.path, allow_pickle=False) as npz:
            for i, stem in enumerate(np.asarray(npz["stems"]).tolist()):
                stem = str(stem)
                self._maps[stem] = self._entry(stem, npz[f"shape_{i}"], npz[f"ids_{i}"])

    def _entry(self, stem: str, shape, ids) -> TileMap:
        grid = np.asarray(shape).astype(np.int64)
        if grid.shape != (2,):
            raise RuntimeError(f"Invalid shape metadata for stem={stem} in {self.path}")
        n_tr, n_tc = (int(v) for v in grid)
        ids = np.asarray(ids)
        if ids.dtype != np.uint16 and ids.dtype != np.uint32:
            ids = ids.astype(np.uint32)
        if ids.size and int(ids.max()) >= n_tr * n_tc:
            raise RuntimeError(f"Out-of-bound fp16 tile id for stem={stem} in {self.path}")
        return TileMap((n_tr, n_tc), ids)

    def __getitem__(self, stem: str) -> TileMap:
        return self._maps[stem]

    def __iter__(self) -> Iterator[str]:
        return iter(self._maps)

    def __len__(self) -> int:
        return len(self._maps)

    def layer(self, layer_name: str) -> TileMap:
        """The entry of a module by its dotted name."""
        stem = layer_name_to_stem(layer_name)
        found = self._maps.get(stem)
        if found is None:
            raise FileNotFoundError(f"Layer stem not found in archive for layer '{layer_name}': stem={stem}")
        return found


# parsed archives by resolved path, with the (mtime, size) they were read at
_OPENED: Dict[Path, Tuple[Tuple[int, int], TileMapArchive]] = {}
_OPENED_LOCK = threading.Lock()


def open_archive(keep_dir, tile_m: int = 64, tile_n: int = 64) -> TileMapArchive:
    """The parsed archive of ``keep_dir``; parsed once per process and again
    only when the file has changed since."""
    path = archive_path(keep_dir, tile_m, tile_n)
    if not path.is_file():
        raise FileNotFoundError(f"FP16 keep-id archive not found: {path}")
    key = path.resolve()
    st = key.stat()
    stamp = (st.st_mtime_ns, st.st_size)
    with _OPENED_LOCK:
        hit = _OPENED.get(key)
        if hit is not None and hit[0] == stamp:
            return hit[1]
    parsed = TileMapArchive(key)
    with _OPENED_LOCK:
        _OPENED[key] = (stamp, parsed)
    return parsed


def _keep_ids_of_mask(mask_keep) -> Tuple[np.ndarray, np.ndarray]:
    """(shape int32 [2], ascending 16-bit tile ids) of one binary 2-D keep mask."""
    grid = np.asarray(mask_keep)
    if grid.ndim != 2:
        raise ValueError(f"mask_keep must be 2D, got shape={tuple(grid.shape)}")
    grid = grid.astype(np.uint8, copy=False)
    present = np.unique(grid)
    if present.size and int(present[-1]) > 1:
        raise ValueError(f"mask_keep must be binary {{0,1}}, got values={present.tolist()}")
    ids = np.nonzero(grid.ravel())[0]
    id_type = np.uint16 if grid.size <= _UINT16_GRID_LIMIT else np.uint32
    return np.array(grid.shape, dtype=np.int32), ids.astype(id_type)


def save_mask_keep_archive(keep_dir, masks_by_stem: Mapping[str, np.ndarray], tile_m: int = 64,
                           tile_n: int = 64) -> Path:
    """Write ``masks_by_stem`` (stem -> binary [n_tr, n_tc] keep mask, 1 = keep
    the tile in 16 bits) as the archive of ``keep_dir``; returns its path."""
    by_stem = {str(stem): mask for stem, mask in masks_by_stem.items()}
    if not by_stem:
        raise ValueError("masks_by_stem is empty")
    arrays: Dict[str, np.ndarray] = {}
    ordered = sorted(by_stem)
    for i, stem in enumerate(ordered):
        arrays[f"shape_{i}"], arrays[f"ids_{i}"] = _keep_ids_of_mask(by_stem[stem])
    arrays["stems"] = np.array(ordered, dtype=np.str_)
    Path(keep_dir).mkdir(parents=True, exist_ok=True)
    path = archive_path(keep_dir, tile_m, tile_n)
    np.savez_compressed(path, **arrays)
    with _OPENED_LOCK:
        _OPENED.pop(path.resolve(), None)
    return path


def load_mask_keep_for_layer(keep_dir, layer_name: str, tile_m: int = 64, tile_n: int = 64) -> torch.Tensor:
    """uint8 [n_tr, n_tc] keep mask of one module (1 = 16-bit tile)."""
    return open_archive(keep_dir, tile_m, tile_n).layer(layer_name).mask_tensor()


def load_fp16_keep_ids_for_layer(keep_dir, layer_name: str, tile_m: int = 64,
                                 tile_n: int = 64) -> Tuple[torch.Tensor, Tuple[int, int]]:
    """(int32 ascending 16-bit tile ids, (n_tr, n_tc)) of one module."""
    entry = open_archive(keep_dir, tile_m, tile_n).layer(layer_name)
    return entry.ids_tensor(), entry.grid


def load_mask_keep_stem_dict(keep_dir, tile_m: int = 64, tile_n: int = 64) -> Dict[str, torch.Tensor]:
    """stem -> uint8 keep mask for every module of the archive."""
    return {stem: entry.mask_tensor() for stem, entry in open_archive(keep_dir, tile_m, tile_n).items()}
