"""Decision/ tile-map archive format and the top-k mask rule, restated.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Archive format (src/kernels/mask_io.py:36-68, 71-95): one npz per keep
directory, named ``fp16_keep_ids_tile64x64.npz``, holding ``stems`` (sorted
unicode module names with '.' -> '_'), and for stem i ``shape_i`` (int32 [2]:
n_tr, n_tc) and ``ids_i`` (flat ids r*n_tc + c of the BF16 tiles, ascending,
uint16 when n_tr*n_tc <= 65535 else uint32).

Mask rule (src/quantization/decisions.py:174-183): keep the k highest-scoring
tiles, k = max(1, ceil(frac * n_tiles)), all tiles when k >= n_tiles.
"""
from __future__ import annotations

import math

import numpy as np


def keep_count(n_tiles: int, keep_frac: float) -> int:
    return max(1, int(math.ceil(float(keep_frac) * int(n_tiles))))


def topk_ids(scores: np.ndarray, keep_frac: float) -> np.ndarray:
    """Flat ids of the k largest scores, ascending.  Ties at the k-th value are
    resolved by a stable sort here; the reference uses np.argpartition, whose
    choice among exact ties is unspecified, so callers compare tie-free cases
    exactly and tie cases by the score multiset."""
    v = np.asarray(scores).reshape(-1)
    k = keep_count(v.size, keep_frac)
    if k >= v.size:
        return np.arange(v.size)
    order = np.argsort(-v.astype(np.float64), kind="stable")
    return np.sort(order[:k])


def read_archive(path) -> dict:
    out = {}
    with np.load(path, allow_pickle=False) as d:
        stems = [str(s) for s in d["stems"].tolist()]
        for i, stem in enumerate(stems):
            shape = tuple(int(v) for v in d[f"shape_{i}"])
            out[stem] = (shape, np.asarray(d[f"ids_{i}"]))
    return out


def write_archive(path, ids_by_stem: dict, shapes: dict) -> None:
    stems = sorted(ids_by_stem)
    payload = {"stems": np.asarray(stems, dtype=np.str_)}
    for i, stem in enumerate(stems):
        n_tr, n_tc = shapes[stem]
        ids = np.sort(np.asarray(ids_by_stem[stem], dtype=np.int64))
        dt = np.uint16 if n_tr * n_tc <= np.iinfo(np.uint16).max else np.uint32
        payload[f"shape_{i}"] = np.asarray([n_tr, n_tc], dtype=np.int32)
        payload[f"ids_{i}"] = ids.astype(dt)
    np.savez_compressed(path, **payload)
