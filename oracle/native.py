"""ctypes wrapper of oracle/tq_oracle.c (built as oracle/libtq_oracle.so).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
LIB_PATH = _HERE / "libtq_oracle.so"
_LIB = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(dtype=np.int8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return LIB_PATH


def lib():
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        L.tqo_act_scales.argtypes = [_f32p, ctypes.c_long, ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p]
        L.tqo_act_quant.argtypes = [_f32p, ctypes.c_long, ctypes.c_int, ctypes.c_int, _f32p, _i8p, ctypes.c_long]
        L.tqo_weight_tiles_quant.argtypes = [_f32p, ctypes.c_long, _f32p, _i8p]
        L.tqo_tile_products_i32.argtypes = [_i8p, ctypes.c_long, ctypes.c_int, ctypes.c_int, _i8p,
                                            _i32p, ctypes.c_long, ctypes.c_int, _i32p]
        vp = ctypes.c_void_p
        L.tqo_gemm_mixed.argtypes = [_i8p, ctypes.c_long, _f32p, _f32p, ctypes.c_long,
                                     _i8p, _f32p, _i32p, _i32p, vp, vp, vp, vp,
                                     ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_int, _f32p, vp, vp]
        L.tqo_round_to_dtype.argtypes = [ctypes.c_float, ctypes.c_int]
        L.tqo_round_to_dtype.restype = ctypes.c_float
        L.tqo_num_threads.restype = ctypes.c_int
        _LIB = L
    return _LIB


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def num_threads() -> int:
    return int(lib().tqo_num_threads())


def act_scales(x: np.ndarray, is_bf16: bool = True) -> np.ndarray:
    x = _c(x, np.float32)
    n, k = x.shape
    sx = np.empty(((k + 63) // 64,), np.float32)
    lib().tqo_act_scales(x, k, n, k, int(is_bf16), sx)
    return sx


def act_quant(x: np.ndarray, sx: np.ndarray) -> np.ndarray:
    x = _c(x, np.float32)
    n, k = x.shape
    q = np.empty((n, k), np.int8)
    lib().tqo_act_quant(x, k, n, k, _c(sx, np.float32), q, k)
    return q


def weight_tiles_quant(tiles: np.ndarray):
    t = _c(tiles, np.float32)
    T = t.shape[0]
    sw = np.empty((T,), np.float32)
    q = np.empty((T, 64, 64), np.int8)
    lib().tqo_weight_tiles_quant(t, T, sw, q)
    return q, sw


def tile_products_i32(xq, w8, ids8, n_tc, K=None) -> np.ndarray:
    xq = _c(xq, np.int8)
    n, k = xq.shape
    K = k if K is None else K
    ids8 = _c(ids8, np.int32)
    out = np.empty((ids8.size, n, 64), np.int32)
    lib().tqo_tile_products_i32(xq, k, n, K, _c(w8, np.int8), ids8, ids8.size, n_tc, out)
    return out


def gemm_mixed(xq, sx, x, w8, sw8, ids8, rp8, w16, ids16, rp16, n_tr, n_tc, M, K,
               bias=None, out_is_bf16=True, want_f64=False):
    """Reference-order fp32 result (as float values on the output grid), and
    optionally (acc64, sumabs) in float64."""
    xq = _c(xq, np.int8)
    x = _c(x, np.float32)
    n = xq.shape[0]
    y = np.empty((n, M), np.float32)
    acc64 = np.empty((n, M), np.float64) if want_f64 else None
    sab = np.empty((n, M), np.float64) if want_f64 else None
    w16c = _c(w16, np.float32) if w16 is not None and np.asarray(w16).size else None
    ids16c = _c(ids16, np.int32)
    rp16c = _c(rp16, np.int32)
    biasc = _c(bias, np.float32) if bias is not None else None

    def ptr(a):
        return None if a is None else a.ctypes.data_as(ctypes.c_void_p)

    lib().tqo_gemm_mixed(xq, xq.shape[1], _c(sx, np.float32), x, x.shape[1],
                         _c(w8, np.int8) if np.asarray(w8).size else np.zeros((1,), np.int8),
                         _c(sw8, np.float32) if np.asarray(sw8).size else np.zeros((1,), np.float32),
                         _c(ids8, np.int32) if np.asarray(ids8).size else np.zeros((1,), np.int32),
                         _c(rp8, np.int32),
                         ptr(w16c), ptr(ids16c), ptr(rp16c), ptr(biasc),
                         n, M, K, n_tr, n_tc, int(out_is_bf16), y, ptr(acc64), ptr(sab))
    if want_f64:
        return y, acc64, sab
    return y


def set_threads(n: int) -> None:
    os.environ["OMP_NUM_THREADS"] = str(int(n))
