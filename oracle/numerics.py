"""numpy restatement of the TileQuant quantization and tile-GEMM closed forms.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

All functions take numpy arrays.  bf16 data is carried as uint16 bit patterns
(``*_bits``) or as float32 values that are exactly representable in bf16.
"""
from __future__ import annotations

import numpy as np

TILE = 64
INT8_MAX = np.float32(127.0)


# ---------------------------------------------------------------------------
# dtype grids
# ---------------------------------------------------------------------------

def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(v: np.ndarray) -> np.ndarray:
    """Round float32 to bf16 (round-half-even), returning uint16 bit patterns."""
    u = np.asarray(v, dtype=np.float32).view(np.uint32).astype(np.uint64)
    special = (u & 0x7F800000) == 0x7F800000
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    out = np.where(special, u >> 16, rounded)
    return out.astype(np.uint16)


def round_bf16(v: np.ndarray) -> np.ndarray:
    return bf16_bits_to_f32(f32_to_bf16_bits(v))


def round_to_dtype(v: np.ndarray, is_bf16: bool) -> np.ndarray:
    v = np.asarray(v, dtype=np.float32)
    if is_bf16:
        return round_bf16(v)
    with np.errstate(over="ignore"):
        return v.astype(np.float16).astype(np.float32)


def bf16_ulp(v: np.ndarray) -> np.ndarray:
    """Spacing of the bf16 grid at |v| (8 significant bits)."""
    a = np.abs(np.asarray(v, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -126)))
    return np.exp2(np.maximum(e, -126.0) - 7.0)


# ---------------------------------------------------------------------------
# activation quantization (quantize_activation.py:29-43, 66-71, 100-109;
# quant_utils.py:68-74, 109-115)
# ---------------------------------------------------------------------------

def _pad_cols(x: np.ndarray, n_tc: int) -> np.ndarray:
    n, k = x.shape
    if k == n_tc * TILE:
        return x
    out = np.zeros((n, n_tc * TILE), dtype=x.dtype)
    out[:, :k] = x
    return out


def act_tile_scales(x: np.ndarray, is_bf16: bool = True) -> np.ndarray:
    """sx[c] = 1 if a == 0 else f32(round_dtype(f32(a) / 127)), a = max|x[:, tile c]|.

    The max runs over ALL rows of the call (one scale per 64-column tile).
    """
    x = np.asarray(x, dtype=np.float32)
    n, k = x.shape
    n_tc = (k + TILE - 1) // TILE
    if n_tc == 0:
        return np.zeros((0,), dtype=np.float32)
    if n == 0:
        return np.ones((n_tc,), dtype=np.float32)
    a = np.abs(_pad_cols(x, n_tc)).reshape(n, n_tc, TILE).max(axis=(0, 2))
    with np.errstate(divide="ignore", invalid="ignore"):
        s = round_to_dtype(a / INT8_MAX, is_bf16)
    return np.where(a > 0, s, np.float32(1.0)).astype(np.float32)


def quant_codes(v: np.ndarray, s: np.ndarray) -> np.ndarray:
    """max(min(rint(f32(v) / s), 127), -127) as int8 (IEEE divide, half-even).

    min/max ignore NaN (np.fmin/np.fmax), in the order of the reference kernel
    (quantize_activation.py:71), so 0/0 from a zero activation scale gives 127.
    """
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        q = np.rint(np.asarray(v, dtype=np.float32) / np.asarray(s, dtype=np.float32))
    return np.fmax(np.fmin(q, np.float32(127)), np.float32(-127)).astype(np.int8)


def act_quant_codes(x: np.ndarray, sx: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    n, k = x.shape
    cols = np.arange(k) // TILE
    return quant_codes(x, np.asarray(sx, dtype=np.float32)[cols][None, :])


def act_quant(x: np.ndarray, is_bf16: bool = True):
    sx = act_tile_scales(x, is_bf16)
    return act_quant_codes(x, sx), sx


# ---------------------------------------------------------------------------
# one scale per tensor (quant_utils.py:17-37 quantize_activation_absmax /
# quantize_activation_per_tensor_absmax, :138-148 quantize_weight_tile_absmax)
# ---------------------------------------------------------------------------

def tensor_quant(x: np.ndarray, dtype: str = "bf16"):
    """(codes int8 like x, scale f32) for x holding values of `dtype`
    ("bf16", "fp16" or "fp32").

    The reference's torch expressions: max_abs = x.abs().max() (exact);
    sx = (max_abs / 127.0).to(float32) -- the quotient stays in x's dtype, so
    it is f32(a) / 127 rounded to that dtype; scale 1 when max_abs == 0 (or x is
    empty).  x_fp / sx divides a 16-bit tensor by a 0-dim fp32 tensor, which
    torch computes in fp32 and rounds to x's dtype; torch.round is half-even;
    clamp to [-127, 127]; cast to int8.  (quant_utils.py:17-32, 138-148)
    """
    x = np.asarray(x, dtype=np.float32)
    rnd = (lambda v: np.asarray(v, dtype=np.float32)) if dtype == "fp32" else (
        lambda v: round_to_dtype(v, dtype == "bf16"))
    if x.size == 0:
        return np.zeros(x.shape, np.int8), np.float32(1.0)
    a = np.float32(np.max(np.abs(x)))
    if a == 0:
        return np.zeros(x.shape, np.int8), np.float32(1.0)
    s = np.float32(rnd(np.float32(a) / np.float32(127.0)))
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        q = np.rint(rnd(x / s))
    return np.clip(q, -127, 127).astype(np.int8), s


# ---------------------------------------------------------------------------
# weight tiles (pack.py:119-130, 163-167)
# ---------------------------------------------------------------------------

def weight_tile_scales(tiles: np.ndarray) -> np.ndarray:
    """sw = 1 if a == 0 else f32(a) / 127 in IEEE fp32 (not rounded to bf16)."""
    t = np.asarray(tiles, dtype=np.float32)
    a = np.abs(t.reshape(t.shape[0], -1)).max(axis=1) if t.shape[0] else np.zeros((0,), np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        s = (a / INT8_MAX).astype(np.float32)
    return np.where(a == 0, np.float32(1.0), s).astype(np.float32)


def weight_tile_quant(tiles: np.ndarray):
    """tiles [T, 64, 64] float values -> (codes int8 [T, 64, 64], sw f32 [T])."""
    t = np.asarray(tiles, dtype=np.float32)
    sw = weight_tile_scales(t)
    return quant_codes(t, sw[:, None, None]), sw


def tiles_of(w: np.ndarray, ids: np.ndarray, n_tc: int) -> np.ndarray:
    """Row-major 64x64 tiles of a padded [M, K] matrix for the given flat ids."""
    w = np.asarray(w)
    m, k = w.shape
    n_tr = m // TILE
    view = w.reshape(n_tr, TILE, n_tc, TILE).transpose(0, 2, 1, 3)
    ids = np.asarray(ids, dtype=np.int64)
    return np.ascontiguousarray(view[ids // n_tc, ids % n_tc])


# ---------------------------------------------------------------------------
# tile GEMM (gemm_rows_splitk_64x64.py:119-153, 184-190)
# ---------------------------------------------------------------------------

def tile_products_i32(xq: np.ndarray, w8: np.ndarray, ids8: np.ndarray, n_tc: int) -> np.ndarray:
    """Exact P[t, n, j] = sum_k xq[n, 64c+k] * w8[t, j, k] with c = ids8[t] % n_tc.

    Columns beyond K read as 0.  Returns int32 [T8, N, 64].
    """
    xq = np.asarray(xq, dtype=np.int8)
    n, k = xq.shape
    xp = _pad_cols(xq, n_tc).astype(np.int64).reshape(n, n_tc, TILE)
    c = np.asarray(ids8, dtype=np.int64) % n_tc
    xt = xp[:, c, :].transpose(1, 0, 2)                     # [T, N, 64]
    w = np.asarray(w8, dtype=np.int64)                      # [T, 64j, 64k]
    p = np.matmul(xt, w.transpose(0, 2, 1))                 # [T, N, 64j]
    return p.astype(np.int32)


def gemm_mixed_f64(xq, sx, x, w8, sw8, ids8, rp8, w16, ids16, rp16, n_tr, n_tc, M, K):
    """float64 sum of every tile term, plus sum |term| (the error-bound input).

    Returns (acc64 [N, M], sumabs [N, M]).
    """
    xq = np.asarray(xq, dtype=np.int8)
    x = np.asarray(x, dtype=np.float64)
    n = xq.shape[0]
    acc = np.zeros((n, n_tr * TILE), dtype=np.float64)
    sab = np.zeros_like(acc)
    ids8 = np.asarray(ids8, dtype=np.int64)
    if ids8.size:
        p = tile_products_i32(xq, w8, ids8, n_tc).astype(np.float64)
        s = np.asarray(sx, np.float64)[ids8 % n_tc] * np.asarray(sw8, np.float64)
        terms = p * s[:, None, None]                      # [T, N, 64]
        rows = ids8 // n_tc
        for r in np.unique(rows):
            sel = rows == r
            acc[:, r * TILE:(r + 1) * TILE] += terms[sel].sum(axis=0)
            sab[:, r * TILE:(r + 1) * TILE] += np.abs(terms[sel]).sum(axis=0)
    ids16 = np.asarray(ids16, dtype=np.int64)
    if ids16.size:
        xp = _pad_cols(x, n_tc).reshape(n, n_tc, TILE)
        w = np.asarray(w16, dtype=np.float64)
        for t, tid in enumerate(ids16):
            r, c = int(tid // n_tc), int(tid % n_tc)
            prod = xp[:, c, None, :] * w[t][None, :, :]       # [N, 64j, 64k]
            acc[:, r * TILE:(r + 1) * TILE] += prod.sum(axis=2)
            sab[:, r * TILE:(r + 1) * TILE] += np.abs(prod).sum(axis=2)
    return acc[:, :M], sab[:, :M]


def gemm_tolerance(acc64: np.ndarray, sumabs: np.ndarray, n_tc: int, bias=None) -> np.ndarray:
    """Per-element bound on |y_device - y_ref| for a bf16 output.

    Two bf16 ulps of the exact result plus the
    worst-case fp32 accumulation error, (n_tc + 64) * 2^-24 * sum|term|
    (n_tc tile additions, up to 64 in-MFMA additions).  With a bias the
    result is rounded twice, so one more ulp of the pre-bias value is allowed.
    """
    ref = acc64 if bias is None else acc64 + np.asarray(bias, np.float64)[None, :]
    tol = 2.0 * bf16_ulp(ref) + (n_tc + 64) * 2.0 ** -24 * sumabs
    if bias is not None:
        tol = tol + bf16_ulp(acc64)
    return tol


def dense_dequant_reference(xq, sx, x, w8, sw8, ids8, w16, ids16, n_tr, n_tc, M, K):
    """Closed-form cross-check: y = Xdq @ Wmixed^T in float64 where the tile
    scales are folded into a dense matrix.  Equal to gemm_mixed_f64's acc
    because sx[c]*sw[t] factor out of each tile's integer dot."""
    xq = np.asarray(xq, dtype=np.int8)
    n = xq.shape[0]
    Kp = n_tc * TILE
    xdq = _pad_cols(xq.astype(np.float64), n_tc) * np.repeat(np.asarray(sx, np.float64), TILE)[None, :]
    xf = _pad_cols(np.asarray(x, np.float64), n_tc)
    acc = np.zeros((n, n_tr * TILE))
    wd8 = np.zeros((n_tr * TILE, Kp))
    wd16 = np.zeros((n_tr * TILE, Kp))
    for t, tid in enumerate(np.asarray(ids8, np.int64)):
        r, c = int(tid // n_tc), int(tid % n_tc)
        wd8[r * TILE:(r + 1) * TILE, c * TILE:(c + 1) * TILE] = np.asarray(w8[t], np.float64) * float(sw8[t])
    for t, tid in enumerate(np.asarray(ids16, np.int64)):
        r, c = int(tid // n_tc), int(tid % n_tc)
        wd16[r * TILE:(r + 1) * TILE, c * TILE:(c + 1) * TILE] = np.asarray(w16[t], np.float64)
    acc = xdq @ wd8.T + xf @ wd16.T
    return acc[:, :M]
