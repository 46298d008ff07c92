"""Mixed INT8/BF16 64x64-tile GEMM (HIP, gfx950).

``gemm_mixed_rows_splitk`` keeps the keyword interface, output validation and
return value of the reference (src/kernels/triton/gemm_rows_splitk_64x64.py:225-323)
and launches ``tq_gemm_mixed_rows`` (``csrc/tq_gemm.hip``) on the current
stream.  One extra keyword, ``tile_layout``, names the storage order inside
each packed tile: ``"row_major"`` (the reference packer's order, the default)
or ``"mfma"`` (the operand-major order this build's packer writes).
"""
from __future__ import annotations

import ctypes
from typing import Dict, List, Optional, Tuple

import torch

from . import _native as nat

# Largest token count the fused quantize + GEMM launch takes (kFusedMaxTokens);
# wide inputs allow fewer (fused_max_tokens).
FUSED_MAX_TOKENS = 16


def fused_max_tokens(K: int) -> int:
    """Largest row count linear_mixed_fused accepts for input width K."""
    return int(nat.lib().tq_linear_mixed_fused_max_tokens(int(K)))


class _SplitKWorkspace:
    """Per (device, stream) zero-initialised fp32 buffer for the split-K
    partials and arrival counters (the analogue of the reference's
    _SplitKWorkspace, gemm_rows_splitk_64x64.py:193-215).  Kernels on one
    stream run in order and leave the counters at zero, so the buffer is
    reused without re-initialisation, also across HIP graph replays.  It only
    grows, and a replaced buffer is kept alive: a captured graph may still
    hold its address.  Growing it while the stream is being captured is an
    error: the zero fill would only be recorded, so eager launches before the
    first replay would find uninitialised arrival counters."""

    def __init__(self) -> None:
        self.buffers: Dict[Tuple[int, int], torch.Tensor] = {}
        self.retired: List[torch.Tensor] = []

    def get(self, device: torch.device, elems: int) -> Optional[torch.Tensor]:
        if elems <= 0:
            return None
        index = device.index if device.index is not None else torch.cuda.current_device()
        key = (index, nat.stream_handle(device))
        buf = self.buffers.get(key)
        if buf is None or buf.numel() < elems:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError(
                    "the split-K workspace must grow during HIP graph capture; run the same call once "
                    "eagerly before capturing")
            if buf is not None:
                self.retired.append(buf)
            buf = torch.zeros((max(elems, 1 << 16),), device=device, dtype=torch.float32)
            self.buffers[key] = buf
        return buf


_WORKSPACE = _SplitKWorkspace()


def _workspace(device, n, M, n_tr, n_tc, split_k):
    elems = int(nat.lib().tq_gemm_workspace_elems(int(n), int(M), int(n_tr), int(n_tc), int(split_k or 0)))
    ws = _WORKSPACE.get(device, elems)
    return (nat.ptr(ws), ws.numel()) if ws is not None else (None, 0)


def _fused_workspace(device, n, M, K, n_tr, n_tc, split_k):
    """The per-stream workspace linear_mixed_fused needs: split-K counters and
    partials, or the cooperative launch's counters, codes and scales."""
    elems = int(nat.lib().tq_linear_mixed_fused_workspace_elems(int(n), int(M), int(K), int(n_tr), int(n_tc),
                                                                int(split_k or 0)))
    ws = _WORKSPACE.get(device, elems)
    return (nat.ptr(ws), ws.numel()) if ws is not None else (None, 0)


class PrefillPlan:
    """Work plan for the prefill GEMM over one packed weight: ``units`` (a
    device int32 tensor) lists row-tile pairs and single row tiles (value
    row | 1 << 30), in dispatch order; the first ``n_first`` units take all
    their token blocks before the others start; ``n_tr`` is the row-tile
    count of the weight it covers (every row tile exactly once).
    ``prefill_plan`` builds one from the row pointers; the outputs do not
    depend on it, as long as it covers the weight's row tiles."""

    __slots__ = ("units", "n_first", "n_tr")

    def __init__(self, units: torch.Tensor, n_first: int, n_tr: int):
        self.units, self.n_first, self.n_tr = units, int(n_first), int(n_tr)


def prefill_plan(*, int8_tile_ids: torch.Tensor, int8_row_ptr: torch.Tensor, fp16_row_ptr: torch.Tensor,
                 n_tr: int, n_tc: int, device=None) -> Optional[PrefillPlan]:
    """Plan the prefill GEMM's work units from the pack's tile bookkeeping:
    row-tile pairs whose many 16-bit tiles would make them finish long after
    the others are split into single row tiles (row order kept).  Returns
    None when no pair needs splitting.
    Copies the row pointers and INT8 ids to the host (a synchronisation):
    call it once per weight, outside graph capture."""
    n_tr, n_tc = int(n_tr), int(n_tc)
    rp8 = int8_row_ptr.detach().to("cpu", torch.int32).contiguous()
    ids8 = int8_tile_ids.detach().to("cpu", torch.int32).contiguous()
    rp16 = fp16_row_ptr.detach().to("cpu", torch.int32).contiguous() if fp16_row_ptr.numel() else None
    if rp8.numel() < n_tr + 1 or (rp16 is not None and rp16.numel() < n_tr + 1):
        raise ValueError("row pointers must have n_tr + 1 entries")
    units = torch.empty(max(n_tr, 1), dtype=torch.int32)
    n_first = ctypes.c_int(0)
    rc = nat.lib().tq_gemm_prefill_plan(
        rp8.data_ptr(), ids8.data_ptr() if ids8.numel() else None,
        rp16.data_ptr() if rp16 is not None else None, n_tr, n_tc, units.data_ptr(), units.numel(),
        ctypes.byref(n_first))
    if rc < 0:   # a count otherwise
        nat.check(rc, "tq_gemm_prefill_plan")
    if rc == 0:
        return None
    dev = device if device is not None else int8_row_ptr.device
    return PrefillPlan(units[:rc].to(dev), n_first.value, n_tr)


def _check_tiles(name: str, t: torch.Tensor, dtype) -> None:
    if t.dtype != dtype:
        raise ValueError(f"{name} must have dtype {dtype}, got {t.dtype}")
    if t.numel() and (not t.is_contiguous() or t.data_ptr() % 16):
        raise ValueError(f"{name} must be contiguous and 16-byte aligned")


def gemm_mixed_rows_splitk(
    *,
    x_fp: torch.Tensor,
    x_int8: torch.Tensor,
    sx: torch.Tensor,
    int8_tiles: torch.Tensor,
    int8_scales: torch.Tensor,
    int8_tile_ids: torch.Tensor,
    int8_row_ptr: torch.Tensor,
    fp16_tiles: torch.Tensor,
    fp16_tile_ids: torch.Tensor,
    fp16_row_ptr: torch.Tensor,
    M: int,
    K: int,
    n_tr: int,
    n_tc: int,
    out_dtype: torch.dtype,
    bias: Optional[torch.Tensor] = None,
    split_k: Optional[int] = None,
    out: Optional[torch.Tensor] = None,
    tile_layout: str = "row_major",
    prefill_plan: Optional[PrefillPlan] = None,
    x_int8_layout: str = "row_major",
    _products=None,
) -> torch.Tensor:
    """Return x @ W^T (+ bias) for a packed mixed INT8/16-bit weight.

    ``bias`` must already have dtype ``out_dtype`` and be contiguous.  ``out``
    (optional) is an (N, M) tensor with unit column stride to write into.
    ``split_k`` (optional, >= 1) fixes how many partitions of each row tile's
    tile list are reduced per output tile (in fixed order); ``None`` picks it
    from the shape.  ``prefill_plan`` (optional, from ``prefill_plan()`` for
    this weight) orders the prefill kernel's work; it does not change the
    result.  ``x_int8_layout="token_blocked"`` takes codes from
    ``quantize_activation_token_blocked`` (1..64 rows; the result is bitwise
    that of the same codes row-major).  Results are bitwise reproducible for
    fixed arguments.
    """
    nat.require_device(x_fp, x_int8, sx, int8_tiles, int8_scales, int8_tile_ids, int8_row_ptr,
                       fp16_tiles, fp16_tile_ids, fp16_row_ptr, bias, out)
    n = int(x_fp.shape[0])
    M, K, n_tr, n_tc = int(M), int(K), int(n_tr), int(n_tc)
    if out is None:
        out = torch.empty((n, M), device=x_fp.device, dtype=out_dtype)
    elif tuple(out.shape) != (n, M) or out.dtype != out_dtype or out.stride(1) != 1:
        raise ValueError("out must be an (N, M) tensor of out_dtype with unit column stride")
    if x_int8_layout == "token_blocked":
        if not 1 <= n <= 64 or K != 64 * n_tc:
            raise ValueError("token-blocked codes take 1..64 rows and K == 64 * n_tc")
        if (x_int8.dtype != torch.int8 or x_int8.dim() != 1 or x_int8.numel() != 16 * ((n + 15) // 16) * K
                or not x_int8.is_contiguous()):
            raise ValueError("token-blocked x_int8 must be a flat contiguous int8 tensor of 16 * ceil(N / 16) * K codes")
        x_int8_stride, layout_flag = K, nat.TQ_XQ_TOKEN_BLOCKED
    elif x_int8_layout == "row_major":
        if x_int8.dim() != 2 or x_int8.shape[0] != n or x_int8.shape[1] < K or x_int8.stride(1) != 1:
            raise ValueError("x_int8 must be an (N, >=K) int8 tensor with unit column stride")
        x_int8_stride, layout_flag = x_int8.stride(0), 0
    else:
        raise ValueError(f"x_int8_layout must be 'row_major' or 'token_blocked', got {x_int8_layout!r}")
    if x_fp.dim() != 2 or x_fp.shape[1] < K or x_fp.stride(1) != 1:
        raise ValueError("x_fp must be an (N, >=K) tensor with unit column stride")
    if sx.dtype != torch.float32 or sx.numel() < n_tc or not sx.is_contiguous():
        raise ValueError("sx must be a contiguous float32 tensor of n_tc scales")
    _check_tiles("int8_tiles", int8_tiles, torch.int8)
    has16 = fp16_tiles.numel() != 0
    if has16:
        _check_tiles("fp16_tiles", fp16_tiles, x_fp.dtype)
    if bias is not None and (bias.dtype != out_dtype or not bias.is_contiguous() or bias.numel() < M):
        raise ValueError("bias must be a contiguous tensor of out_dtype with M entries")
    if split_k is not None and int(split_k) < 1:
        raise ValueError(f"split_k must be >= 1, got {split_k}")
    if tile_layout not in nat.TQ_LAYOUT:
        raise ValueError(f"tile_layout must be one of {tuple(nat.TQ_LAYOUT)}, got {tile_layout!r}")
    for name, t in (("int8_tile_ids", int8_tile_ids), ("int8_row_ptr", int8_row_ptr),
                    ("fp16_tile_ids", fp16_tile_ids), ("fp16_row_ptr", fp16_row_ptr)):
        if t.dtype != torch.int32 or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous int32 tensor")
    if n == 0 or M == 0:
        return out
    ws_ptr, ws_elems = _workspace(x_fp.device, n, M, n_tr, n_tc, split_k)
    args = (nat.ptr(x_int8), x_int8_stride, nat.ptr(sx),
            nat.ptr(int8_tiles), nat.ptr(int8_scales), nat.ptr(int8_tile_ids), nat.ptr(int8_row_ptr),
            nat.ptr(x_fp), x_fp.stride(0), nat.dtype_code(x_fp.dtype),
            nat.ptr(fp16_tiles) if has16 else None, nat.ptr(fp16_tile_ids) if has16 else None,
            nat.ptr(fp16_row_ptr) if has16 else None,
            nat.ptr(out), out.stride(0), nat.dtype_code(out_dtype), nat.ptr(bias),
            n, M, K, n_tr, n_tc, int(split_k or 0), nat.TQ_LAYOUT[tile_layout] | layout_flag, ws_ptr, ws_elems)
    units = None
    if prefill_plan is not None:
        units = prefill_plan.units
        if units.device != x_fp.device or units.dtype != torch.int32 or not units.is_contiguous():
            raise ValueError("prefill_plan.units must be a contiguous int32 tensor on the input's device")
        if (prefill_plan.n_tr != n_tr or not 0 < units.numel() <= n_tr
                or not 0 <= prefill_plan.n_first <= units.numel()):
            raise ValueError(f"prefill_plan covers {prefill_plan.n_tr} row tiles, the weight has {n_tr}")
    if _products is not None:   # test-only DUMP launch (gemm_mixed_rows_products_i32)
        prod, row0, rows, kernel = _products
        rc = nat.lib().tq_gemm_mixed_rows_products_i32(
            *args, nat.ptr(units), units.numel() if units is not None else 0,
            prefill_plan.n_first if units is not None else 0, nat.ptr(prod), row0, rows, ctypes.byref(kernel),
            nat.stream_handle(x_fp.device))
        nat.check(rc, "tq_gemm_mixed_rows_products_i32")
    elif units is not None:
        rc = nat.lib().tq_gemm_mixed_rows_planned(*args, nat.ptr(units), units.numel(), prefill_plan.n_first,
                                                  nat.stream_handle(x_fp.device))
        nat.check(rc, "tq_gemm_mixed_rows_planned")
    else:
        rc = nat.lib().tq_gemm_mixed_rows(*args, nat.stream_handle(x_fp.device))
        nat.check(rc, "tq_gemm_mixed_rows")
    return out


def linear_mixed_fused(
    *,
    x_fp: torch.Tensor,
    int8_tiles: torch.Tensor,
    int8_scales: torch.Tensor,
    int8_tile_ids: torch.Tensor,
    int8_row_ptr: torch.Tensor,
    fp16_tiles: torch.Tensor,
    fp16_tile_ids: torch.Tensor,
    fp16_row_ptr: torch.Tensor,
    M: int,
    K: int,
    n_tr: int,
    n_tc: int,
    out_dtype: torch.dtype,
    bias: Optional[torch.Tensor] = None,
    split_k: Optional[int] = None,
    out: Optional[torch.Tensor] = None,
    tile_layout: str = "row_major",
    _products=None,
) -> torch.Tensor:
    """Activation quantization + mixed tile GEMM in ONE launch (decode sizes,
    at most FUSED_MAX_TOKENS rows).  Same result, bit for bit, as
    ``quantize_activation_tile_absmax`` followed by ``gemm_mixed_rows_splitk``
    with the same ``split_k``; no reference counterpart (the reference always
    launches the two kernels, mixed_linear.py:233-239).  Shapes with too many
    rows x columns for the LDS-staged quantizing kernel run cooperatively: 8
    workgroups quantize once into the per-stream workspace while the GEMM
    workgroups' weight loads are in flight (tq_linear_mixed_fused)."""
    nat.require_device(x_fp, int8_tiles, int8_scales, int8_tile_ids, int8_row_ptr, fp16_tiles, fp16_tile_ids,
                       fp16_row_ptr, bias, out)
    n = int(x_fp.shape[0])
    M, K, n_tr, n_tc = int(M), int(K), int(n_tr), int(n_tc)
    if n > fused_max_tokens(K):
        raise ValueError(f"linear_mixed_fused takes at most {fused_max_tokens(K)} rows for K={K}, got {n}")
    if x_fp.dim() != 2 or x_fp.shape[1] < K or x_fp.stride(1) != 1:
        raise ValueError("x_fp must be an (N, >=K) tensor with unit column stride")
    if out is None:
        out = torch.empty((n, M), device=x_fp.device, dtype=out_dtype)
    elif tuple(out.shape) != (n, M) or out.dtype != out_dtype or out.stride(1) != 1:
        raise ValueError("out must be an (N, M) tensor of out_dtype with unit column stride")
    _check_tiles("int8_tiles", int8_tiles, torch.int8)
    has16 = fp16_tiles.numel() != 0
    if has16:
        _check_tiles("fp16_tiles", fp16_tiles, x_fp.dtype)
    if bias is not None and (bias.dtype != out_dtype or not bias.is_contiguous() or bias.numel() < M):
        raise ValueError("bias must be a contiguous tensor of out_dtype with M entries")
    if n == 0 or M == 0:
        return out
    ws_ptr, ws_elems = _fused_workspace(x_fp.device, n, M, K, n_tr, n_tc, split_k)
    args = (nat.ptr(x_fp), x_fp.stride(0), nat.dtype_code(x_fp.dtype),
            nat.ptr(int8_tiles), nat.ptr(int8_scales), nat.ptr(int8_tile_ids), nat.ptr(int8_row_ptr),
            nat.ptr(fp16_tiles) if has16 else None, nat.ptr(fp16_tile_ids) if has16 else None,
            nat.ptr(fp16_row_ptr) if has16 else None,
            nat.ptr(out), out.stride(0), nat.dtype_code(out_dtype), nat.ptr(bias),
            n, M, K, n_tr, n_tc, int(split_k or 0), nat.TQ_LAYOUT[tile_layout], ws_ptr, ws_elems)
    if _products is not None:   # test-only DUMP launch (gemm_mixed_rows_products_i32)
        prod, row0, rows, kernel = _products
        rc = nat.lib().tq_linear_mixed_fused_products_i32(*args, nat.ptr(prod), row0, rows, ctypes.byref(kernel),
                                                          nat.stream_handle(x_fp.device))
        nat.check(rc, "tq_linear_mixed_fused_products_i32")
    else:
        rc = nat.lib().tq_linear_mixed_fused(*args, nat.stream_handle(x_fp.device))
        nat.check(rc, "tq_linear_mixed_fused")
    return out


# TQ_KERNEL_* codes of include/tilequant.h
KERNEL_FAMILIES = {1: "decode", 2: "decode_quant", 3: "splitk", 4: "splitk_token_blocked", 5: "splitk_quant",
                   6: "prefill_v5", 7: "prefill_v3", 8: "prefill_async", 9: "prefill_register", 10: "decode_coop",
                   11: "decode_quant_help"}


def gemm_mixed_rows_products_i32(*, rows: Optional[Tuple[int, int]] = None, fused: bool = False, **kwargs):
    """TEST ONLY.  Runs ``gemm_mixed_rows_splitk(**kwargs)`` -- or, with
    ``fused=True``, ``linear_mixed_fused(**kwargs)`` -- through the DUMP
    instantiation of the very kernel the automatic schedule picks for those
    arguments, and returns ``(out, products, kernel)``: the usual output, the
    exact INT32 products int32 [T8, rows, 64] of every INT8 tile with token
    rows ``row0 .. row0 + count - 1`` (``rows=(row0, count)``, default all) as
    that kernel's v_mfma_i32_16x16x64_i8 produced them before the scale FMA,
    and the kernel family's name (``KERNEL_FAMILIES``).  The quantity is the
    reference's tl.dot(x_i8, w_i8^T) (gemm_rows_splitk_64x64.py:125-137).
    bf16 activations only."""
    x_fp = kwargs["x_fp"]
    n = int(x_fp.shape[0])
    row0, count = (0, n) if rows is None else (int(rows[0]), int(rows[1]))
    if not (0 <= row0 and 1 <= count <= n - row0):
        raise ValueError(f"rows must lie inside the {n} input rows, got {rows}")
    t8 = int(kwargs["int8_tiles"].shape[0])
    prod = torch.full((max(t8, 1), count, 64), -2**31, device=x_fp.device, dtype=torch.int32)
    kernel = ctypes.c_int(0)
    if fused:
        out = linear_mixed_fused(**kwargs, _products=(prod, row0, count, kernel))
    else:
        out = gemm_mixed_rows_splitk(**kwargs, _products=(prod, row0, count, kernel))
    return out, prod[:t8], KERNEL_FAMILIES.get(kernel.value, str(kernel.value))
