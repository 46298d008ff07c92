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

import ctypes
import weakref
from typing import Any, Dict, Optional, Tuple

import torch
import torch.nn as nn

from . import _native as nat
from ._config import cfg_value
from .gemm_rows_splitk_64x64 import (PrefillPlan, _fused_workspace, _workspace, fused_max_tokens,
                                     gemm_mixed_rows_splitk, linear_mixed_fused, prefill_plan)
from .pack import Pack, concat_packs_along_rows
from .quantize_activation import quantize_activation_token_blocked, token_blocked_elems
from .quant_utils import (
    activation_tile_absmax_scales,
    quantize_activation_tile_absmax,
    quantize_activation_tile_with_scales,
)

DEFAULT_ACTIVATION_ROW_CHUNK_SIZE = 16384
# Above this many rows the GEMM runs its prefill kernel, which takes a work
# plan (16-bit-heavy row-tile pairs split into single row tiles; _prefill_plan).
PLAN_MIN_ROWS = 64
# Rows up to which cfg.fused_decode = "auto" fuses quantization into the GEMM
# (measured on MI355X: 1 row saves ~2 us per projection, 4 rows break even).
FUSED_AUTO_MAX_ROWS = 2
# ... and up to this many rows when the repeated quantization is cheap: inputs
# of at most FUSED_AUTO_NARROW_K columns whose decode grid (four workgroups
# per 64-row output tile) gives no CU a second workgroup.  Such a workgroup
# quantizes with one thread per 8-column chunk of a row (register + DPP
# absmax, one barrier).  At 4 rows on MI355X (28 layers, cold weights): O
# (3072 x 3072, 192 workgroups) 7.0 us fused vs 7.7 quantize + GEMM, Down
# (3072 x 8192, 192 workgroups) 10.5 vs 11.2; Q/K/V (320 workgroups, 10.0 vs
# 9.8) and Gate/Up (1024, 22.1 vs 14.5) stay two launches.
FUSED_AUTO_NARROW_ROWS = 4
FUSED_AUTO_NARROW_K = 8192


def _device_cus(device: torch.device) -> int:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    cus = _CU_COUNT.get(idx)
    if cus is None:
        cus = _CU_COUNT[idx] = int(torch.cuda.get_device_properties(idx).multi_processor_count)
    return cus


_CU_COUNT: Dict[int, int] = {}
# Sibling projections reuse one activation quantization for inputs of at least
# this many rows (the reference's threshold, mixed_linear.py:20-21).
ACTIVATION_QUANT_CACHE_MIN_ROWS = 32


def _linear_forward():
    fn = _LINEAR_FORWARD[0]
    if fn is None:
        fn = _LINEAR_FORWARD[0] = nat.lib().tq_linear_forward
    return fn


_LINEAR_FORWARD = [None]



def _view_key(t: torch.Tensor) -> Tuple[Any, ...]:
    """What makes two uses of a tensor see the same values: its storage view
    and its version counter (inference tensors have none; they cannot be
    modified in place outside inference mode either)."""
    try:
        version = int(t._version)
    except RuntimeError:
        version = None
    return (t.data_ptr(), t.storage_offset(), tuple(t.shape), tuple(t.stride()), t.dtype, t.device, version)


class ServeOnce:
    """Holds at most one value computed from one source tensor and hands it to
    each consumer at most once.

    The source is referenced weakly: when it dies the value is released.  A
    lookup hits only for the same live tensor with the same view key (so an
    in-place update in between is a miss) and a consumer that has not taken
    the value yet; a consumer asking twice means a new forward pass, which
    must recompute.  With ``consumers`` set, the value is also released once
    that many distinct consumers have taken it.

    Two uses: the INT8 codes + scales of one activation shared by the sibling
    projections that read it (the reference's per-stream sibling cache,
    mixed_linear.py:24-111), and the stacked output of a projection group
    shared by its members (mixed_linear.py:257-333)."""

    __slots__ = ("consumers", "_source", "_key", "_taken", "_value")

    def __init__(self, consumers: Optional[int] = None) -> None:
        self.consumers = consumers
        self.clear()

    def clear(self) -> None:
        self._source = None
        self._key = None
        self._taken: frozenset = frozenset()
        self._value = None

    def take(self, source: torch.Tensor, key, consumer) -> Optional[Any]:
        if self._source is None or self._source() is not source or self._key != key or consumer in self._taken:
            return None
        value = self._value
        self._taken = self._taken | {consumer}
        if self.consumers is not None and len(self._taken) >= self.consumers:
            self.clear()
        return value

    def put(self, source: torch.Tensor, key, consumer, value) -> None:
        self.clear()   # never keep the previous activation's value alive alongside the new one
        if self.consumers is not None and self.consumers <= 1:
            return

        def released(ref, memo=self):
            if memo._source is ref:
                memo.clear()

        try:
            self._source = weakref.ref(source, released)
        except TypeError:
            return
        self._key, self._taken, self._value = key, frozenset((consumer,)), value


# One memo per (device, stream): kernels on one stream run in order, so codes
# made there are complete for every later launch on it.
_SHARED_QUANT: Dict[Tuple[int, int], ServeOnce] = {}


def _blockable(x_work: torch.Tensor) -> bool:
    """Rows the token-blocked quantizer takes: full 64-column tiles, unit
    column stride, 16-byte aligned rows."""
    return (x_work.shape[1] % 64 == 0 and x_work.stride(1) == 1 and x_work.stride(0) % 8 == 0
            and x_work.data_ptr() % 16 == 0)


def _quantize(x_work: torch.Tensor, tile_n: int, blocked: bool) -> Tuple[torch.Tensor, torch.Tensor]:
    if blocked:
        return quantize_activation_token_blocked(x_work)
    return quantize_activation_tile_absmax(x_work, tile_n=tile_n)


def _quantize_for(module: nn.Module, x: torch.Tensor, x_work: torch.Tensor,
                  blocked: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """Codes and scales of ``x_work`` (the 2-D view of ``x``) for ``module``
    (token-blocked when ``blocked``), shared with its sibling projections
    under inference mode for inputs of at least ACTIVATION_QUANT_CACHE_MIN_ROWS
    rows."""
    if x_work.shape[0] < ACTIVATION_QUANT_CACHE_MIN_ROWS or not x_work.is_cuda \
            or not torch.is_inference_mode_enabled():
        return _quantize(x_work, module.tile_n, blocked)
    slot = (x_work.device.index or 0, torch.cuda.current_stream(x_work.device).cuda_stream)
    memo = _SHARED_QUANT.get(slot)
    if memo is None:
        memo = _SHARED_QUANT[slot] = ServeOnce()
    key = (_view_key(x), module.tile_n, blocked)
    hit = memo.take(x, key, id(module))
    if hit is not None:
        return hit
    codes = _quantize(x_work, module.tile_n, blocked)
    memo.put(x, key, id(module), codes)
    return codes


# Eager inputs of fewer rows than this (and below the sibling-cache threshold,
# so sharing semantics are unchanged) run through a cached launch descriptor.
LAUNCH_CACHE_MAX_ROWS = ACTIVATION_QUANT_CACHE_MIN_ROWS - 1
# Descriptors kept per module (each holds its own scratch codes); the oldest
# is dropped beyond this.
LAUNCH_CACHE_MAX_ENTRIES = 64


class _Launch:
    """A validated tq_linear_desc for one (rows, layout, stream, weights) key
    and the scratch it points to; per call only x, out change.  ``bias_copy``
    is the output-dtype copy of a bias of another dtype (None when the
    descriptor points at the bias itself): it is refreshed from the live
    parameter before every launch, so in-place bias updates are always seen."""

    __slots__ = ("desc", "ref", "keep", "bias_copy")

    def __init__(self, desc, keep, bias_copy=None) -> None:
        self.desc = desc
        self.ref = ctypes.byref(desc)
        self.keep = keep   # tensors the descriptor points to
        self.bias_copy = bias_copy


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
        self._launches: Dict[Tuple[Any, ...], _Launch] = {}
        self._blocked_rows: Dict[int, bool] = {}
        self._plan: Optional[Tuple[Optional[PrefillPlan]]] = None   # (plan,) once built

    def _apply(self, fn, recurse=True):
        self._launches = {}   # descriptors point at the old tensors
        self._plan = None
        return super()._apply(fn, recurse)

    # the tile storage order travels with the state_dict
    def get_extra_state(self):
        return {"tile_layout": self.tile_layout}

    def set_extra_state(self, state):
        if isinstance(state, dict) and "tile_layout" in state:
            self.tile_layout = str(state["tile_layout"])

    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys, unexpected_keys,
                              error_msgs):
        # A state_dict that replaces this module's tiles without the layout
        # record was written by the reference (or a module packed in its
        # order): its tiles are row-major.  A dict that does not carry the
        # tiles (a partial strict=False load) leaves the layout alone.
        key = prefix + "_extra_state"
        if key not in state_dict and (prefix + "int8_tiles" in state_dict or prefix + "fp16_tiles" in state_dict):
            self.tile_layout = "row_major"
        self._launches = {}
        self._plan = None
        super()._load_from_state_dict(state_dict, prefix, local_metadata, strict, missing_keys, unexpected_keys,
                                      error_msgs)
        if key not in state_dict and key in missing_keys:
            missing_keys.remove(key)

    def to_pack(self) -> Pack:
        return Pack(M_orig=self.M_orig, K_orig=self.K_orig, M=self.M, K=self.K, tile_m=self.tile_m,
                    tile_n=self.tile_n, n_tr=self.n_tr, n_tc=self.n_tc,
                    **{name: getattr(self, name) for name in _BUFFERS}, tile_layout=self.tile_layout)

    def _out_dtype(self) -> torch.dtype:
        dtype_out = cfg_value(self.cfg, "dtype_out", "fp16")
        return torch.bfloat16 if dtype_out in ("bf16", torch.bfloat16) else torch.float16

    def _activation_row_chunk_size(self) -> int:
        return max(1, int(cfg_value(self.cfg, "activation_row_chunk_size", DEFAULT_ACTIVATION_ROW_CHUNK_SIZE)))

    def _out_bias(self, out_dtype: torch.dtype) -> Optional[torch.Tensor]:
        bias = self.bias
        if bias is None:
            return None
        if bias.dtype != out_dtype or not bias.is_contiguous():
            bias = bias.to(dtype=out_dtype).contiguous()
        return bias

    def _prefill_plan(self, n_rows: int) -> Optional[PrefillPlan]:
        """The prefill kernel's work plan for this weight (None: plain pair
        order).  Built once, on the first call above the decode sizes outside
        graph capture (it reads the row pointers on the host); until then, and
        for decode sizes, calls run without one.  Outputs do not depend on it."""
        if n_rows <= PLAN_MIN_ROWS:
            return None
        if self._plan is None:
            if not self.int8_row_ptr.is_cuda or torch.cuda.is_current_stream_capturing():
                return None
            self._plan = (prefill_plan(int8_tile_ids=self.int8_tile_ids, int8_row_ptr=self.int8_row_ptr,
                                       fp16_row_ptr=self.fp16_row_ptr, n_tr=self.n_tr, n_tc=self.n_tc),)
        return self._plan[0]

    def _gemm_bias(self, x_fp: torch.Tensor, x_int8: torch.Tensor, sx: torch.Tensor,
                   out: Optional[torch.Tensor] = None, x_int8_layout: str = "row_major") -> torch.Tensor:
        out_dtype = self._out_dtype()
        return gemm_mixed_rows_splitk(
            x_fp=x_fp, x_int8=x_int8, sx=sx,
            int8_tiles=self.int8_tiles, int8_scales=self.int8_scales, int8_tile_ids=self.int8_tile_ids,
            int8_row_ptr=self.int8_row_ptr, fp16_tiles=self.fp16_tiles, fp16_tile_ids=self.fp16_tile_ids,
            fp16_row_ptr=self.fp16_row_ptr, M=self.M_orig, K=self.K_orig, n_tr=self.n_tr, n_tc=self.n_tc,
            out_dtype=out_dtype, bias=self._out_bias(out_dtype), out=out, tile_layout=self.tile_layout,
            prefill_plan=self._prefill_plan(int(x_fp.shape[0])), x_int8_layout=x_int8_layout,
        )

    def token_blocked_codes(self, n_rows: int) -> bool:
        """Whether this module quantizes ``n_rows``-row inputs into
        token-blocked codes: where the GEMM's schedule runs faster on them
        (``tq_gemm_prefers_token_blocked``: 17..64 rows, and fewer where the
        codes do not fit the LDS-staged kernel or rows hold 256+ column
        tiles).  Outputs are bitwise those of
        row-major codes; only the operand loads change (each 16-row x 64-column
        slice one contiguous 1 KiB instead of 16 row pieces of 64 bytes)."""
        hit = self._blocked_rows.get(n_rows)
        if hit is None:
            hit = self._blocked_rows[n_rows] = self.tile_n == 64 and bool(nat.lib().tq_gemm_prefers_token_blocked(
                int(n_rows), self.K_orig, self.n_tr, self.n_tc))
        return hit

    def _fused_limit(self) -> int:
        limit = getattr(self, "_fused_rows", None)
        if limit is None:
            limit = self._fused_rows = fused_max_tokens(self.K_orig)
        return limit

    def _fused_rows_for_cfg(self) -> int:
        mode = cfg_value(self.cfg, "fused_decode", None)
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

    def _build_launch(self, x_work: torch.Tensor, stream: int, out_dtype: torch.dtype, fused: bool) -> _Launch:
        """Validate once and fill the descriptor (the checks of the two-launch
        path: dtypes, contiguity, 16-byte aligned tiles)."""
        n, k = x_work.shape
        dev = x_work.device
        if x_work.dtype not in nat.TQ_DTYPE or x_work.stride(1) != 1:
            raise ValueError("x must be a bf16 / fp16 tensor with unit column stride")
        for name in ("int8_tiles", "fp16_tiles"):
            t = getattr(self, name)
            if t.numel() and (not t.is_contiguous() or t.data_ptr() % 16):
                raise ValueError(f"{name} must be contiguous and 16-byte aligned")
        has16 = self.fp16_tiles.numel() != 0
        if has16 and self.fp16_tiles.dtype != x_work.dtype:
            raise ValueError(f"fp16_tiles must have dtype {x_work.dtype}, got {self.fp16_tiles.dtype}")
        bias = self._out_bias(out_dtype)
        keep = [bias]
        d = nat.LinearDesc()
        d.stream = stream
        d.x_stride, d.out_stride = x_work.stride(0), self.M_orig
        d.n, d.m, d.k, d.n_tr, d.n_tc = n, self.M_orig, self.K_orig, self.n_tr, self.n_tc
        d.x_dtype, d.out_dtype = nat.dtype_code(x_work.dtype), nat.dtype_code(out_dtype)
        d.tile_layout, d.fused = nat.TQ_LAYOUT[self.tile_layout], int(fused)
        if not fused and self.token_blocked_codes(n) and _blockable(x_work):
            d.tile_layout |= nat.TQ_XQ_TOKEN_BLOCKED
            x_int8 = torch.empty((token_blocked_elems(n, k),), device=dev, dtype=torch.int8)
            sx = torch.empty((self.n_tc,), device=dev, dtype=torch.float32)
            keep += [x_int8, sx]
            d.x_int8, d.sx = x_int8.data_ptr(), sx.data_ptr()
        elif not fused:
            x_int8 = torch.empty((n, k), device=dev, dtype=torch.int8)
            sx = torch.empty((self.n_tc,), device=dev, dtype=torch.float32)
            keep += [x_int8, sx]
            d.x_int8, d.sx = x_int8.data_ptr(), sx.data_ptr()
        d.int8_tiles, d.int8_scales = self.int8_tiles.data_ptr(), self.int8_scales.data_ptr()
        d.int8_tile_ids, d.int8_row_ptr = self.int8_tile_ids.data_ptr(), self.int8_row_ptr.data_ptr()
        if has16:
            d.fp16_tiles, d.fp16_tile_ids = self.fp16_tiles.data_ptr(), self.fp16_tile_ids.data_ptr()
            d.fp16_row_ptr = self.fp16_row_ptr.data_ptr()
        d.bias = None if bias is None else bias.data_ptr()
        # the per-stream workspace the uncached calls use (split-K partials and
        # counters; the cooperative launch's counters, codes and scales), so an
        # eager call takes the same kernels as a captured one
        if fused:
            d.workspace, d.workspace_elems = _fused_workspace(dev, n, self.M_orig, self.K_orig, self.n_tr,
                                                              self.n_tc, 0)
        else:
            d.workspace, d.workspace_elems = _workspace(dev, n, self.M_orig, self.n_tr, self.n_tc, 0)
        return _Launch(d, keep, bias if bias is not None and bias is not self.bias else None)

    def _cached_forward(self, x_work: torch.Tensor) -> torch.Tensor:
        """Decode-size eager forward through a cached launch descriptor: one
        foreign call per forward, no per-call validation or argument
        marshalling (the role of the reference's CachedLauncher)."""
        n = x_work.shape[0]
        dev = x_work.device
        stream = torch._C._cuda_getCurrentRawStream(dev.index)
        out_dtype = self._out_dtype()
        bias = self.bias
        fused = 0 < n <= min(self._fused_rows_for_cfg(), self._activation_row_chunk_size())
        key = (n, x_work.stride(0), x_work.dtype, dev.index, stream, self.int8_tiles.data_ptr(),
               0 if bias is None else bias.data_ptr(), out_dtype, self.tile_layout, fused, _blockable(x_work))
        launch = self._launches.get(key)
        if launch is None:
            if len(self._launches) >= LAUNCH_CACHE_MAX_ENTRIES:
                self._launches.pop(next(iter(self._launches)))
            launch = self._launches[key] = self._build_launch(x_work, stream, out_dtype, fused)
        if launch.bias_copy is not None:
            launch.bias_copy.copy_(bias)
        out = torch.empty((n, self.M_orig), device=dev, dtype=out_dtype)
        desc = launch.desc
        desc.x = x_work.data_ptr()
        desc.out = out.data_ptr()
        rc = _linear_forward()(launch.ref)
        if rc:
            nat.check(rc, "tq_linear_forward")
        return out

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
        if (0 < n_rows <= LAUNCH_CACHE_MAX_ROWS and x_work.is_cuda and self.int8_tiles.is_cuda
                and not torch.cuda.is_current_stream_capturing()):
            y = self._cached_forward(x_work)
            return y.reshape(in_shape[0], in_shape[1], self.M_orig) if x.dim() == 3 else y
        chunk = self._activation_row_chunk_size()
        if 0 < n_rows <= min(self._fused_rows_for_cfg(), chunk):
            y = self._fused_decode(x_work)
        elif n_rows <= chunk:
            blocked = self.token_blocked_codes(n_rows) and _blockable(x_work)
            x_int8, sx = _quantize_for(self, x, x_work, blocked)
            y = self._gemm_bias(x_fp=x_work, x_int8=x_int8, sx=sx,
                                x_int8_layout="token_blocked" if blocked else "row_major")
        else:
            sx = activation_tile_absmax_scales(x_work, tile_n=self.tile_n)
            y = torch.empty((n_rows, self.M_orig), device=x_work.device, dtype=self._out_dtype())
            for start in range(0, n_rows, chunk):
                self._forward_chunk(x_work[start:start + chunk], sx, y[start:start + chunk])
        if x.dim() == 3:
            y = y.reshape(in_shape[0], in_shape[1], self.M_orig)
        return y


class MixedLinearGroup(nn.Module):
    """Sibling projections of one activation run as ONE stacked MixedLinear
    (mixed_linear.py:265-333): the members' packs concatenated along output
    rows (``concat_packs_along_rows``), one quantization and one GEMM per
    activation, each member served its column slice of the stacked output.
    Every output element comes from the same tile sequence and arithmetic as
    the member's own MixedLinear, so slices equal the members bitwise."""

    def __init__(self, members):
        super().__init__()
        if len(members) < 2:
            raise ValueError("A projection group needs at least two members")
        biased = {m.bias is not None for m in members}
        if len(biased) > 1:
            raise ValueError("Projection group members must all have or all lack bias")
        bias = torch.cat([m.bias.detach() for m in members]) if True in biased else None
        self.linear = MixedLinear(concat_packs_along_rows([m.to_pack() for m in members]), bias, members[0].cfg)
        ends = torch.tensor([m.M_orig for m in members]).cumsum(0).tolist()
        self.bounds = tuple(zip([0] + ends[:-1], ends))
        self._shared = ServeOnce(consumers=len(members))

    def output_for(self, x: torch.Tensor, index: int) -> torch.Tensor:
        """Stacked output for ``x``: computed when member ``index`` is the
        first to ask for this activation (or asks again), reused otherwise."""
        key = _view_key(x)
        out = self._shared.take(x, key, index)
        if out is None:
            out = self.linear(x)
            self._shared.put(x, key, index, out)
        return out

    def reset_pending(self) -> None:
        self._shared.clear()


class MixedLinearSlice(nn.Module):
    """Member ``index`` of a MixedLinearGroup: its column slice of the group's
    stacked output.  The group itself is registered on the parent module (so
    its buffers are counted once); the slice keeps a plain attribute to it."""

    def __init__(self, group: MixedLinearGroup, index: int):
        super().__init__()
        self.__dict__["group"] = group   # plain attribute: bypasses submodule registration
        self.index = int(index)
        self.start, self.stop = group.bounds[self.index]
        self.out_features = self.stop - self.start
        self.in_features = group.linear.K_orig

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.group.output_for(x, self.index)[..., self.start:self.stop]


# (attribute the group is registered under, member attribute names), per parent module
PROJECTION_GROUPS = (
    ("tilequant_qkv", ("q_proj", "k_proj", "v_proj")),
    ("tilequant_gate_up", ("gate_proj", "up_proj")),
)


def _stackable(members) -> bool:
    """Members can share one stacked pack: same input width and tile shape,
    whole output row tiles (so member boundaries are tile boundaries), one
    device, one tile layout, bias on all or none."""
    if not all(isinstance(m, MixedLinear) for m in members):
        return False
    first = members[0]
    same = lambda f: len({f(m) for m in members}) == 1   # noqa: E731
    return (same(lambda m: m.K_orig) and same(lambda m: (m.tile_m, m.tile_n)) and same(lambda m: m.tile_layout)
            and same(lambda m: m.int8_tiles.device) and same(lambda m: m.bias is None)
            and all(m.M_orig % first.tile_m == 0 for m in members))


def fuse_projection_groups(model: nn.Module) -> int:
    """Stack the Q/K/V and Gate/Up MixedLinear siblings of every module into
    MixedLinearGroups (mixed_linear.py:359-386); each member attribute becomes
    a MixedLinearSlice.  Returns the number of groups formed."""
    plan = []
    for parent in model.modules():
        for group_attr, names in PROJECTION_GROUPS:
            members = [getattr(parent, n, None) for n in names]
            if _stackable(members):
                plan.append((parent, group_attr, names, members))
    for parent, group_attr, names, members in plan:
        group = MixedLinearGroup(members)
        parent.add_module(group_attr, group)
        for i, n in enumerate(names):
            setattr(parent, n, MixedLinearSlice(group, i))
    return len(plan)


def reset_projection_groups(model: nn.Module) -> None:
    """Forget every group's shared output (e.g. between independent requests)."""
    for module in model.modules():
        if isinstance(module, MixedLinearGroup):
            module.reset_pending()
