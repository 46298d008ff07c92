"""ctypes binding of ``_lib/libtilequant_hip.so`` (C ABI: ``include/tilequant.h``).

The library is built in-tree for gfx950 by ``tilequant_amd.build.build()``.
There is no fallback: if the library is missing, or a tensor is not on a ROCm
device, the calling op raises.
"""
from __future__ import annotations

import ctypes
from pathlib import Path
from typing import Optional

import torch

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libtilequant_hip.so"
ABI_VERSION = 3

TQ_DTYPE = {torch.bfloat16: 0, torch.float16: 1}
TQ_LAYOUT = {"row_major": 0, "mfma": 1}
# flag OR'ed into the GEMM's tile_layout argument: the INT8 codes are token-blocked
TQ_XQ_TOKEN_BLOCKED = 0x100

TQ_ERR_ARG = -1

_LIB: Optional[ctypes.CDLL] = None

_p = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64

# name -> (restype, argtypes); mirrors include/tilequant.h
_SIGNATURES = {
    "tq_error_string": (ctypes.c_char_p, [_i]),
    "tq_abi_version": (_i, []),
    "tq_act_quant_fused": (_i, [_p, _i64, _i64, _i, _i, _i, _p, _i64, _p, _p]),
    "tq_act_quant_token_blocked": (_i, [_p, _i64, _i, _i, _i, _p, _p, _p]),
    "tq_gemm_prefers_token_blocked": (_i, [_i, _i, _i, _i]),
    "tq_read_probe": (_i, [_p, _i64, _p, _p]),
    "tq_act_absmax_workspace_elems": (_i64, [_i, _i]),
    "tq_act_absmax_scales": (_i, [_p, _i64, _i64, _i, _i, _i, _p, _p, _i64, _p]),
    "tq_act_quant_with_scales": (_i, [_p, _i64, _i64, _i, _i, _i, _p, _p, _i64, _p]),
    "tq_act_quant_two_level": (_i, [_p, _i64, _i, _i, _i, _p, _i64, _p, _p, _i64, _p]),
    "tq_quant_tensor_workspace_elems": (_i64, [_i64]),
    "tq_quant_tensor_absmax": (_i, [_p, _i64, _i, _p, _p, _p, _i64, _p]),
    "tq_gemm_workspace_elems": (_i64, [_i, _i, _i, _i, _i]),
    "tq_gemm_mixed_rows": (_i, [_p, _i64, _p,
                                _p, _p, _p, _p,
                                _p, _i64, _i,
                                _p, _p, _p,
                                _p, _i64, _i, _p,
                                _i, _i, _i, _i, _i,
                                _i, _i, _p, _i64, _p]),
    "tq_linear_mixed_fused_max_tokens": (_i, [_i]),
    "tq_linear_mixed_fused_workspace_elems": (_i64, [_i, _i, _i, _i, _i, _i]),
    "tq_test_set_coop_spin": (None, [_i]),
    "tq_gemm_mixed_rows_planned": (_i, [_p, _i64, _p,
                                        _p, _p, _p, _p,
                                        _p, _i64, _i,
                                        _p, _p, _p,
                                        _p, _i64, _i, _p,
                                        _i, _i, _i, _i, _i,
                                        _i, _i, _p, _i64,
                                        _p, _i, _i, _p]),
    "tq_gemm_prefill_plan": (_i, [_p, _p, _p, _i, _i, _p, _i, ctypes.POINTER(_i)]),
    "tq_linear_mixed_fused": (_i, [_p, _i64, _i,
                                   _p, _p, _p, _p,
                                   _p, _p, _p,
                                   _p, _i64, _i, _p,
                                   _i, _i, _i, _i, _i,
                                   _i, _i, _p, _i64, _p]),
    "tq_gemm_mixed_rows_products_i32": (_i, [_p, _i64, _p,
                                             _p, _p, _p, _p,
                                             _p, _i64, _i,
                                             _p, _p, _p,
                                             _p, _i64, _i, _p,
                                             _i, _i, _i, _i, _i,
                                             _i, _i, _p, _i64,
                                             _p, _i, _i,
                                             _p, _i, _i, ctypes.POINTER(_i), _p]),
    "tq_linear_mixed_fused_products_i32": (_i, [_p, _i64, _i,
                                                _p, _p, _p, _p,
                                                _p, _p, _p,
                                                _p, _i64, _i, _p,
                                                _i, _i, _i, _i, _i,
                                                _i, _i, _p, _i64,
                                                _p, _i, _i, ctypes.POINTER(_i), _p]),
    "tq_decode_attention_workspace_elems": (_i64, [_i, _i, _i]),
    "tq_decode_attention_plan": (_i, [_i, _i, _i, _i, _i, _i, _p, _p]),
    "tq_decode_attention": (_i, [_p, _i64, _i64, _p, _p, _i64, _i64, _i64, _p, _p, _i64, _i64,
                                 _i, _i, _i, _i, _i, _i, ctypes.c_float, _p, _i64, _p]),
    "tq_decode_attention_noalloc": (_i, [_p, _i64, _i64, _p, _p, _i64, _i64, _i64, _p, _p, _i64, _i64,
                                         _i, _i, _i, _i, _i, _i, ctypes.c_float, _p]),
    "tq_decode_attention_quant": (_i, [_p, _i64, _i64, _p, _p, _i64, _i64, _i64, _p, _p, _i64, _i64,
                                       _p, _i64, _p, _i, _i, _i, _i, _i, _i, ctypes.c_float, _p, _i64, _p]),
    "tq_decode_attention_rope": (_i, [_p, _i64, _p, _p, _p, _p, _p, _i64, _i64, _i64, _p, _p, _i64, _i64,
                                      _p, _i64, _p, _i, _i, _i, _i, _i, _i, ctypes.c_float, _p, _i64, _p, _p]),
    "tq_greedy_step_workspace_elems": (_i64, [_i]),
    "tq_greedy_step": (_i, [_p, _i64, _i, _i, _i, _p, _i64, _p, _p, _p, _i64, _i, _p, _i, _p, _p]),
    "tq_add_rmsnorm_quant": (_i, [_p, _i64, _p, _i64, _p, ctypes.c_float, _p, _i64, _p, _i64, _p, _i64, _p,
                                  _i, _i, _i, _p, _p]),
    "tq_silu_mul_quant": (_i, [_p, _i64, _p, _i64, _p, _i64, _p, _i, _i, _i, _p, _p]),
    "tq_gemm_l2_warm_ok": (_i, [_i, _i, _i, _i]),
    "tq_add_rmsnorm_rows": (_i, [_p, _i64, _p, _i64, _p, ctypes.c_float, _p, _i64, _p, _i64, _i, _i, _i, _p]),
    "tq_silu_mul_rows": (_i, [_p, _i64, _p, _i64, _i, _i, _i, _p]),
    "tq_rope_prefill": (_i, [_p, _i64, _p, _p, _i64, _p, _i64, _i64, _i64, _p, _p, _i64, _i64, _i64, _i, _i, _i,
                             _i, _i, _i, _i, _p]),
    "tq_rope_cache": (_i, [_p, _i64, _p, _p, _p, _p, _i64, _i64, _p, _p, _i64, _i64, _i64, _i, _i, _i, _i, _i,
                           _i, _p]),
    "tq_pack_int8_tiles": (_i, [_p, _i64, _i, _i, _i, _p, _i64, _i, _i, _p, _p, _p, _p]),
    "tq_pack_16bit_tiles": (_i, [_p, _i64, _i, _i, _i, _p, _i64, _i, _i, _p, _p]),
    "tq_tiles_relayout": (_i, [_p, _p, _i64, _i, _i, _i, _p]),
}



class LinearDesc(ctypes.Structure):
    """Mirror of tq_linear_desc (include/tilequant.h)."""

    _fields_ = [
        ("x", _p), ("out", _p), ("stream", _p),
        ("x_stride", _i64), ("out_stride", _i64),
        ("n", _i), ("m", _i), ("k", _i), ("n_tr", _i), ("n_tc", _i), ("x_dtype", _i), ("out_dtype", _i),
        ("tile_layout", _i), ("fused", _i),
        ("x_int8", _p), ("sx", _p),
        ("int8_tiles", _p), ("int8_scales", _p), ("int8_tile_ids", _p), ("int8_row_ptr", _p),
        ("fp16_tiles", _p), ("fp16_tile_ids", _p), ("fp16_row_ptr", _p),
        ("bias", _p), ("workspace", _p), ("workspace_elems", _i64),
    ]


_SIGNATURES["tq_linear_forward"] = (_i, [ctypes.POINTER(LinearDesc)])


class L2Warm(ctypes.Structure):
    """Mirror of tq_l2_warm (include/tilequant.h): the next decode GEMM's
    packed tiles and row pointers, and the producer's extra workgroup count.
    Passed by address (the trailing ``warm`` argument of the producers); NULL
    means no warm-up."""

    _fields_ = [("int8_tiles", _p), ("fp16_tiles", _p), ("int8_row_ptr", _p), ("fp16_row_ptr", _p),
                ("n_tr", _i), ("blocks", _i)]

EXPORTED_SYMBOLS = tuple(_SIGNATURES)


class NativeLibraryMissing(RuntimeError):
    pass


def load(path: Optional[Path] = None) -> ctypes.CDLL:
    """Load the library and attach signatures.  Loading needs no GPU."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise NativeLibraryMissing(
            f"{p} is not built; run tilequant_amd.build.build() (hipcc --offload-arch=gfx950)"
        )
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.tq_abi_version() != ABI_VERSION:
        raise NativeLibraryMissing(f"{p} has ABI {lib.tq_abi_version()}, expected {ABI_VERSION}; rebuild it")
    if path is None:
        _LIB = lib
    return lib


def lib() -> ctypes.CDLL:
    return _LIB if _LIB is not None else load()


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().tq_error_string(int(rc)).decode()
        if rc == TQ_ERR_ARG:
            raise ValueError(f"{what}: {msg}")
        raise RuntimeError(f"{what} failed (code {rc}): {msg}")


def require_device(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                "tilequant_amd kernels run on a ROCm GPU only (no CPU fallback); got a tensor on "
                f"{t.device}"
            )


def stream_handle(device: torch.device) -> int:
    return int(torch.cuda.current_stream(device).cuda_stream)


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else int(t.data_ptr())


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return TQ_DTYPE[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}; expected torch.bfloat16 or torch.float16") from None
