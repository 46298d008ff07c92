"""Decode attention over a static KV cache (HIP, gfx950).

``decode_attention`` runs ``tq_decode_attention`` (``csrc/tq_attention.hip``):
one query token per sequence against the valid prefix ``seq_used[b]`` of a
preallocated cache, the length read on the device so that one captured launch
serves every decode position.  It takes the place of the reference graph
decoder's ``aten._flash_attention_forward(..., seqused_k=...)`` call
(src/runtime/graph_decode.py:56-71).
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _native as nat


def decode_attention_workspace(batch: int, q_heads: int, max_len: int, device) -> torch.Tensor:
    """fp32 scratch for the split partials of ``decode_attention``."""
    elems = int(nat.lib().tq_decode_attention_workspace_elems(int(batch), int(q_heads), int(max_len)))
    return torch.empty((max(elems, 1),), device=device, dtype=torch.float32)


def decode_attention(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    seq_used: torch.Tensor,
    *,
    scale: float,
    out: Optional[torch.Tensor] = None,
    workspace: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """softmax(scale * q k^T) v over keys [0, seq_used[b]) of each sequence.

    query: [B, Hq, D] (any strides with a unit last stride); key_cache /
    value_cache: [B, Hkv, L, D] views sharing strides (head- or token-major
    storage); seq_used: int32 [B] on the device.  Returns [B, Hq, D] in the
    query dtype (or writes ``out``)."""
    nat.require_device(query, key_cache, value_cache, seq_used, out, workspace)
    if query.dim() != 3 or key_cache.dim() != 4 or key_cache.shape != value_cache.shape:
        raise ValueError("expected query [B, Hq, D] and caches [B, Hkv, L, D] of one shape")
    if key_cache.stride() != value_cache.stride():
        raise ValueError("key and value caches must share strides")
    B, Hq, D = query.shape
    _, Hkv, L, Dk = key_cache.shape
    if Dk != D or key_cache.shape[0] != B:
        raise ValueError("query and cache shapes disagree")
    if query.stride(-1) != 1 or key_cache.stride(-1) != 1:
        raise ValueError("the head dimension must have unit stride")
    if seq_used.dtype != torch.int32 or seq_used.numel() < B:
        raise ValueError("seq_used must be an int32 tensor with one entry per sequence")
    if out is None:
        out = torch.empty((B, Hq, D), device=query.device, dtype=query.dtype)
    if workspace is None:
        workspace = decode_attention_workspace(B, Hq, L, query.device)
    rc = nat.lib().tq_decode_attention(
        nat.ptr(query), query.stride(0), query.stride(1),
        nat.ptr(key_cache), nat.ptr(value_cache), key_cache.stride(0), key_cache.stride(2), key_cache.stride(1),
        nat.ptr(seq_used), nat.ptr(out), out.stride(0), out.stride(1),
        nat.dtype_code(query.dtype), B, Hq, Hkv, D, L, float(scale),
        nat.ptr(workspace), workspace.numel(), nat.stream_handle(query.device))
    nat.check(rc, "tq_decode_attention")
    return out
