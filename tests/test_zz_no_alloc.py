"""GPU: the allocation-free decode attention entry point (tq_decode_attention_noalloc).

It has no reference counterpart: it is tq_decode_attention with the split
records in the library's fixed per-GPU device array instead of a caller
workspace.  Bar: outputs bitwise equal to tq_decode_attention with a
workspace, on two calls in a row (the second smaller, so it runs over what the
first left in the array), and a size past the array's capacity refused
without a launch.
"""
from __future__ import annotations

import pytest
import torch

from tilequant_amd import _native as nat
from tilequant_amd.attention import decode_attention

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _inputs(B, Hq, Hkv, L, lens, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((B, Hq, 128), generator=g).to(torch.bfloat16).to(DEV)
    k = torch.randn((B, Hkv, L, 128), generator=g).to(torch.bfloat16).to(DEV)
    v = torch.randn((B, Hkv, L, 128), generator=g).to(torch.bfloat16).to(DEV)
    seq = torch.tensor(lens, dtype=torch.int32, device=DEV)
    return q, k, v, seq


def _noalloc(q, k, v, seq, scale):
    B, Hq, D = q.shape
    _, Hkv, L, _ = k.shape
    out = torch.full((B, Hq, D), float("nan"), dtype=q.dtype, device=DEV)
    rc = nat.lib().tq_decode_attention_noalloc(
        nat.ptr(q), q.stride(0), q.stride(1), nat.ptr(k), nat.ptr(v), k.stride(0), k.stride(2), k.stride(1),
        nat.ptr(seq), nat.ptr(out), out.stride(0), out.stride(1), nat.dtype_code(q.dtype), B, Hq, Hkv, D, L,
        float(scale), nat.stream_handle(DEV))
    return rc, out


def test_noalloc_attention_equals_workspace_entry_on_consecutive_calls():
    scale = 128 ** -0.5
    cases = [(4, 24, 8, 2304, [2304, 2049, 1, 1500], 1),   # the Llama-3.2-3B decode shape
             (2, 8, 2, 300, [300, 17], 2)]                  # smaller: reuses the array the first call filled
    for B, Hq, Hkv, L, lens, seed in cases:
        q, k, v, seq = _inputs(B, Hq, Hkv, L, lens, seed)
        ref = decode_attention(q, k, v, seq, scale=scale)
        rc, out = _noalloc(q, k, v, seq, scale)
        assert rc == 0, nat.lib().tq_error_string(rc)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), (B, Hq, L)


def test_noalloc_attention_refuses_sizes_past_its_array():
    # 16 sequences x 64 query heads at 4096 keys need 8.5 Mi floats of split records (> 4 Mi)
    B, Hq, Hkv, L = 16, 64, 8, 4096
    assert nat.lib().tq_decode_attention_workspace_elems(B, Hq, L) > 4 << 20
    q, k, v, seq = _inputs(1, 8, 1, 64, [64], 3)   # valid pointers; the size check comes first
    out = torch.empty((1, 8, 128), dtype=torch.bfloat16, device=DEV)
    rc = nat.lib().tq_decode_attention_noalloc(
        nat.ptr(q), q.stride(0), q.stride(1), nat.ptr(k), nat.ptr(v), k.stride(0), k.stride(2), k.stride(1),
        nat.ptr(seq), nat.ptr(out), out.stride(0), out.stride(1), 0, B, Hq, Hkv, 128, L, 0.1, nat.stream_handle(DEV))
    assert rc == -4   # TQ_ERR_WORKSPACE, nothing launched
