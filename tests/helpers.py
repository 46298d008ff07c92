"""Shared seeded inputs and checks for the test suite (synthetic data only)."""
from __future__ import annotations

import numpy as np
import torch

from oracle import numerics as nm
from oracle import packing as opk

TILE = 64


def gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(int(seed))
    return g


def make_x(n: int, k: int, seed: int = 0, dtype=torch.bfloat16, outlier_frac=0.005, outlier_scale=20.0):
    """N(0,1) activations with round(frac*k) outlier input channels x scale."""
    g = gen(seed)
    x = torch.randn((n, k), generator=g, dtype=torch.float32)
    n_out = int(round(outlier_frac * k))
    if n_out:
        ch = torch.randperm(k, generator=g)[:n_out]
        x[:, ch] *= outlier_scale
    return x.to(dtype)


def make_w(m: int, k: int, seed: int = 1, dtype=torch.bfloat16, std=0.02):
    g = gen(seed)
    return (torch.randn((m, k), generator=g, dtype=torch.float32) * std).to(dtype)


def uniform_fp16_ids(n_tr: int, n_tc: int, frac: float, seed: int = 2) -> np.ndarray:
    """k = max(1, ceil(frac * n_tiles)) tile ids uniformly without replacement, ascending."""
    import math

    n = n_tr * n_tc
    k = max(1, int(math.ceil(frac * n))) if frac > 0 else 0
    rng = np.random.default_rng(seed)
    return np.sort(rng.choice(n, size=min(k, n), replace=False)).astype(np.int64)


def complement(ids: np.ndarray, n: int) -> np.ndarray:
    return opk.int8_ids_complement(ids, n).astype(np.int64)


def bits(t: torch.Tensor) -> np.ndarray:
    """uint16 bit patterns of a bf16/fp16 CPU tensor."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def values(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().to(torch.float32).numpy()


def oracle_pack(W: torch.Tensor, fp16_ids: np.ndarray) -> opk.OraclePack:
    return opk.pack_weight(bits(W), fp16_ids)


def assert_gemm_close(y: torch.Tensor, acc64: np.ndarray, sumabs: np.ndarray, n_tc: int, bias=None):
    """|y - exact| <= 2 bf16 ulp + fp32 accumulation bound (oracle.numerics.gemm_tolerance)."""
    yv = values(y).astype(np.float64)
    ref = acc64 if bias is None else acc64 + np.asarray(bias, np.float64)[None, :]
    tol = nm.gemm_tolerance(acc64, sumabs, n_tc, bias)
    err = np.abs(yv - ref)
    bad = err > tol
    assert not bad.any(), (
        f"{int(bad.sum())} of {bad.size} outputs outside tolerance; worst err {err.max():.3e} "
        f"(tol there {tol.reshape(-1)[np.argmax(err)]:.3e})"
    )
    return float((err / nm.bf16_ulp(ref)).max())


def clustered_weight(m: int, k: int, frac: float, seed: int):
    """BASELINE configs[3] weights and masks: N(0, 0.02) with 3% of the
    64-column input blocks x4 and 3% of the 64-row output blocks x3, BF16
    tiles chosen by the reference's top-k rule on per-tile sum|W|
    (k = max(1, ceil(frac * tiles)), src/quantization/decisions.py:174-183),
    so the BF16 tiles cluster in those bands and row tiles get very uneven
    BF16/INT8 mixes.  Returns (W bf16 [m, k], sorted BF16 tile ids)."""
    from oracle import masks as om

    g = gen(seed)
    n_tr, n_tc = -(-m // 64), -(-k // 64)
    W = torch.randn((m, k), generator=g, dtype=torch.float32) * 0.02
    cb = torch.randperm(n_tc, generator=g)[: max(1, round(0.03 * n_tc))]
    rb = torch.randperm(n_tr, generator=g)[: max(1, round(0.03 * n_tr))]
    W4 = W.view(n_tr, 64, n_tc, 64)
    W4[:, :, cb, :] *= 4
    W4[rb] *= 3
    W = W.to(torch.bfloat16)
    scores = W.float().abs().view(n_tr, 64, n_tc, 64).sum(dim=(1, 3)).numpy()
    return W, om.topk_ids(scores, frac)
