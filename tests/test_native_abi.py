"""The C-ABI library loads and exports every symbol include/tilequant.h declares.

No compute: only pure host entry points are called (argument validation,
workspace sizing, error strings), so this runs without a GPU.
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from tilequant_amd import _native as nat

HEADER = Path(__file__).resolve().parents[1] / "include" / "tilequant.h"


def header_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(tq_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return nat.load()


def test_header_declares_what_the_binding_knows():
    assert header_functions() == sorted(nat.EXPORTED_SYMBOLS)


def test_every_declared_symbol_is_exported(lib):
    for name in header_functions():
        assert hasattr(lib, name), name
        assert ctypes.cast(getattr(lib, name), ctypes.c_void_p).value


def test_abi_version_and_error_strings(lib):
    assert lib.tq_abi_version() == nat.ABI_VERSION
    assert lib.tq_error_string(0) == b"ok"
    for code in (-1, -2, -3, -4):
        assert b"unknown" not in lib.tq_error_string(code)


def test_argument_errors_return_before_any_launch(lib):
    # negative sizes / bad dtype codes are rejected on the host
    assert lib.tq_act_quant_fused(None, 0, 1, 0, -1, 64, None, 64, None, None) == -1
    assert lib.tq_act_quant_fused(None, 64, 1, 7, 1, 64, None, 64, None, None) == -2
    assert lib.tq_gemm_mixed_rows(None, 0, None, None, None, None, None, None, 0, 0, None, None, None,
                                  None, 0, 0, None, -1, 64, 64, 1, 1, 0, 1, None, 0, None) == -1
    assert lib.tq_gemm_mixed_rows(None, 0, None, None, None, None, None, None, 0, 0, None, None, None,
                                  None, 0, 0, None, 1, 64, 64, 1, 1, 0, 5, None, 0, None) == -2
    assert lib.tq_tiles_relayout(None, None, 1, 3, 0, 1, None) == -1
    # token-blocked codes: 1..64 rows, k a multiple of 64 (no device memory touched)
    assert lib.tq_act_quant_token_blocked(None, 64, 0, 0, 64, None, None, None) == -1
    assert lib.tq_act_quant_token_blocked(None, 64, 0, 65, 64, None, None, None) == -1
    assert lib.tq_act_quant_token_blocked(None, 100, 0, 4, 100, None, None, None) == -1
    assert lib.tq_act_quant_token_blocked(None, 64, 3, 4, 64, None, None, None) == -2
    blocked = nat.TQ_LAYOUT["mfma"] | nat.TQ_XQ_TOKEN_BLOCKED
    assert lib.tq_gemm_mixed_rows(None, 0, None, None, None, None, None, None, 0, 0, None, None, None,
                                  None, 0, 0, None, 65, 64, 64, 1, 1, 0, blocked, None, 0, None) == -1
    assert lib.tq_gemm_mixed_rows(None, 0, None, None, None, None, None, None, 0, 0, None, None, None,
                                  None, 0, 0, None, 4, 64, 100, 1, 2, 0, blocked, None, 0, None) == -1
    assert lib.tq_gemm_mixed_rows(None, 0, None, None, None, None, None, None, 0, 0, None, None, None,
                                  None, 0, 0, None, 0, 64, 64, 1, 1, 0, blocked, None, 0, None) == 0
    # empty problems are a no-op success
    assert lib.tq_gemm_mixed_rows(None, 0, None, None, None, None, None, None, 0, 0, None, None, None,
                                  None, 0, 0, None, 0, 64, 64, 1, 1, 0, 1, None, 0, None) == 0
    assert lib.tq_pack_int8_tiles(None, 64, 0, 64, 64, None, 0, 1, 1, None, None, None, None) == 0
    # the read-probe measurement helper: sizes in whole 16-byte words, aligned data, a sink
    assert lib.tq_read_probe(None, 0, None, None) == 0
    assert lib.tq_read_probe(None, 17, None, None) == -1 and lib.tq_read_probe(None, -16, None, None) == -1
    assert lib.tq_read_probe(None, 16, None, None) == -1
    assert lib.tq_read_probe(ctypes.c_void_p(8), 16, ctypes.c_void_p(256), None) == -3


def test_token_blocked_preference(lib):
    """Token-blocked codes for 17..64 rows; below that only where the codes do
    not fit the LDS-staged decode kernel (144 KiB: k = 8192 fits up to 16
    rows, k = 13824 up to 9) or rows hold 256+ column tiles (k >= 16384)."""
    pref = lib.tq_gemm_prefers_token_blocked
    assert pref(64, 3072, 80, 48) == 1 and pref(33, 3072, 48, 48) == 1 and pref(17, 3072, 256, 48) == 1
    assert pref(32, 8192, 48, 128) == 1
    assert pref(16, 3072, 80, 48) == 0 and pref(4, 3072, 256, 48) == 0 and pref(4, 8192, 48, 128) == 0
    assert pref(16, 8192, 48, 128) == 0 and pref(12, 8192, 48, 128) == 0
    assert pref(9, 13824, 80, 216) == 0 and pref(10, 13824, 80, 216) == 1
    assert pref(1, 18944, 56, 296) == 1 and pref(4, 18944, 56, 296) == 1 and pref(4, 16384, 48, 256) == 1
    assert pref(4, 16320, 48, 255) == 0
    assert pref(65, 3072, 48, 48) == 0 and pref(0, 3072, 48, 48) == 0 and pref(16, 3000, 48, 47) == 0


def test_workspace_sizing(lib):
    assert lib.tq_act_absmax_workspace_elems(128, 3072) == 0
    assert lib.tq_act_absmax_workspace_elems(8192, 3072) == 32 * 48
    # automatic decode plan: no cross-workgroup split, no workspace
    assert lib.tq_gemm_workspace_elems(16, 3072, 48, 48, 0) == 0
    assert lib.tq_gemm_workspace_elems(4, 16384, 256, 48, 0) == 0
    # explicit split_k = 8: a fixed 4096-entry counter region, then partials per
    # (unit, split, row, 64 cols); units = 4 j-block groups per row tile below
    # 192 row tiles, whole row tiles from there on
    assert lib.tq_gemm_workspace_elems(16, 3072, 48, 48, 8) == 4096 + 48 * 4 * 8 * 16 * 64
    # up to 8 tokens every row tile has four one-j-block workgroups (units)
    assert lib.tq_gemm_workspace_elems(4, 16384, 256, 48, 8) == 4096 + 256 * 4 * 8 * 4 * 64
    # whole-tile workgroups (one unit per row tile) from 9 tokens on 192+ row tiles
    assert lib.tq_gemm_workspace_elems(16, 16384, 256, 48, 8) == 4096 + 256 * 8 * 16 * 64
    assert lib.tq_gemm_workspace_elems(4, 1 << 20, 1 << 14, 48, 8) == 0   # beyond the counter cap
    assert lib.tq_gemm_workspace_elems(100, 3072, 48, 48, 0) == 0     # general kernel: none


def test_fused_workspace_sizing(lib):
    """linear_mixed_fused's workspace: the split-K one, or for a cooperative
    launch (a shape the LDS-staged quantizing kernel cannot take: too many
    rows x columns for its chunks per thread) a 4096-entry head of flags and
    counts, the int8 codes [n][k] rounded up to 16 bytes, then n_tc scales."""
    def coop(n, k, n_tc):
        return 4096 + (n * k + 15) // 16 * 4 + n_tc
    q = lib.tq_linear_mixed_fused_workspace_elems
    # Llama-3.2-3B Q/K/V (5120 x 3072): the quantizing kernel up to 4 rows
    # (no workspace), cooperative at 8 and 16
    for n in (1, 2, 4):
        assert q(n, 5120, 3072, 80, 48, 0) == 0
    assert q(8, 5120, 3072, 80, 48, 0) == coop(8, 3072, 48) == 4096 + 6144 + 48
    assert q(16, 3072, 3072, 48, 48, 0) == coop(16, 3072, 48)
    # Gate/Up (16384 x 3072): 12-tile batches leave no room at 4 rows
    assert q(4, 16384, 3072, 256, 48, 0) == coop(4, 3072, 48)
    assert q(2, 16384, 3072, 256, 48, 0) == 0
    # Qwen2.5-14B Q/K/V at 16 rows: beyond the fused path's 64 KiB of codes
    assert q(16, 7168, 5120, 112, 80, 0) == 0
    # an explicit split is the split-K kernel's workspace only
    assert q(8, 5120, 3072, 80, 48, 2) == lib.tq_gemm_workspace_elems(8, 5120, 80, 48, 2) > 0
    assert q(0, 5120, 3072, 80, 48, 0) == 0
    assert q(100, 5120, 3072, 80, 48, 0) == 0


def _attention_plan(lib, batch, q_heads, kv_heads, max_len, rope, cus):
    s, w = ctypes.c_int(0), ctypes.c_int(0)
    rc = lib.tq_decode_attention_plan(batch, q_heads, kv_heads, max_len, int(rope), cus, ctypes.byref(s),
                                      ctypes.byref(w))
    assert rc == 0
    return s.value, w.value


@pytest.mark.parametrize("batch,q_heads,kv_heads,max_len,rope", [
    (4, 24, 8, 2304, True), (4, 24, 8, 2304, False), (1, 24, 8, 2304, True), (4, 28, 4, 2304, True),
    (4, 40, 8, 2304, True), (2, 7, 1, 300, True), (1, 8, 1, 64, False), (3, 40, 8, 513, True),
    (2, 8, 2, 8400, False), (16, 24, 8, 9000, False), (1, 8, 2, 131072, False), (5, 8, 8, 1, True)])
def test_decode_attention_plan_invariants(lib, batch, q_heads, kv_heads, max_len, rope):
    """The split plan (host logic of tq_decode_attention*): every split fits its
    workgroup (<= 32 keys per wave), the RoPE prologue has its 16 (G + 2)
    threads, the workspace covers the plan, and no other (waves, splits) choice
    gives the most loaded CU fewer keys."""
    cus = 256
    S, W = _attention_plan(lib, batch, q_heads, kv_heads, max_len, rope, cus)
    G = q_heads // kv_heads
    assert 2 <= W <= 4 and S >= 1
    assert -(-max_len // S) <= 32 * W
    if rope:
        assert 16 * (G + 2) <= 64 * W
    assert lib.tq_decode_attention_workspace_elems(batch, q_heads, max_len) >= batch * q_heads * S * 130
    cap = max(-(-max_len // 128), min(64, -(-max_len // 32)))
    assert S <= cap
    load = lambda s: -(-(batch * kv_heads * s) // cus) * -(-max_len // s)
    best = min(load(s) for w in (2, 3, 4) if not (rope and 16 * (G + 2) > 64 * w)
               for s in range(-(-max_len // (32 * w)), cap + 1))
    assert load(S) == best


def test_decode_attention_plan_balances_the_llama_decode_shape(lib):
    # B = 4 x 8 kv heads at 2304 keys: 24 splits of 3 waves = 768 workgroups, 3 per CU
    assert _attention_plan(lib, 4, 24, 8, 2304, True, 256) == (24, 3)
    assert lib.tq_decode_attention_plan(0, 24, 8, 2304, 1, 256, None, None) != 0


def test_l2_warm_descriptor_validation_and_shape_query(lib):
    """A tq_l2_warm the producers cannot use is rejected on the host, before
    any launch; tq_gemm_l2_warm_ok follows the decode schedule's XCD mapping."""
    fake = 1 << 20   # non-null, 16-byte aligned host values: nothing is dereferenced before the check
    good = dict(int8_tiles=fake, fp16_tiles=None, int8_row_ptr=fake, fp16_row_ptr=None, n_tr=80, blocks=64)
    bad = [dict(good, blocks=7), dict(good, blocks=-8), dict(good, blocks=2048), dict(good, n_tr=0),
           dict(good, int8_row_ptr=None), dict(good, fp16_tiles=fake, fp16_row_ptr=None)]
    for fields in bad:
        w = nat.L2Warm(**fields)
        assert lib.tq_add_rmsnorm_quant(fake, 3072, None, 0, fake, 1e-5, None, 0, fake, 3072, fake, 3072, fake, 0, 4,
                                        3072, ctypes.byref(w), None) == -1, fields
        assert lib.tq_silu_mul_quant(fake, 16384, fake, 8192, fake, 8192, fake, 0, 4, 8192, ctypes.byref(w),
                                     None) == -1, fields
    # one-j-block decode grids map row tile r to XCD r % 8 only when n_tr % 8 == 0
    assert lib.tq_gemm_l2_warm_ok(4, 3072, 80, 48) == 1       # Llama-3.2-3B stacked QKV at 4 tokens
    assert lib.tq_gemm_l2_warm_ok(4, 8192, 48, 128) == 1      # Down
    assert lib.tq_gemm_l2_warm_ok(4, 3072, 50, 48) == 0
    assert lib.tq_gemm_l2_warm_ok(12, 3072, 201, 48) == 1     # whole-tile workgroups: unit = row tile
    assert lib.tq_gemm_l2_warm_ok(128, 3072, 80, 48) == 0     # prefill sizes: another kernel
    assert lib.tq_gemm_l2_warm_ok(4, 3000, 80, 48) == 0       # k != 64 n_tc
