"""One-token decode step of a Llama / Qwen2 model from fused kernels.

``FusedDecodeStep`` computes what the model's own forward computes for one
new token per sequence over a ``StaticCache`` -- embedding, 28-ish decoder
layers, final norm, LM head -- with per layer:

  add_rmsnorm_quant  residual add + input RMSNorm + INT8 codes of the result
  QKV GEMM           stacked Q/K/V MixedLinear on the codes (or F.linear)
  decode attention   split kernel that applies RoPE to q/k and writes the new
                     token's k/v into the cache, + merge that quantizes for O
  O GEMM
  add_rmsnorm_quant  residual add + post-attention RMSNorm + codes
  Gate/Up GEMM       stacked
  silu_mul_quant     SiLU(gate) * up + codes
  Down GEMM

i.e. 9 launches per layer where the modules issue ~40 (norm, RoPE, cache
update, residual and activation elementwise kernels, one quantization per
GEMM).  The arithmetic follows the modules op by op (see csrc/tq_fused.hip);
the GEMMs are exactly the MixedLinear kernels on exactly the activation
codes MixedLinear would compute.  Dense ``nn.Linear`` projections (the bf16
baseline) run through ``F.linear`` on stacked weights, with the same fused
glue, so both models are timed with the same non-GEMM work.

This is the decode-latency step of the ranked "fewer launches per layer" item
of the reference's hot path (activation quantization fused into its producer,
src/models/mixed_linear.py:233-239 -> quant_utils.py:119-134); the reference
runs the Hugging Face modules inside its captured decode graph
(src/runtime/graph_decode.py:350-385).
"""
from __future__ import annotations

import ctypes
from typing import List, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _native as nat
from .attention import decode_attention_workspace
from .gemm_rows_splitk_64x64 import gemm_mixed_rows_splitk
from .mixed_linear import MixedLinear


def _stacked(parent: nn.Module, group_attr: str, names) -> nn.Module:
    """The stacked projection of a group: a MixedLinear (grouped by
    fuse_projection_groups) or a dense nn.Linear built from the members."""
    group = getattr(parent, group_attr, None)
    if group is not None:
        return group.linear
    members = [getattr(parent, n) for n in names]
    if not all(isinstance(m, nn.Linear) for m in members):
        raise ValueError(f"cannot stack {names}: expected a projection group or nn.Linear members")
    w = torch.cat([m.weight.detach() for m in members], dim=0)
    lin = nn.Linear(w.shape[1], w.shape[0], bias=members[0].bias is not None, device=w.device, dtype=w.dtype)
    lin.weight = nn.Parameter(w, requires_grad=False)
    if lin.bias is not None:
        lin.bias = nn.Parameter(torch.cat([m.bias.detach() for m in members]), requires_grad=False)
    return lin


class _Layer:
    def __init__(self, layer: nn.Module) -> None:
        attn, mlp = layer.self_attn, layer.mlp
        self.qkv = _stacked(attn, "tilequant_qkv", ("q_proj", "k_proj", "v_proj"))
        self.o = attn.o_proj
        self.gate_up = _stacked(mlp, "tilequant_gate_up", ("gate_proj", "up_proj"))
        self.down = mlp.down_proj
        self.ln1, self.ln2 = layer.input_layernorm, layer.post_attention_layernorm
        act = getattr(getattr(mlp, "config", None), "hidden_act", "silu")
        if act not in ("silu", "swish"):
            raise ValueError(f"fused decode supports SiLU MLPs, got {act}")
        # L2 warm-up descriptors of the four GEMMs (set by FusedDecodeStep)
        self.warm = {"qkv": None, "o": None, "gate_up": None, "down": None}


# Warm-up sizing: about this many bytes of an XCD's share per warm-up workgroup,
# at most this many workgroups per XCD.
WARM_BYTES_PER_BLOCK = 64 * 1024
WARM_MAX_BLOCKS_PER_XCD = 128
# GEMMs whose weights are warmed.  Measured on MI355X (Llama-3.2-3B keep01, B=4,
# 2304-token cache; TPOT, ms): none 1.905, QKV 1.888, QKV+O+Down 1.893-1.912,
# Down 1.936, all four 2.12.  Only the QKV weights (16 MB) arrive within the
# norm kernel that precedes them; O (inside the short attention merge), Gate/Up
# (50 MB: more than the XCDs' L2) and Down (25 MB inside the SiLU kernel)
# stretch their producer by more than their GEMM gains.  Since the glue kernels
# load their arguments in one round trip (3.4 us norm instead of 4.6) the
# effect is within 0.2% either way: none 1.676, QKV 1.674, QKV+O+Down 1.673.
WARM_GEMMS = ("qkv",)


def l2_warm_descriptor(lin: nn.Module, n_rows: int) -> Optional[nat.L2Warm]:
    """The tq_l2_warm of a MixedLinear's decode GEMM at ``n_rows`` rows, or
    None: a dense projection, or a shape whose GEMM schedule does not read
    row tile r from XCD r mod 8 only (tq_gemm_l2_warm_ok).  The descriptor
    holds raw pointers into the module's buffers: rebuild it if they change."""
    if not isinstance(lin, MixedLinear):
        return None
    if not nat.lib().tq_gemm_l2_warm_ok(int(n_rows), lin.K_orig, lin.n_tr, lin.n_tc):
        return None
    t8, t16 = int(lin.int8_tiles.shape[0]), int(lin.fp16_tiles.shape[0])
    per_xcd_bytes = (4096 * t8 + 8192 * t16) / 8
    per = max(1, min(WARM_MAX_BLOCKS_PER_XCD, -(-int(per_xcd_bytes) // WARM_BYTES_PER_BLOCK)))
    return nat.L2Warm(nat.ptr(lin.int8_tiles), nat.ptr(lin.fp16_tiles) if t16 else None, nat.ptr(lin.int8_row_ptr),
                      nat.ptr(lin.fp16_row_ptr) if t16 else None, lin.n_tr, 8 * per)


# Architectures whose decoder layer is exactly what the fused step computes:
# pre-norm RMSNorm, full-width RoPE on q and k (no per-head q/k norm), grouped-
# query attention, SiLU-gated MLP.  Anything else replays the model's own
# forward (the decoder catches the ValueError).
FUSED_MODEL_TYPES = ("llama", "qwen2")
# RoPE variants whose factors depend on the position only, so one table of
# every cache position serves all steps ("dynamic" / "longrope" rescale with
# the sequence length).
FUSED_ROPE_TYPES = ("default", "llama3", "linear")


def check_fused_architecture(cfg, attention_module: nn.Module) -> None:
    """Raise ValueError unless the fused step computes this model exactly."""
    model_type = str(getattr(cfg, "model_type", ""))
    if model_type not in FUSED_MODEL_TYPES:
        raise ValueError(f"fused decode serves {FUSED_MODEL_TYPES}, got model_type={model_type!r}")
    for name in ("q_norm", "k_norm"):
        if getattr(attention_module, name, None) is not None:
            raise ValueError(f"fused decode has no per-head {name}")
    rope = getattr(cfg, "rope_scaling", None) or getattr(cfg, "rope_parameters", None) or {}
    rope_type = str(rope.get("rope_type", rope.get("type", "default"))) if isinstance(rope, dict) else "default"
    if rope_type not in FUSED_ROPE_TYPES:
        raise ValueError(f"fused decode needs position-only RoPE factors, got rope_type={rope_type!r}")
    partial = getattr(cfg, "partial_rotary_factor", 1.0)
    if partial is not None and float(partial) != 1.0:
        raise ValueError("fused decode rotates the whole head (partial_rotary_factor must be 1)")


class FusedDecodeStep:
    """Decode forward for a bound model and static cache (batch fixed)."""

    def __init__(self, model: nn.Module, cache, batch: int, max_cache_len: int, device: torch.device,
                 l2_warm: bool = True) -> None:
        cfg = model.config.get_text_config(decoder=True)
        check_fused_architecture(cfg, model.model.layers[0].self_attn)
        self.model = model
        self.text = model.model
        self.cache = cache
        self.B = int(batch)
        self.L = int(max_cache_len)
        self.device = device
        self.hidden = int(cfg.hidden_size)
        self.hq, self.hkv = int(cfg.num_attention_heads), int(cfg.num_key_value_heads)
        self.head_dim = int(getattr(cfg, "head_dim", None) or self.hidden // self.hq)
        if self.head_dim != 128:
            raise ValueError("fused decode serves head_dim 128")
        if self.B > 16:
            raise ValueError("fused decode serves at most 16 sequences")
        self.inter = int(cfg.intermediate_size)
        self.layers: List[_Layer] = [_Layer(l) for l in self.text.layers]
        # Each GEMM's packed weights are read, by the producer kernel that runs
        # just before it (norm, attention merge, SiLU * up), into the L2 of the
        # XCD that will read them (tq_l2_warm): that producer leaves the
        # memory system idle, and the GEMM then starts on warm lines.
        self.set_l2_warm(l2_warm)
        self.dtype = self.text.embed_tokens.weight.dtype
        self.code = nat.dtype_code(self.dtype)
        self.scale = float(self.text.layers[0].self_attn.scaling)
        B, H, dt, dev = self.B, self.hidden, self.dtype, device
        qkv_w = (self.hq + 2 * self.hkv) * self.head_dim
        e = lambda *s, d=dt: torch.empty(s, device=dev, dtype=d)   # noqa: E731
        # static activations (graph-stable addresses)
        self.h = [e(B, H), e(B, H)]            # residual stream, ping-pong
        self.y = e(B, H)
        self.yq, self.ysx = e(B, H, d=torch.int8), e(H // 64, d=torch.float32)
        self.qkv_out = e(B, qkv_w)
        self.attn = e(B, self.hq * self.head_dim)
        self.aq = e(B, self.hq * self.head_dim, d=torch.int8)
        self.asx = e(self.hq * self.head_dim // 64, d=torch.float32)
        self.o_out = e(B, H)
        self.gu = e(B, 2 * self.inter)
        self.m = e(B, self.inter)
        self.mq, self.msx = e(B, self.inter, d=torch.int8), e(self.inter // 64, d=torch.float32)
        self.d_out = e(B, H)
        self.final = e(B, H)
        self.attn_ws = decode_attention_workspace(B, self.hq, self.L, dev)
        # RoPE factors of every cache position, from the model's own rotary
        # module (per position the same fp32 product inv_freq * p, cos/sin and
        # rounding as a one-position call, so the rows equal the per-step
        # values); the attention kernel reads the row at the device position
        with torch.inference_mode():
            pos = torch.arange(self.L, device=dev).view(1, -1)
            cos, sin = self.text.rotary_emb(torch.empty((1, 1, 1), device=dev, dtype=dt), pos)
        self.cos_table = cos.reshape(self.L, self.head_dim).contiguous()
        self.sin_table = sin.reshape(self.L, self.head_dim).contiguous()

    def set_l2_warm(self, enabled: bool) -> None:
        """Switch the L2 warm-up of the GEMM weights on or off (outputs are the
        same either way); takes effect for steps issued or captured later."""
        self.l2_warm = bool(enabled)
        for ly in self.layers:
            for name in ly.warm:
                on = self.l2_warm and name in WARM_GEMMS
                ly.warm[name] = l2_warm_descriptor(getattr(ly, name), self.B) if on else None

    # -- kernels -------------------------------------------------------------
    @staticmethod
    def _warm_arg(warm: Optional[nat.L2Warm]):
        return ctypes.byref(warm) if warm is not None else None

    def _norm(self, x, delta, ln, h_out, y_out, q_out, sx_out, warm=None) -> None:
        rc = nat.lib().tq_add_rmsnorm_quant(
            nat.ptr(x), x.stride(0), nat.ptr(delta), delta.stride(0) if delta is not None else 0,
            nat.ptr(ln.weight), float(ln.variance_epsilon), nat.ptr(h_out), h_out.stride(0) if h_out is not None else 0,
            nat.ptr(y_out), y_out.stride(0), nat.ptr(q_out), q_out.stride(0) if q_out is not None else 0,
            nat.ptr(sx_out), self.code, self.B, self.hidden, self._warm_arg(warm), nat.stream_handle(self.device))
        nat.check(rc, "tq_add_rmsnorm_quant")

    def _linear(self, lin: nn.Module, x, xq, sx, out) -> None:
        if isinstance(lin, MixedLinear):
            gemm_mixed_rows_splitk(x_fp=x, x_int8=xq, sx=sx, int8_tiles=lin.int8_tiles, int8_scales=lin.int8_scales,
                                   int8_tile_ids=lin.int8_tile_ids, int8_row_ptr=lin.int8_row_ptr,
                                   fp16_tiles=lin.fp16_tiles, fp16_tile_ids=lin.fp16_tile_ids,
                                   fp16_row_ptr=lin.fp16_row_ptr, M=lin.M_orig, K=lin.K_orig, n_tr=lin.n_tr,
                                   n_tc=lin.n_tc, out_dtype=out.dtype, bias=lin._out_bias(out.dtype), out=out,
                                   tile_layout=lin.tile_layout)
        else:
            torch.matmul(x, lin.weight.t(), out=out)
            if lin.bias is not None:
                out.add_(lin.bias)

    @staticmethod
    def _quantized(lin: nn.Module) -> bool:
        return isinstance(lin, MixedLinear)

    # -- step -----------------------------------------------------------------
    @torch.inference_mode()
    def __call__(self, token: torch.Tensor, position: torch.Tensor, seq_used: torch.Tensor) -> torch.Tensor:
        """token [B, 1] int64, position [1] int64 (cache index of the token),
        seq_used [B] int32 (= position + 1).  Returns logits [B, 1, V]."""
        B, dev = self.B, self.device
        stream = nat.stream_handle(dev)
        x = self.text.embed_tokens(token).view(B, self.hidden)
        cur, delta = x, None
        k = 0
        for li, ly in enumerate(self.layers):
            h_new = self.h[k]
            q8 = self._quantized(ly.qkv)
            self._norm(cur, delta, ly.ln1, h_new if delta is not None else None, self.y,
                       self.yq if q8 else None, self.ysx if q8 else None, ly.warm["qkv"])
            resid = h_new if delta is not None else cur
            self._linear(ly.qkv, self.y, self.yq, self.ysx, self.qkv_out)
            layer_cache = self.cache.layers[li]
            kc, vc = layer_cache.keys, layer_cache.values
            # RoPE, the cache write of the new token and attention (+ the O
            # projection's quantization) in one split pass and one merge
            q8o = self._quantized(ly.o)
            rc = nat.lib().tq_decode_attention_rope(
                nat.ptr(self.qkv_out), self.qkv_out.stride(0), nat.ptr(self.cos_table), nat.ptr(self.sin_table),
                nat.ptr(position),
                nat.ptr(kc), nat.ptr(vc), kc.stride(0), kc.stride(2), kc.stride(1), nat.ptr(seq_used),
                nat.ptr(self.attn), self.attn.stride(0), self.head_dim,
                nat.ptr(self.aq) if q8o else None, self.aq.stride(0), nat.ptr(self.asx) if q8o else None,
                self.code, B, self.hq, self.hkv, self.head_dim, self.L, self.scale, nat.ptr(self.attn_ws),
                self.attn_ws.numel(), self._warm_arg(ly.warm["o"]), stream)
            nat.check(rc, "tq_decode_attention_rope")
            self._linear(ly.o, self.attn, self.aq, self.asx, self.o_out)
            k ^= 1
            h2 = self.h[k]
            q8g = self._quantized(ly.gate_up)
            self._norm(resid, self.o_out, ly.ln2, h2, self.y, self.yq if q8g else None, self.ysx if q8g else None,
                       ly.warm["gate_up"])
            self._linear(ly.gate_up, self.y, self.yq, self.ysx, self.gu)
            q8d = self._quantized(ly.down)
            rc = nat.lib().tq_silu_mul_quant(nat.ptr(self.gu), self.gu.stride(0), nat.ptr(self.m), self.m.stride(0),
                                             nat.ptr(self.mq) if q8d else None, self.mq.stride(0),
                                             nat.ptr(self.msx) if q8d else None, self.code, B, self.inter,
                                             self._warm_arg(ly.warm["down"]), stream)
            nat.check(rc, "tq_silu_mul_quant")
            self._linear(ly.down, self.m, self.mq, self.msx, self.d_out)
            cur, delta = h2, self.d_out
            k ^= 1
        norm = self.text.norm
        self._norm(cur, delta, norm, self.h[k], self.final, None, None)
        logits = self.model.lm_head(self.final.view(B, 1, self.hidden))
        return logits


class FusedPrefillStep:
    """Prompt forward (``batch`` sequences of ``prompt_len`` tokens, positions
    0 .. prompt_len - 1) for a bound model and static cache: what the model's
    own forward computes at prefill, with the row-parallel forms of the glue
    kernels -- ``tq_add_rmsnorm_rows`` for the residual adds and both
    RMSNorms, ``tq_rope_prefill`` for RoPE and the cache writes,
    ``tq_silu_mul_rows`` for SiLU(gate) * up -- around the model's own
    projections (MixedLinear or stacked dense) and the decoder's causal SDPA.
    The modules spend ~7 elementwise launches per RMSNorm and several more per
    RoPE, SiLU and cache update over the 8192 x 3072 activations.  Returns the
    logits of each sequence's last token [B, 1, V] (the ``logits_to_keep=1``
    forward).  Element arithmetic follows the modules op by op; the fp32 sum
    of squares of each RMSNorm is the only reordered reduction."""

    def __init__(self, model: nn.Module, cache, batch: int, prompt_len: int, max_cache_len: int,
                 device: torch.device, attention, layers: Optional[List["_Layer"]] = None,
                 cos_table: Optional[torch.Tensor] = None, sin_table: Optional[torch.Tensor] = None) -> None:
        cfg = model.config.get_text_config(decoder=True)
        check_fused_architecture(cfg, model.model.layers[0].self_attn)
        self.model, self.text, self.cache = model, model.model, cache
        self.B, self.P, self.L = int(batch), int(prompt_len), int(max_cache_len)
        if self.P > self.L:
            raise ValueError("prompt longer than the cache")
        self.device = device
        self.attention = attention
        self.hidden = int(cfg.hidden_size)
        self.hq, self.hkv = int(cfg.num_attention_heads), int(cfg.num_key_value_heads)
        self.head_dim = int(getattr(cfg, "head_dim", None) or self.hidden // self.hq)
        if self.head_dim != 128:
            raise ValueError("fused prefill serves head_dim 128")
        if self.hidden % 8 or self.hidden > 8192:
            raise ValueError("fused prefill serves hidden sizes <= 8192, multiples of 8")
        self.inter = int(cfg.intermediate_size)
        self.layers: List[_Layer] = layers if layers is not None else [_Layer(l) for l in self.text.layers]
        self.dtype = self.text.embed_tokens.weight.dtype
        self.code = nat.dtype_code(self.dtype)
        self.scale = float(self.text.layers[0].self_attn.scaling)
        N, H, dt, dev = self.B * self.P, self.hidden, self.dtype, device
        e = lambda *s: torch.empty(s, device=dev, dtype=dt)   # noqa: E731
        self.h = [e(N, H), e(N, H)]                          # residual stream, ping-pong
        self.y = e(N, H)                                     # normed activations
        # rotated queries, token-major [B, P, Hq, D], handed to SDPA as the [B, Hq, P, D] view: the fused
        # backends then return token-major output, which the O projection reads without a transpose copy
        self.q = e(self.B, self.P, self.hq, self.head_dim).transpose(1, 2)
        self.m = e(N, self.inter)                            # silu(gate) * up
        self.h_last = e(self.B, H)
        self.final = e(self.B, H)
        if cos_table is None or sin_table is None:
            with torch.inference_mode():
                pos = torch.arange(self.P, device=dev).view(1, -1)
                cos, sin = self.text.rotary_emb(torch.empty((1, 1, 1), device=dev, dtype=dt), pos)
            cos_table = cos.reshape(self.P, self.head_dim).contiguous()
            sin_table = sin.reshape(self.P, self.head_dim).contiguous()
        self.cos_table, self.sin_table = cos_table, sin_table

    def _norm(self, x, delta, ln, h_out, y_out, n) -> None:
        rc = nat.lib().tq_add_rmsnorm_rows(
            nat.ptr(x), x.stride(0), nat.ptr(delta), delta.stride(0) if delta is not None else 0,
            nat.ptr(ln.weight), float(ln.variance_epsilon), nat.ptr(h_out), h_out.stride(0) if h_out is not None else 0,
            nat.ptr(y_out), y_out.stride(0), self.code, n, self.hidden, nat.stream_handle(self.device))
        nat.check(rc, "tq_add_rmsnorm_rows")

    @staticmethod
    def _project(lin: nn.Module, x: torch.Tensor) -> torch.Tensor:
        return lin(x)

    @torch.inference_mode()
    def __call__(self, prompt: torch.Tensor) -> torch.Tensor:
        """prompt [B, P] int64 -> logits [B, 1, V]; the cache holds the prompt's k/v afterwards."""
        B, P, N, H = self.B, self.P, self.B * self.P, self.hidden
        stream = nat.stream_handle(self.device)
        layers = self.cache.layers
        if not layers[0].is_initialized:
            self.cache.early_initialization(B, self.hkv, self.head_dim, self.dtype, self.device)
        x = self.text.embed_tokens(prompt).view(N, H)
        cur, delta = x, None
        k = 0
        for li, ly in enumerate(self.layers):
            h_new = self.h[k]
            self._norm(cur, delta, ly.ln1, h_new if delta is not None else None, self.y, N)
            resid = h_new if delta is not None else cur
            qkv = self._project(ly.qkv, self.y)
            kc, vc = layers[li].keys, layers[li].values
            rc = nat.lib().tq_rope_prefill(
                nat.ptr(qkv), qkv.stride(0), nat.ptr(self.cos_table), nat.ptr(self.sin_table),
                self.cos_table.stride(0), nat.ptr(self.q), self.q.stride(0), self.q.stride(1), self.q.stride(2),
                nat.ptr(kc), nat.ptr(vc), kc.stride(0), kc.stride(1), kc.stride(2), self.code, B, P, self.hq,
                self.hkv, self.head_dim, kc.shape[2], stream)
            nat.check(rc, "tq_rope_prefill")
            layers[li].cumulative_length.add_(P)   # the cache's own bookkeeping, as its update() keeps it
            attn = self.attention(self.q, kc[:, :, :P], vc[:, :, :P], self.scale)   # [B, P, Hq, D]
            o = self._project(ly.o, attn.reshape(N, self.hq * self.head_dim))
            k ^= 1
            h2 = self.h[k]
            self._norm(resid, o, ly.ln2, h2, self.y, N)
            gu = self._project(ly.gate_up, self.y)
            rc = nat.lib().tq_silu_mul_rows(nat.ptr(gu), gu.stride(0), nat.ptr(self.m), self.m.stride(0), self.code,
                                            N, self.inter, stream)
            nat.check(rc, "tq_silu_mul_rows")
            d = self._project(ly.down, self.m)
            cur, delta = h2, d
            k ^= 1
        # final norm on each sequence's last token only (the norm is per row)
        last = lambda t: t.view(B, P, H)[:, P - 1]   # noqa: E731  [B, H], row stride P * H
        self._norm(last(cur), last(delta), self.text.norm, self.h_last, self.final, B)
        return self.model.lm_head(self.final.view(B, 1, H))
