"""Fixed-shape HIP-graph greedy decoding (mirror of src/runtime/graph_decode.py).

``CudaGraphGreedyDecoder`` keeps the reference's interface -- ``prepare``,
``prefill``, ``decode``, ``generate``, ``generate_timed``, ``close`` and the
``GreedyGenerationTiming`` record (graph_decode.py:76-479) -- for a Hugging
Face decoder-only model whose linears may be ``MixedLinear``.  One prefill body
(cache reset included) and one one-token decode body are captured as HIP
graphs through ``torch.cuda.CUDAGraph``; every replay launches exactly the
captured kernels, so the arithmetic equals the eager forward.

ROCm specifics (this build's own design):

* Decode attention is ``tilequant_amd.attention.decode_attention`` -- a HIP
  split-sequence kernel that reads the cache only up to a device-resident
  length -- where the reference calls FlashAttention with ``seqused_k``.  It
  reads the cache in the static cache's own head-major storage, so no
  token-major re-layout is needed.
* Prefill attention is SDPA restricted to the fused flash / memory-efficient
  backends (causal, grouped-query); the unfused math backend is never used.
* The one-token step runs ``FusedDecodeStep`` (9 launches per decoder layer:
  residual + RMSNorm + INT8 quantization, attention with RoPE and the cache
  write in its split kernel and a merge that quantizes for O, SiLU * up +
  quantization, four GEMMs) for Llama /
  Qwen2 layouts with head_dim 128 and up to 16 sequences; ``fused_decode=False``
  (or any other architecture) replays the model's own forward as the reference
  does.
* The prompt forward of the same architectures runs ``FusedPrefillStep``: the
  model's projections and this module's SDPA, with the residual adds,
  RMSNorms, RoPE + cache writes and SiLU * up in row-parallel HIP kernels
  instead of the modules' elementwise chains; ``fused_prefill=False`` runs the
  model's forward.
* Argmax, token feedback and the position counter stay on the device, as in
  the reference (graph_decode.py:347-385): no scalar leaves the GPU between
  replays.
"""
from __future__ import annotations

import time
from dataclasses import dataclass
from typing import Optional, Sequence

import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel
from transformers import AttentionInterface, StaticCache
from transformers.masking_utils import AttentionMaskInterface

from . import _native as nat
from .attention import decode_attention, decode_attention_workspace

_GRAPH_ATTENTION = "tilequant_hip_graph"
# Prefills above this many tokens run eagerly into the static cache
# (graph_decode.py:21-24): their GPU time dwarfs launch cost, and a captured
# prefill would pin all of its activations in the graph pool.
MAX_CAPTURED_PREFILL_TOKENS = 16384
_DECODER_ATTRIBUTE = "_tilequant_graph_decoder"
_FUSED_SDPA = (SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION)


def _graph_attention(module, query, key, value, attention_mask, dropout: float = 0.0,
                     scaling: Optional[float] = None, **_):
    """Attention for a bound decoder: causal SDPA over the prompt prefix of
    the static cache at prefill, the HIP decode kernel over the valid prefix
    at decode.  Returns [B, T, Hq, D] like the library backends."""
    dec = getattr(module, _DECODER_ATTRIBUTE)
    scale = float(scaling) if scaling is not None else query.shape[-1] ** -0.5
    if dec._attention_is_prefill:
        P = dec.prompt_tokens
        if query.shape[2] != P:
            raise RuntimeError("captured prefill query length changed")
        return _prefill_attention(dec, query, key[:, :, :P], value[:, :, :P], dropout, scale), None
    if query.shape[2] != 1:
        raise RuntimeError("captured decode requires one query token")
    B, Hq, _, D = query.shape
    out = torch.empty((B, 1, Hq, D), device=query.device, dtype=query.dtype)
    decode_attention(query[:, :, 0, :], key, value, dec._decode_seq_used, scale=scale, out=out[:, 0],
                     workspace=dec._attention_workspace)
    return out, None


def _prefill_attention(dec, query, key, value, dropout: float, scale: float) -> torch.Tensor:
    """Causal SDPA on the fused backends.  Grouped-query heads go in directly
    where the backend takes them; otherwise (found once, in the eager warm-up
    before capture) the kv heads are repeated to the query heads first.  The
    backends return their output in the query's memory layout, so a query
    that is a [B, H, P, D] view of token-major storage (the fused prefill's)
    gives token-major output and the final ``contiguous()`` copies nothing."""
    with sdpa_kernel(list(_FUSED_SDPA)):
        if dec._sdpa_gqa is not False:
            try:
                out = F.scaled_dot_product_attention(query, key, value, dropout_p=dropout, is_causal=True,
                                                     scale=scale, enable_gqa=True)
                dec._sdpa_gqa = True
                return out.transpose(1, 2).contiguous()
            except RuntimeError:
                if dec._sdpa_gqa:
                    raise
                dec._sdpa_gqa = False
        g = query.shape[1] // key.shape[1]
        out = F.scaled_dot_product_attention(query, key.repeat_interleave(g, dim=1),
                                             value.repeat_interleave(g, dim=1), dropout_p=dropout, is_causal=True,
                                             scale=scale)
    return out.transpose(1, 2).contiguous()


def _no_attention_mask(*_, **__):
    return None


@dataclass(frozen=True)
class GreedyGenerationTiming:
    """Host timestamps around one synchronized fixed-length request (graph_decode.py:76-93)."""

    start_s: float
    first_token_s: float
    end_s: float

    @property
    def ttft_ms(self) -> float:
        return (self.first_token_s - self.start_s) * 1_000

    @property
    def decode_ms(self) -> float:
        return (self.end_s - self.first_token_s) * 1_000


class CudaGraphGreedyDecoder:
    """Reusable fixed-batch, fixed-length greedy decoder over a ``StaticCache``
    (graph_decode.py:96-479).  ``prepare`` captures the bodies once; each
    ``prefill`` copies a prompt into static storage and replays the reset-and-
    prefill graph; ``decode`` replays the one-token graph."""

    def __init__(self, model: torch.nn.Module, *, prompt_tokens: int, max_new_tokens: int, batch_size: int = 1,
                 device="cuda", prefill_only: bool = False, fused_decode: bool = True,
                 fused_prefill: bool = True, l2_warm: bool = True) -> None:
        if prompt_tokens < 1:
            raise ValueError("prompt_tokens must be positive")
        if batch_size < 1:
            raise ValueError("batch_size must be positive")
        minimum = 0 if prefill_only else 1
        if max_new_tokens < minimum:
            raise ValueError(f"max_new_tokens must be at least {minimum}")
        self.model = model
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("CudaGraphGreedyDecoder requires a ROCm (cuda) device")
        cfg = model.config.get_text_config(decoder=True)
        if getattr(cfg, "_attn_implementation", None) not in ("sdpa", _GRAPH_ATTENTION):
            raise ValueError("model must use the SDPA attention implementation")
        if model.training or getattr(cfg, "attention_dropout", 0.0) != 0.0:
            raise ValueError("CudaGraphGreedyDecoder requires eval-mode zero-dropout attention")
        if getattr(cfg, "sliding_window", None) is not None and getattr(cfg, "use_sliding_window", True):
            raise ValueError("CudaGraphGreedyDecoder requires full causal attention")
        if cfg.num_attention_heads % cfg.num_key_value_heads:
            raise ValueError("CudaGraphGreedyDecoder requires grouped-query attention")
        index = self.device.index if self.device.index is not None else torch.cuda.current_device()
        places = {(p.device.type, p.device.index) for p in model.parameters()}
        places |= {(b.device.type, b.device.index) for b in model.buffers() if b.numel()}
        if places != {("cuda", index)}:
            raise ValueError("CudaGraphGreedyDecoder requires a single-device model")
        self.device = torch.device("cuda", index)

        self.prompt_tokens = int(prompt_tokens)
        self.batch_size = int(batch_size)
        self.max_new_tokens = int(max_new_tokens)
        self._prefill_only = bool(prefill_only)
        self.max_cache_len = self.prompt_tokens if prefill_only else self.prompt_tokens + self.max_new_tokens
        self.cache = StaticCache(config=model.config, max_cache_len=self.max_cache_len)
        self._attention_is_prefill = True
        self._sdpa_gqa: Optional[bool] = None   # fused SDPA accepts grouped-query heads (learned in warm-up)
        q_heads = cfg.num_attention_heads
        self._attention_workspace = decode_attention_workspace(self.batch_size, q_heads, self.max_cache_len,
                                                               self.device)

        # Graph inputs/outputs: fixed storage addresses, never replaced.
        dev = self.device
        self._prompt = torch.empty((self.batch_size, self.prompt_tokens), dtype=torch.long, device=dev)
        self._prefill_positions = torch.arange(self.prompt_tokens, dtype=torch.long, device=dev)
        self._token = self._position = self._next_token = self._generated = None
        self._decode_seq_used = None
        if not prefill_only:
            self._token = torch.empty((self.batch_size, 1), dtype=torch.long, device=dev)
            self._position = torch.empty((1,), dtype=torch.long, device=dev)
            self._next_token = torch.empty_like(self._token)
            self._generated = torch.empty((self.batch_size, self.max_new_tokens), dtype=torch.long, device=dev)
            self._decode_seq_used = torch.empty((self.batch_size,), dtype=torch.int32, device=dev)
            self._greedy_ws = torch.empty((max(1, nat.lib().tq_greedy_step_workspace_elems(self.batch_size)),),
                                          dtype=torch.int32, device=dev)
        self._install_attention_backend()
        # One-token steps from fused kernels where the architecture allows
        # (tilequant_amd.fused_decode); otherwise the model's own forward.
        self._fused = None
        if fused_decode and not prefill_only:
            from .fused_decode import FusedDecodeStep

            try:
                self._fused = FusedDecodeStep(model, self.cache, self.batch_size, self.max_cache_len, self.device,
                                              l2_warm=l2_warm)
            except (ValueError, AttributeError):
                self._fused = None
        # The prompt forward from the row-parallel glue kernels where the
        # architecture allows (tilequant_amd.fused_decode.FusedPrefillStep);
        # otherwise the model's own forward.  It shares the decode step's
        # stacked projections and RoPE tables.
        self._fused_prefill = None
        if fused_prefill:
            from .fused_decode import FusedPrefillStep

            try:
                fd = self._fused
                self._fused_prefill = FusedPrefillStep(
                    model, self.cache, self.batch_size, self.prompt_tokens, self.max_cache_len, self.device,
                    attention=lambda q, k, v, scale: _prefill_attention(self, q, k, v, 0.0, scale),
                    layers=fd.layers if fd is not None else None,
                    cos_table=fd.cos_table if fd is not None else None,
                    sin_table=fd.sin_table if fd is not None else None)
            except (ValueError, AttributeError):
                self._fused_prefill = None
        self._prefill_graph: Optional[torch.cuda.CUDAGraph] = None
        self._graph: Optional[torch.cuda.CUDAGraph] = None
        self._prefill_logits: Optional[torch.Tensor] = None
        self._decode_logits: Optional[torch.Tensor] = None
        self.last_logits: Optional[torch.Tensor] = None
        self.prefill_captured = False
        self._prepared = False
        # decode steps replayed since the last prefill (the warm-up counts as
        # a prefill and one step); bounds decode() to the prepared cache
        self._steps_done = 0

    # ---- model binding ------------------------------------------------------
    def _install_attention_backend(self) -> None:
        AttentionInterface.register(_GRAPH_ATTENTION, _graph_attention)
        # The backend reads no mask; a default mask builder could synchronise
        # the host, which capture forbids (graph_decode.py:234-237).
        AttentionMaskInterface.register(_GRAPH_ATTENTION, _no_attention_mask)
        mods = [m for m in self.model.modules() if hasattr(m, "num_key_value_groups") and hasattr(m, "layer_idx")]
        if not mods:
            raise ValueError("model has no compatible attention modules")
        if any(hasattr(m, _DECODER_ATTRIBUTE) for m in mods):
            raise RuntimeError("model already has a CudaGraphGreedyDecoder attached")
        for m in mods:
            setattr(m, _DECODER_ATTRIBUTE, self)
        self.model.set_attn_implementation(_GRAPH_ATTENTION)

    def close(self, attn_implementation: str = "sdpa") -> None:
        """Detach from the model and release the graphs and the cache."""
        for m in self.model.modules():
            if getattr(m, _DECODER_ATTRIBUTE, None) is self:
                delattr(m, _DECODER_ATTRIBUTE)
        self.model.set_attn_implementation(attn_implementation)
        self._prefill_graph = self._graph = None
        self.cache = None
        self._prefill_logits = self._decode_logits = self.last_logits = None

    # ---- capture ------------------------------------------------------------
    @classmethod
    @torch.inference_mode()
    def prepare(cls, model: torch.nn.Module, *, prompt_tokens: int = 128, max_new_tokens: int = 512,
                batch_size: int = 1, device="cuda", prefill_only: bool = False,
                fused_decode: bool = True, fused_prefill: bool = True,
                l2_warm: bool = True) -> "CudaGraphGreedyDecoder":
        """Allocate, warm up and capture the prefill and decode graphs.
        ``l2_warm`` (fused decode step only): the producer kernel before each
        GEMM reads that GEMM's weights into the L2 of the XCD that will use
        them; the tokens and logits are the same either way."""
        dec = cls(model, prompt_tokens=prompt_tokens, max_new_tokens=max_new_tokens, batch_size=batch_size,
                  device=device, prefill_only=prefill_only, fused_decode=fused_decode, fused_prefill=fused_prefill,
                  l2_warm=l2_warm)
        try:
            dec._capture()
        except BaseException:
            dec.close()
            raise
        return dec

    @torch.inference_mode()
    def _capture(self) -> None:
        with torch.cuda.device(self.device):
            # Eager warm-up: allocates the cache and every lazily created
            # workspace before capture.
            self._prompt.zero_()
            self._prefill_body()
            decodes = not self._prefill_only and self.max_new_tokens > 1
            if decodes:
                self._decode_body()
            torch.cuda.synchronize(self.device)
            torch.cuda.empty_cache()
            self.prefill_captured = self.batch_size * self.prompt_tokens <= MAX_CAPTURED_PREFILL_TOKENS
            if self.prefill_captured:
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    self._prefill_body()
                self._prefill_graph = g
            else:
                self._prefill_body()
            if decodes:
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    self._decode_body()
                self._graph = g
            torch.cuda.synchronize(self.device)
        self._prepared = True
        self._steps_done = 1 if decodes else 0

    @torch.inference_mode()
    def _prefill_body(self) -> None:
        self._attention_is_prefill = True
        self.cache.reset()
        if not self._prefill_only:
            self._generated.zero_()
            self._position.fill_(self.prompt_tokens)
            self._decode_seq_used.fill_(self.prompt_tokens + 1)   # valid length of the first decode step
        if self._fused_prefill is not None:
            logits = self._fused_prefill(self._prompt)
        else:
            logits = self.model(input_ids=self._prompt, attention_mask=None,
                                position_ids=self._prefill_positions.view(1, -1), past_key_values=self.cache,
                                cache_position=self._prefill_positions, use_cache=True, logits_to_keep=1).logits
        self._prefill_logits = logits
        if not self._prefill_only:
            self._token.copy_(logits.argmax(dim=-1))
            self._generated[:, :1].copy_(self._token)

    @torch.inference_mode()
    def _decode_body(self) -> None:
        self._attention_is_prefill = False
        if self._fused is not None:
            logits = self._fused(self._token, self._position, self._decode_seq_used)
        else:
            logits = self.model(input_ids=self._token, attention_mask=None, position_ids=self._position.view(1, 1),
                                past_key_values=self.cache, cache_position=self._position, use_cache=True,
                                logits_to_keep=1).logits
        self._decode_logits = logits
        # position P consumes generated token P - prompt and produces the next one;
        # seq_used becomes the next step's valid length
        if logits.dtype in (torch.bfloat16, torch.float16) and logits.stride(-1) == 1:
            lg = logits.reshape(self.batch_size, -1)
            rc = nat.lib().tq_greedy_step(
                nat.ptr(lg), lg.stride(0), nat.dtype_code(lg.dtype), self.batch_size, lg.shape[1],
                nat.ptr(self._greedy_ws), self._greedy_ws.numel(), nat.ptr(self._next_token), nat.ptr(self._token),
                nat.ptr(self._generated), self._generated.stride(0), self.max_new_tokens, nat.ptr(self._position),
                self.prompt_tokens, nat.ptr(self._decode_seq_used), nat.stream_handle(self.device))
            nat.check(rc, "tq_greedy_step")
        else:
            self._next_token.copy_(logits.argmax(dim=-1))
            col = (self._position - self.prompt_tokens + 1).view(1, 1).expand(self.batch_size, 1)
            self._generated.scatter_(1, col, self._next_token)
            self._token.copy_(self._next_token)
            self._position.add_(1)
            self._decode_seq_used.copy_(self._position + 1)

    # ---- requests -----------------------------------------------------------
    def _prompt_from_host(self, prompt_ids) -> torch.Tensor:
        prompt = prompt_ids.to(dtype=torch.long) if isinstance(prompt_ids, torch.Tensor) else torch.tensor(
            prompt_ids, dtype=torch.long)
        if prompt.ndim == 1:
            prompt = prompt.unsqueeze(0)
        if tuple(prompt.shape) != (self.batch_size, self.prompt_tokens):
            raise ValueError(f"expected {(self.batch_size, self.prompt_tokens)}, got {tuple(prompt.shape)}")
        return prompt

    @torch.inference_mode()
    def prefill(self, prompt_ids) -> torch.Tensor:
        """Copy the prompt to the device and replay the reset-and-prefill graph.
        Returns the first generated token ids [B, 1] (or the last-position
        logits with ``prefill_only``)."""
        if self._prefill_graph is None and not self._prepared:
            raise RuntimeError("call CudaGraphGreedyDecoder.prepare() before prefill")
        prompt = self._prompt_from_host(prompt_ids)
        self._prompt.copy_(prompt, non_blocking=prompt.device.type == "cpu" and prompt.is_pinned())
        if self._prefill_graph is not None:
            self._prefill_graph.replay()
        else:
            self._prefill_body()
        if self._prefill_logits is None:
            raise RuntimeError("prefill graph did not retain logits")
        self.last_logits = self._prefill_logits
        self._steps_done = 0
        return self._prefill_logits if self._prefill_only else self._token

    @torch.inference_mode()
    def decode(self, steps: Optional[int] = None) -> torch.Tensor:
        """Replay the decode graph ``steps`` times (default: to the prepared
        bound) and return a device view of the generated ids so far."""
        if not self._prepared:
            raise RuntimeError("call CudaGraphGreedyDecoder.prepare() before decoding")
        if self._prefill_only:
            raise RuntimeError("decode() is unavailable after prepare(prefill_only=True)")
        if steps is None:
            steps = self.max_new_tokens - 1
        if not 0 <= steps <= self.max_new_tokens - 1:
            raise ValueError(f"steps must be in [0, {self.max_new_tokens - 1}]")
        if steps and self._graph is None:
            raise RuntimeError("call CudaGraphGreedyDecoder.prepare() before decoding")
        if self._steps_done + steps > self.max_new_tokens - 1:
            # the kernels would clamp at the cache end and return stale ids
            raise ValueError(f"{self._steps_done} decode steps since the last prefill; {steps} more would pass "
                             f"the prepared bound of {self.max_new_tokens - 1} (call prefill() first)")
        for _ in range(steps):
            self._graph.replay()
        self._steps_done += steps
        if steps:
            if self._decode_logits is None:
                raise RuntimeError("decode graph did not retain logits")
            self.last_logits = self._decode_logits
        return self._generated[:, : self._steps_done + 1]

    @torch.inference_mode()
    def generate(self, prompt_ids, *, new_tokens: Optional[int] = None) -> torch.Tensor:
        """One request; greedy ids on the device, no host synchronisation."""
        if new_tokens is None:
            new_tokens = self.max_new_tokens
        if not 1 <= new_tokens <= self.max_new_tokens:
            raise ValueError(f"new_tokens must be in [1, {self.max_new_tokens}]")
        self.prefill(prompt_ids)
        return self.decode(new_tokens - 1)

    @torch.inference_mode()
    def generate_timed(self, prompt_ids, *, new_tokens: Optional[int] = None):
        """Generate with synchronised timestamps (the benchmark protocol)."""
        if new_tokens is None:
            new_tokens = self.max_new_tokens
        torch.cuda.synchronize(self.device)
        start = time.perf_counter()
        self.prefill(prompt_ids)
        torch.cuda.synchronize(self.device)
        first = time.perf_counter()
        generated = self.decode(new_tokens - 1)
        torch.cuda.synchronize(self.device)
        return generated, GreedyGenerationTiming(start, first, time.perf_counter())
