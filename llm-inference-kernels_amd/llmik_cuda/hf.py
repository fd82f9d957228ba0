"""Hugging Face transformers (>= 5) integration of the llmik decode path.

The reference hooks transformers 4.x by rebinding
torch.nn.functional.scaled_dot_product_attention (integration/attention_patch.py:38-85,
prealloc_cache.py:82-110) and by replacing LlamaSdpaAttention.forward for its
INT4 cache (attention_patch.py:178-273). transformers 5 has neither
LlamaSdpaAttention nor a repeat_kv before the attention call: LlamaAttention
looks its attention function up by name in a registry
(ALL_ATTENTION_FUNCTIONS[config._attn_implementation]) and passes K/V
un-expanded [B, Hkv, S, D]. This module plugs into that registry:

* ``register()`` adds the attention implementation ``"llmik"`` (and its mask
  function, the SDPA one). Use it with
  ``model.set_attn_implementation("llmik")`` or
  ``from_pretrained(..., attn_implementation="llmik")``. One-token decode
  steps over an fp16 cache run ``decode_attention``; over a ``KIVICache``
  they run ``decode_attention_int4`` on the packed buffers; prefill, padded
  batches (an explicit mask) and anything else run transformers' own SDPA
  path, as the reference's hooks fall back to the original SDPA.
* ``PreallocCache``: the reference's cat-free fp16 cache
  (prealloc_cache.py:42-79) as a transformers 5 Cache; attention reads the
  preallocated buffers in place over the live length (the ``seqlen`` of
  decode_attention).
* ``KIVICache``: the reference's Int4KIVICache (kv_int4_cache.py:70-245) as a
  transformers 5 Cache over the cat-free llmik_cuda.kv_cache.Int4KIVICache:
  prefill sees the reference's fp16 view (dequantised full groups plus the
  fp16 tokens of the open group, kv_int4_cache.py:225-245); decode sees the
  packed buffers.
* ``QuantizedLinear`` / ``patch_model_w4a16``: integration/w4a16_patch.py:56-174
  (W4A16 projections; the GEMM below the measured crossover, 448-768 rows,
  dequantise + matmul from there),
  with the weights quantised on the GPU (quantize_pack_weights_int4, the
  same bits as the reference's torch quantiser).
* ``fused_ops()``: the fused RMSNorm / SwiGLU / RoPE patches of
  prealloc_cache.fused_decode (:113-144).
"""
from __future__ import annotations

import contextlib
import weakref
from typing import Optional, Tuple

import torch
import torch.nn as nn
from transformers import AttentionInterface
from transformers.cache_utils import Cache, CacheLayerMixin
from transformers.integrations.sdpa_attention import sdpa_attention_forward
from transformers.masking_utils import AttentionMaskInterface, sdpa_mask

from . import (decode_attention, quantize_pack_weights_int4, rmsnorm, rope, silu_mul,
               w4a16_dequantize, w4a16_gemm)
from .kv_cache import Int4KIVICache

ATTN_IMPLEMENTATION = "llmik"

# Packed K buffer (data_ptr) -> the KIVI cache layer that owns it. A KIVI
# layer's update() hands its packed buffers to the attention function in
# place of fp16 K/V; this map finds the layer (scales, group size, live
# length) from them.
_KIVI_LAYERS: "weakref.WeakValueDictionary[int, KIVILayer]" = weakref.WeakValueDictionary()


def _full_buffer(t: torch.Tensor) -> Optional[torch.Tensor]:
    """If t [B, Hkv, L, D] is the token prefix [:, :, :L] of a contiguous
    [B, Hkv, max_len, D] buffer, that whole buffer (a view); else None."""
    B, H, L, D = t.shape
    s0, s1, s2, s3 = t.stride()
    if s3 != 1 or s2 != D or s1 % D != 0 or (B > 1 and s0 != H * s1) or s1 // D < L:
        return None
    off = t.storage_offset()
    if off % s1 != 0 or off + B * H * s1 > t.untyped_storage().nbytes() // t.element_size():
        return None   # not starting at token 0 of a row, or not a whole buffer
    return torch.as_strided(t, (B, H, s1 // D, D), (H * s1, s1, D, 1))


def _decode_fp16(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                 scale: float) -> Optional[torch.Tensor]:
    q = query[:, :, 0].contiguous()
    if key.is_contiguous() and value.is_contiguous():
        return decode_attention(q, key, value, scale)
    kf, vf = _full_buffer(key), _full_buffer(value)
    if kf is None or vf is None or kf.shape != vf.shape:
        return None
    return decode_attention(q, kf, vf, scale, key.shape[2])


def llmik_attention_forward(module: nn.Module, query: torch.Tensor, key: torch.Tensor,
                            value: torch.Tensor, attention_mask: Optional[torch.Tensor],
                            dropout: float = 0.0, scaling: Optional[float] = None,
                            **kwargs) -> Tuple[torch.Tensor, None]:
    """transformers 5 attention function: query [B, H, q_len, D], key/value
    [B, Hkv, S, D] (or a KIVI layer's packed buffers) -> ([B, q_len, H, D], None)."""
    scale = float(scaling) if scaling is not None else query.shape[-1] ** -0.5
    # The decode kernels compute plain softmax(scale q K^T) V over the whole
    # live cache (the reference hooks Llama only): logit soft-capping,
    # attention sinks (s_aux), sliding windows and additive position biases
    # take the SDPA path.
    plain = all(kwargs.get(name) is None for name in ("softcap", "s_aux", "sliding_window", "position_bias"))
    decode = (query.dim() == 4 and query.shape[2] == 1 and query.shape[-1] == 128
              and query.dtype == torch.float16 and query.is_cuda and attention_mask is None
              and not dropout and not kwargs.get("output_attentions", False) and plain)
    out = None
    if key.dtype == torch.int8:
        layer = _KIVI_LAYERS.get(key.data_ptr())
        if layer is None:
            raise RuntimeError("llmik attention: int8 K/V that no KIVICache layer owns")
        if decode:
            out = layer.attention(query[:, :, 0].contiguous(), scale)
        else:
            key, value = layer.fp16_view()
    elif decode and key.dtype == torch.float16:
        out = _decode_fp16(query, key, value, scale)
    if out is None:
        return sdpa_attention_forward(module, query, key, value, attention_mask, dropout=dropout,
                                      scaling=scaling, **kwargs)
    return out.unsqueeze(1), None


def register() -> str:
    """Register the "llmik" attention implementation (idempotent); returns its name."""
    AttentionInterface.register(ATTN_IMPLEMENTATION, llmik_attention_forward)
    AttentionMaskInterface.register(ATTN_IMPLEMENTATION, sdpa_mask)
    return ATTN_IMPLEMENTATION


# ------------------------------------------------------------------ caches

class PreallocLayer(CacheLayerMixin):
    """One layer's fp16 K/V in [B, Hkv, max_len, D] buffers written in place;
    update() returns the live prefix (views of the buffers)."""

    is_sliding = False

    def __init__(self, max_len: int) -> None:
        super().__init__()
        self.max_len = max_len
        self.length = 0

    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        B, H, _, D = key_states.shape
        self.keys = key_states.new_zeros((B, H, self.max_len, D))
        self.values = value_states.new_zeros((B, H, self.max_len, D))
        self.is_initialized = True

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args, **kwargs
               ) -> Tuple[torch.Tensor, torch.Tensor]:
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        n = key_states.shape[-2]
        if self.length + n > self.max_len:
            raise RuntimeError(f"PreallocCache: {self.length + n} tokens exceed max_len {self.max_len}")
        self.keys[:, :, self.length:self.length + n] = key_states
        self.values[:, :, self.length:self.length + n] = value_states
        self.length += n
        return self.keys[:, :, :self.length], self.values[:, :, :self.length]

    def get_mask_sizes(self, query_length: int) -> Tuple[int, int]:
        return self.length + query_length, 0

    def get_seq_length(self) -> int:
        return self.length

    def get_max_length(self) -> int:
        return self.max_len

    def reset(self) -> None:
        self.length = 0


class PreallocCache(Cache):
    """Cat-free fp16 KV cache of `max_len` tokens per layer
    (integration/prealloc_cache.py:42-79 for transformers 5)."""

    def __init__(self, max_len: int) -> None:
        super().__init__(layer_class_to_replicate=lambda: PreallocLayer(max_len))
        self.max_len = max_len


class KIVILayer(CacheLayerMixin):
    """One layer's KIVI INT4 cache (K per channel in groups of `group_size`
    tokens, V per token) in preallocated buffers, plus the fp16 tokens of the
    open group for the reference's prefill view."""

    is_sliding = False

    def __init__(self, max_len: int, group_size: int) -> None:
        super().__init__()
        self.max_len, self.group_size = max_len, group_size
        self.cache: Optional[Int4KIVICache] = None
        self.v_open: Optional[torch.Tensor] = None

    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        B, H, _, D = key_states.shape
        self.cache = Int4KIVICache(B, H, self.max_len, self.group_size, D, device=key_states.device)
        self.v_open = value_states.new_zeros((B, H, self.group_size, D))
        _KIVI_LAYERS[self.cache.k_q.data_ptr()] = self
        self.is_initialized = True

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args, **kwargs
               ) -> Tuple[torch.Tensor, torch.Tensor]:
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        c, g = self.cache, self.group_size
        n = key_states.shape[-2]
        start = c.length
        c.append(key_states.contiguous(), value_states.contiguous())
        # fp16 V tokens of the (new) open group, for fp16_view()
        open0 = c.length // g * g
        lo = max(open0, start)
        if c.length > lo:
            self.v_open[:, :, lo - open0:c.length - open0] = value_states[:, :, lo - start:]
        if n == 1:
            return c.k_q, c.v_q   # decode: the attention function reads the packed cache
        return self.fp16_view()

    def attention(self, q: torch.Tensor, scale: float) -> torch.Tensor:
        return self.cache.attention(q, scale)

    def fp16_view(self) -> Tuple[torch.Tensor, torch.Tensor]:
        """The reference cache's fp16 view (kv_int4_cache.py:225-245):
        dequantised full groups (fp32 code * scale -> fp16) and the fp16
        tokens of the open group."""
        c, g = self.cache, self.group_size
        full = c.length // g * g
        k_q = _unpack_int4(c.k_q[:, :, :full])
        v_q = _unpack_int4(c.v_q[:, :, :full])
        grp = torch.arange(full, device=k_q.device) // g
        k = (k_q.float() * c.k_scale.index_select(2, grp).float()).half()
        v = (v_q.float() * c.v_scale[:, :, :full].float().unsqueeze(-1)).half()
        r = c.length - full
        return (torch.cat([k, c.k_open[:, :, :r]], dim=2),
                torch.cat([v, self.v_open[:, :, :r]], dim=2))

    def get_mask_sizes(self, query_length: int) -> Tuple[int, int]:
        return self.get_seq_length() + query_length, 0

    def get_seq_length(self) -> int:
        return self.cache.length if self.cache is not None else 0

    def get_max_length(self) -> int:
        return self.max_len

    def reset(self) -> None:
        if self.cache is not None:
            self.cache.reset()


class KIVICache(Cache):
    """KIVI INT4 KV cache for transformers 5 (integration/kv_int4_cache.py:70-245),
    cat-free: `max_len` tokens per layer, K groups of `group_size` tokens."""

    def __init__(self, max_len: int, group_size: int = 32) -> None:
        super().__init__(layer_class_to_replicate=lambda: KIVILayer(max_len, group_size))
        self.max_len, self.group_size = max_len, group_size


def _unpack_int4(p: torch.Tensor) -> torch.Tensor:
    """[..., D/2] packed int8 (even channel in the low nibble) -> [..., D] int8."""
    x = p.to(torch.int32)
    lo = (x << 28) >> 28
    hi = (x << 24) >> 28
    return torch.stack([lo, hi], dim=-1).reshape(*p.shape[:-1], 2 * p.shape[-1]).to(torch.int8)


# ------------------------------------------------------------------ W4A16

_TARGET_LINEAR_NAMES = ("q_proj", "k_proj", "v_proj", "o_proj", "up_proj", "gate_proj", "down_proj")


def dequant_path_threshold(N: int) -> int:
    """Rows from which dequantise + matmul (hipBLASLt) beats w4a16_gemm on
    MI355X, measured at the Llama-3-8B shapes: w4a16_gemm is faster up to
    1024 rows for N = 4096 (K = 4096 or 14336; 47.1 against 52.6 us and
    129.1 against 151.5 at 1024, 70.2 against 64.1 at 1536) and up to 768
    for N = 14336 (113.2 against 114.3; 139.3 against 122.6 at 1024). The
    reference switches at 256
    (integration/w4a16_patch.py:89), where w4a16_gemm is 2.0-2.4x faster.
    Below the threshold the output is also the exact one (fp32 accumulation
    of unrounded weights, within 2e-3 of the float64 product; the fp16
    dequantised weights of the other path are not)."""
    return 1536 if N <= 8192 else 1024


class QuantizedLinear(nn.Module):
    """W4A16 replacement for nn.Linear(bias=False) (integration/w4a16_patch.py:56-141):
    packed INT4 weights [K/8, N] int32 and fp16 scales [K/g, N]; forward runs
    w4a16_gemm below dequant_path_threshold(N) rows and dequantise + matmul
    from there."""

    def __init__(self, weight_fp16: torch.Tensor, group_size: int = 128) -> None:
        super().__init__()
        N, K = weight_fp16.shape
        if K % group_size != 0 or K % 8 != 0:
            raise RuntimeError(f"in_features={K} must be a multiple of group_size={group_size} and of 8")
        self.in_features, self.out_features, self.group_size = K, N, group_size
        packed, scale = quantize_pack_weights_int4(weight_fp16.detach().t().contiguous().float(),
                                                   group_size)
        self.register_buffer("weight_packed", packed)
        self.register_buffer("scale", scale)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        shape = x.shape
        x2 = x.reshape(-1, self.in_features).contiguous()
        if x2.shape[0] < dequant_path_threshold(self.out_features):
            out = w4a16_gemm(x2, self.weight_packed, self.scale, self.group_size)
        else:
            out = torch.matmul(x2, w4a16_dequantize(self.weight_packed, self.scale, self.group_size))
        return out.reshape(*shape[:-1], self.out_features)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"group_size={self.group_size}, bits=4")


def patch_model_w4a16(model: nn.Module, *, group_size: int = 128) -> int:
    """Replace each bias-free q/k/v/o/gate/up/down projection Linear of
    model.model.layers with a QuantizedLinear (one-way, as the reference's
    patch_model_w4a16, w4a16_patch.py:143-174). Returns the count."""
    replaced = 0
    for layer in model.model.layers:
        for parent_name in ("self_attn", "mlp"):
            parent = getattr(layer, parent_name)
            for name, child in list(parent.named_children()):
                if name in _TARGET_LINEAR_NAMES and isinstance(child, nn.Linear):
                    if child.bias is not None:
                        raise RuntimeError(f"{parent_name}.{name} has a bias; QuantizedLinear has none")
                    setattr(parent, name, QuantizedLinear(child.weight, group_size))
                    replaced += 1
    return replaced


# ------------------------------------------------------------------ fused ops

@contextlib.contextmanager
def fused_ops():
    """RMSNorm, SwiGLU and RoPE of transformers' Llama as the llmik fused
    kernels for the duration of the block (prealloc_cache.fused_decode,
    integration/prealloc_cache.py:113-144). Restores the originals on exit."""
    from transformers.models.llama import modeling_llama as ml
    orig = (ml.LlamaRMSNorm.forward, ml.LlamaMLP.forward, ml.apply_rotary_pos_emb)

    def rms_fwd(self, hidden_states):
        return rmsnorm(hidden_states, self.weight, self.variance_epsilon)

    def mlp_fwd(self, x):
        return self.down_proj(silu_mul(self.gate_proj(x), self.up_proj(x)))

    def rope_fwd(q, k, cos, sin, unsqueeze_dim=1):
        return rope(q, cos, sin), rope(k, cos, sin)

    ml.LlamaRMSNorm.forward, ml.LlamaMLP.forward, ml.apply_rotary_pos_emb = rms_fwd, mlp_fwd, rope_fwd
    try:
        yield
    finally:
        ml.LlamaRMSNorm.forward, ml.LlamaMLP.forward, ml.apply_rotary_pos_emb = orig
