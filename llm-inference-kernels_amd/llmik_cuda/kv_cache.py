"""Cat-free quantised KV caches: preallocated buffers appended in place.

The reference keeps its INT4 KIVI cache as a list of packed chunks that it
torch.cat's onto the whole cache whenever a group of tokens is drained and
again, with the freshly quantised fp16 residual, before every decode-step
attention call (Int4KIVICache.append_only / get_quantized_for_attention,
integration/kv_int4_cache.py:104-144,168-206). Here the cache is one
preallocated buffer per tensor of capacity `max_len`; appends quantise
straight into it at the live offset (the *_into writers) and attention reads
it in place over the live length (`seqlen`). The stored codes and scales are
bit-identical to the reference cache's view after the same appends:

* Int4KIVICache: K per channel grouped along the sequence (full groups
  quantised once, from the same fp16 tokens the reference drains), the
  trailing partial group -- the reference's fp16 residual -- re-quantised on
  every append from the fp16 tokens kept here, exactly as the reference
  re-quantises its residual before each attention call; V per token.
* Int8KVCache: K and V per token (the INT8 path of the reference has no
  cache class; this is its prealloc_cache.PreallocCache layout,
  integration/prealloc_cache.py:42-79, in INT8).
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import (decode_attention_int4, decode_attention_int8, kivi_append_token_int4,
               quantize_k_per_channel_groupwise_int4_into, quantize_per_token_into,
               quantize_v_per_token_int4_into)


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _check_append(k: torch.Tensor, v: torch.Tensor, batch: int, n_kv_heads: int, head_dim: int,
                  length: int, max_len: int) -> int:
    _require(k.shape == v.shape and k.dim() == 4, "k and v must be [batch, n_kv_heads, n, head_dim]")
    _require(k.dtype == torch.float16 and v.dtype == torch.float16, "k and v must be fp16")
    _require(k.size(0) == batch and k.size(1) == n_kv_heads and k.size(3) == head_dim,
             "k/v shape does not match the cache")
    n = k.size(2)
    _require(length + n <= max_len, "append exceeds the cache capacity")
    return n


class Int8KVCache:
    """INT8 per-token K and V in preallocated [batch, n_kv_heads, max_len, ...]
    buffers; `append` quantises new tokens in place, `attention` runs the
    INT8 decode attention over the live length."""

    def __init__(self, batch: int, n_kv_heads: int, max_len: int, head_dim: int = 128,
                 device: Optional[torch.device] = None) -> None:
        dev = torch.device("cuda") if device is None else torch.device(device)
        self.batch, self.n_kv_heads, self.max_len, self.head_dim = batch, n_kv_heads, max_len, head_dim
        shape = (batch, n_kv_heads, max_len, head_dim)
        self.k_q = torch.zeros(shape, dtype=torch.int8, device=dev)
        self.v_q = torch.zeros(shape, dtype=torch.int8, device=dev)
        self.k_scale = torch.zeros(shape[:3], dtype=torch.float16, device=dev)
        self.v_scale = torch.zeros(shape[:3], dtype=torch.float16, device=dev)
        self.length = 0

    def append(self, k: torch.Tensor, v: torch.Tensor) -> None:
        """k, v [batch, n_kv_heads, n, head_dim] fp16."""
        n = _check_append(k, v, self.batch, self.n_kv_heads, self.head_dim, self.length,
                          self.max_len)
        if n == 0:
            return
        quantize_per_token_into(k, self.k_q, self.k_scale, self.length)
        quantize_per_token_into(v, self.v_q, self.v_scale, self.length)
        self.length += n

    def get_quantized_for_attention(self) -> Tuple[torch.Tensor, ...]:
        """(k_q, k_scale, v_q, v_scale, length): the whole buffers and the
        live length to pass as `seqlen`."""
        return self.k_q, self.k_scale, self.v_q, self.v_scale, self.length

    def attention(self, q: torch.Tensor, softmax_scale: float) -> torch.Tensor:
        """q [batch, n_heads, head_dim] fp16 over the live tokens."""
        _require(self.length > 0, "the cache is empty")
        return decode_attention_int8(q, self.k_q, self.k_scale, self.v_q, self.v_scale,
                                     softmax_scale, self.length)

    def reset(self) -> None:
        self.length = 0


class Int4KIVICache:
    """KIVI INT4 cache (K per channel in groups of `group_size` tokens along
    the sequence, V per token, packed two codes per byte) in preallocated
    buffers, with the fp16 tokens of the open (partial) K group kept for
    re-quantisation. Same stored codes and scales as the reference's
    Int4KIVICache after the same appends (see the module docstring)."""

    def __init__(self, batch: int, n_kv_heads: int, max_len: int, group_size: int = 32,
                 head_dim: int = 128, device: Optional[torch.device] = None) -> None:
        _require(group_size > 0, "group_size must be positive")
        dev = torch.device("cuda") if device is None else torch.device(device)
        self.batch, self.n_kv_heads, self.max_len = batch, n_kv_heads, max_len
        self.group_size, self.head_dim = group_size, head_dim
        n_groups = (max_len + group_size - 1) // group_size
        self.k_q = torch.zeros((batch, n_kv_heads, max_len, head_dim // 2), dtype=torch.int8,
                               device=dev)
        self.v_q = torch.zeros_like(self.k_q)
        self.k_scale = torch.zeros((batch, n_kv_heads, n_groups, head_dim), dtype=torch.float16,
                                   device=dev)
        self.v_scale = torch.zeros((batch, n_kv_heads, max_len), dtype=torch.float16, device=dev)
        # fp16 tokens of the open K group (positions group_start .. length-1)
        self.k_open = torch.zeros((batch, n_kv_heads, group_size, head_dim), dtype=torch.float16,
                                  device=dev)
        self.length = 0

    def append(self, k: torch.Tensor, v: torch.Tensor) -> None:
        """k, v [batch, n_kv_heads, n, head_dim] fp16."""
        n = _check_append(k, v, self.batch, self.n_kv_heads, self.head_dim, self.length,
                          self.max_len)
        if n == 0:
            return
        g = self.group_size
        if n == 1 and g <= 128 and self.head_dim == 128:
            # A decode step: one launch for the V token, the open group's new
            # fp16 token and its re-quantisation.
            kivi_append_token_int4(k, v, self.k_open, self.k_q, self.k_scale, self.v_q, self.v_scale,
                                   self.length, g)
            self.length += 1
            return
        quantize_v_per_token_int4_into(v, self.v_q, self.v_scale, self.length)
        pos = 0
        r = self.length % g
        if r:
            # Fill the open group and re-quantise it (still partial, or now full).
            take = min(g - r, n)
            self.k_open[:, :, r:r + take].copy_(k[:, :, :take])
            quantize_k_per_channel_groupwise_int4_into(
                self.k_open[:, :, :r + take], self.k_q, self.k_scale, self.length - r, g)
            pos = take
        full = (n - pos) // g * g
        if full:
            # Whole groups straight from the input.
            quantize_k_per_channel_groupwise_int4_into(
                k[:, :, pos:pos + full], self.k_q, self.k_scale, self.length + pos, g)
            pos += full
        rest = n - pos
        if rest:
            # A new open group.
            self.k_open[:, :, :rest].copy_(k[:, :, pos:])
            quantize_k_per_channel_groupwise_int4_into(
                self.k_open[:, :, :rest], self.k_q, self.k_scale, self.length + pos, g)
        self.length += n

    def get_quantized_for_attention(self) -> Tuple[torch.Tensor, ...]:
        """(k_q, k_scale, v_q, v_scale, length): the whole buffers and the
        live length to pass as `seqlen` (the reference returns freshly
        concatenated tensors of exactly the live length instead)."""
        return self.k_q, self.k_scale, self.v_q, self.v_scale, self.length

    def attention(self, q: torch.Tensor, softmax_scale: float) -> torch.Tensor:
        """q [batch, n_heads, head_dim] fp16 over the live tokens."""
        _require(self.length > 0, "the cache is empty")
        return decode_attention_int4(q, self.k_q, self.k_scale, self.v_q, self.v_scale,
                                     self.group_size, softmax_scale, self.length)

    def get_seq_length(self) -> int:
        return self.length

    def reset(self) -> None:
        self.length = 0
