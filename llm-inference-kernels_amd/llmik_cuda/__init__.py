"""llmik_cuda — gfx950 drop-in for the `llmik_cuda` torch extension of
bundle-adjuster/llm-inference-kernels.

Same module name, the same twelve functions with the same argument names,
order, defaults and return types as the reference binding
(bindings/extension.cpp:476-502), and the same validation messages, raised
as RuntimeError like the reference's TORCH_CHECK. Every op enqueues HIP
kernels from libllmik_hip.so on torch's current stream of the input's device
and allocates its outputs with torch, as the reference does. There is no
CPU or eager fallback: without the built library the import fails.

Additions beyond the reference surface (all optional, defaults reproduce
the reference):
  * `seqlen=-1` on decode_attention_int8 / decode_attention_int4: live
    length inside a preallocated cache, as decode_attention already has;
  * `w4a16_gemm_f32out`: the same GEMM with an fp32 output, used to gate
    the kernel against an fp32-accumulated oracle without fp16 rounding;
  * `quantize_per_token_into`, `quantize_v_per_token_int4_into`,
    `quantize_k_per_channel_groupwise_int4_into`: the writers quantising
    into a preallocated cache at a token offset (no torch.cat), used by the
    cat-free caches in `llmik_cuda.kv_cache`;
  * `quantize_weights_int4_groupwise`, `pack_int4_along_k`: GPU versions of
    the reference's host-side weight quantiser and packer
    (reference/quant_matmul_ref.py:39-88, 140-165), same arguments and
    results bit for bit, and `quantize_pack_weights_int4`, the two fused
    into the buffers QuantizedLinear registers
    (integration/w4a16_patch.py:78-84).
"""
from __future__ import annotations

from typing import Dict, List, Tuple

import torch

from ._lib import LIB_PATH, check, lib

__all__ = [
    "decode_attention", "decode_attention_v3", "quantize_per_token", "decode_attention_int8",
    "quantize_k_per_channel_groupwise_int4", "quantize_v_per_token_int4",
    "decode_attention_int4", "w4a16_gemm", "w4a16_dequantize", "rmsnorm", "silu_mul", "rope",
    "w4a16_gemm_f32out", "quantize_per_token_into", "quantize_v_per_token_int4_into",
    "quantize_k_per_channel_groupwise_int4_into", "quantize_weights_int4_groupwise",
    "pack_int4_along_k", "quantize_pack_weights_int4", "kivi_append_token_int4", "rope_qkv_append", "add_rmsnorm", "silu_mul_halves",
    "LIB_PATH",
]


def _is_device(t: torch.Tensor) -> bool:
    return t.is_cuda


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


# Zero-filled workspaces, one per (device, stream). The kernels leave the
# completion counters at the start of a workspace zeroed, so a workspace is
# reused by later calls on the same stream (stream order serialises them).
_WORKSPACES: Dict[Tuple[int, int], torch.Tensor] = {}
# Buffers replaced by a larger one. A HIP graph captured on a stream keeps the
# address of the workspace it was captured with, and replays keep writing
# partials and counters there, so a replaced buffer is never freed (the
# doubling growth bounds what is held to twice the largest workspace).
_RETIRED_WORKSPACES: List[torch.Tensor] = []


def _workspace(device: torch.device, stream: int, nbytes: int) -> Tuple[int, int]:
    if nbytes == 0:
        return 0, 0
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        size = max(nbytes, 2 * ws.numel() if ws is not None else 0)
        if ws is not None:
            _RETIRED_WORKSPACES.append(ws)
        ws = torch.zeros(size, dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws.data_ptr(), ws.numel()


def _ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


# ---------------------------------------------------------------- attention

def decode_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                     softmax_scale: float, seqlen: int = -1) -> torch.Tensor:
    """Split-K GQA decode attention over an fp16 KV cache.

    q [batch, n_heads, head_dim]; k, v [batch, n_kv_heads, kv_buf_len, head_dim],
    fp16, contiguous. `seqlen` (<= 0: the full kv_buf_len) is the live length
    of a preallocated cache read in place. Returns out [batch, n_heads,
    head_dim] fp16. Mirrors bindings/extension.cpp:26-83.
    """
    _require(_is_device(q) and _is_device(k) and _is_device(v), "q, k, v must be CUDA tensors")
    _require(q.dtype == torch.float16, "fp16 only for now")
    _require(q.is_contiguous() and k.is_contiguous() and v.is_contiguous(),
             "inputs must be contiguous")
    _require(k.dtype == torch.float16 and v.dtype == torch.float16, "k and v must be fp16")
    _require(q.dim() == 3 and k.dim() == 4 and v.dim() == 4,
             "q must be [batch, n_heads, head_dim] and k/v [batch, n_kv_heads, S, head_dim]")
    _require(k.shape == v.shape, "k and v must have the same shape")
    batch, n_heads, head_dim = q.shape
    n_kv_heads, kv_buf_len = k.size(1), k.size(2)
    _require(k.size(0) == batch and k.size(3) == head_dim, "q and k/v shapes disagree")
    seqlen_kv = int(seqlen) if seqlen > 0 else kv_buf_len
    _require(seqlen_kv <= kv_buf_len, "seqlen exceeds allocated cache length")
    out = torch.empty_like(q)
    with torch.cuda.device(q.device):
        stream = _stream(q)
        ws, ws_bytes = _workspace(q.device, stream, lib.llmik_attention_workspace_size(
            batch, n_heads, n_kv_heads, seqlen_kv, head_dim))
        check(lib.llmik_decode_attention_f16(
            _ptr(q), _ptr(k), _ptr(v), _ptr(out), batch, n_heads, n_kv_heads, seqlen_kv,
            head_dim, kv_buf_len, float(softmax_scale), ws, ws_bytes, stream))
    return out


def decode_attention_v3(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                        softmax_scale: float) -> torch.Tensor:
    """The reference's single-warp kernel entry (bindings/extension.cpp:89-115).

    Same result semantics as decode_attention over the whole cache; on this
    build it runs the same split-K kernel.
    """
    _require(_is_device(q) and _is_device(k) and _is_device(v), "q, k, v must be CUDA tensors")
    _require(q.dtype == torch.float16, "fp16 only for now")
    _require(q.is_contiguous() and k.is_contiguous() and v.is_contiguous(),
             "inputs must be contiguous")
    return decode_attention(q, k, v, softmax_scale, -1)


def decode_attention_int8(q: torch.Tensor, k_q: torch.Tensor, k_scale: torch.Tensor,
                          v_q: torch.Tensor, v_scale: torch.Tensor, softmax_scale: float,
                          seqlen: int = -1) -> torch.Tensor:
    """Decode attention over an INT8 per-token KV cache, dequant fused.

    k_q, v_q [batch, n_kv_heads, S, head_dim] int8; k_scale, v_scale
    [batch, n_kv_heads, S] fp16. Mirrors bindings/extension.cpp:152-194;
    `seqlen` is an addition (see module docstring).
    """
    _require(all(_is_device(t) for t in (q, k_q, k_scale, v_q, v_scale)),
             "all inputs must be CUDA tensors")
    _require(q.dtype == torch.float16, "q must be fp16")
    _require(k_q.dtype == torch.int8 and v_q.dtype == torch.int8, "k_q and v_q must be int8")
    _require(k_scale.dtype == torch.float16 and v_scale.dtype == torch.float16,
             "k_scale and v_scale must be fp16")
    _require(all(t.is_contiguous() for t in (q, k_q, k_scale, v_q, v_scale)),
             "all tensors must be contiguous")
    _require(q.dim() == 3 and k_q.dim() == 4 and k_q.shape == v_q.shape,
             "q must be [batch, n_heads, head_dim] and k_q/v_q [batch, n_kv_heads, S, head_dim]")
    batch, n_heads, head_dim = q.shape
    n_kv_heads, kv_buf_len = k_q.size(1), k_q.size(2)
    _require(k_q.size(0) == batch and k_q.size(3) == head_dim, "q and k_q/v_q shapes disagree")
    _require(tuple(k_scale.shape) == (batch, n_kv_heads, kv_buf_len)
             and k_scale.shape == v_scale.shape,
             "k_scale/v_scale must be [batch, n_kv_heads, S]")
    seqlen_kv = int(seqlen) if seqlen > 0 else kv_buf_len
    _require(seqlen_kv <= kv_buf_len, "seqlen exceeds allocated cache length")
    out = torch.empty_like(q)
    with torch.cuda.device(q.device):
        stream = _stream(q)
        ws, ws_bytes = _workspace(q.device, stream, lib.llmik_attention_workspace_size(
            batch, n_heads, n_kv_heads, seqlen_kv, head_dim))
        check(lib.llmik_decode_attention_int8(
            _ptr(q), _ptr(k_q), _ptr(k_scale), _ptr(v_q), _ptr(v_scale), _ptr(out), batch,
            n_heads, n_kv_heads, seqlen_kv, head_dim, kv_buf_len, float(softmax_scale), ws,
            ws_bytes, stream))
    return out


def decode_attention_int4(q: torch.Tensor, k_q: torch.Tensor, k_scale: torch.Tensor,
                          v_q: torch.Tensor, v_scale: torch.Tensor, group_size: int,
                          softmax_scale: float, seqlen: int = -1) -> torch.Tensor:
    """Decode attention over an INT4 KIVI KV cache, dequant fused.

    k_q, v_q [batch, n_kv_heads, S, head_dim/2] packed int4 (int8 dtype);
    k_scale [batch, n_kv_heads, n_groups, head_dim] fp16; v_scale
    [batch, n_kv_heads, S] fp16. Mirrors bindings/extension.cpp:269-314;
    `seqlen` is an addition (see module docstring).
    """
    _require(all(_is_device(t) for t in (q, k_q, k_scale, v_q, v_scale)),
             "all inputs must be CUDA tensors")
    _require(q.dtype == torch.float16, "q must be fp16")
    _require(k_q.dtype == torch.int8 and v_q.dtype == torch.int8,
             "k_q and v_q must be int8 (packed int4)")
    _require(k_scale.dtype == torch.float16 and v_scale.dtype == torch.float16,
             "k_scale and v_scale must be fp16")
    _require(all(t.is_contiguous() for t in (q, k_q, k_scale, v_q, v_scale)),
             "all tensors must be contiguous")
    _require(q.dim() == 3 and k_q.dim() == 4 and k_q.shape == v_q.shape and k_scale.dim() == 4,
             "q must be [batch, n_heads, head_dim], k_q/v_q [batch, n_kv_heads, S, head_dim/2]")
    batch, n_heads, head_dim = q.shape
    n_kv_heads, kv_buf_len = k_q.size(1), k_q.size(2)
    _require(k_q.size(0) == batch and 2 * k_q.size(3) == head_dim,
             "q and k_q/v_q shapes disagree")
    n_groups = k_scale.size(2)
    _require(k_scale.size(0) == batch and k_scale.size(1) == n_kv_heads
             and k_scale.size(3) == head_dim, "k_scale must be [batch, n_kv_heads, n_groups, head_dim]")
    _require(tuple(v_scale.shape) == (batch, n_kv_heads, kv_buf_len),
             "v_scale must be [batch, n_kv_heads, S]")
    _require(group_size > 0, "group_size must be positive")
    seqlen_kv = int(seqlen) if seqlen > 0 else kv_buf_len
    _require(seqlen_kv <= kv_buf_len, "seqlen exceeds allocated cache length")
    out = torch.empty_like(q)
    with torch.cuda.device(q.device):
        stream = _stream(q)
        ws, ws_bytes = _workspace(q.device, stream, lib.llmik_attention_workspace_size(
            batch, n_heads, n_kv_heads, seqlen_kv, head_dim))
        check(lib.llmik_decode_attention_int4(
            _ptr(q), _ptr(k_q), _ptr(k_scale), _ptr(v_q), _ptr(v_scale), _ptr(out), batch,
            n_heads, n_kv_heads, seqlen_kv, head_dim, kv_buf_len, int(group_size), n_groups,
            float(softmax_scale), ws, ws_bytes, stream))
    return out


# ---------------------------------------------------------------- KV writers

def _check_writer_input(x: torch.Tensor) -> Tuple[int, int, int, int]:
    _require(_is_device(x), "x must be CUDA")
    _require(x.dtype == torch.float16, "x must be fp16")
    _require(x.is_contiguous(), "x must be contiguous")
    _require(x.dim() == 4, "x must be [batch, n_kv_heads, seqlen, head_dim]")
    batch, n_kv_heads, seqlen, head_dim = x.shape
    _require(head_dim == 128, "only head_dim=128 supported")
    return batch, n_kv_heads, seqlen, head_dim


def quantize_per_token(x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """INT8 symmetric per-token quantisation (bindings/extension.cpp:120-146).

    x [batch, n_kv_heads, seqlen, 128] fp16 -> (q int8 same shape,
    scale [batch, n_kv_heads, seqlen] fp16), bit-exact with
    reference/kv_cache_ref.py quantize_per_token(x.float(), bits=8).
    """
    batch, n_kv_heads, seqlen, head_dim = _check_writer_input(x)
    q = torch.empty((batch, n_kv_heads, seqlen, head_dim), dtype=torch.int8, device=x.device)
    scale = torch.empty((batch, n_kv_heads, seqlen), dtype=torch.float16, device=x.device)
    with torch.cuda.device(x.device):
        check(lib.llmik_quantize_per_token_int8(_ptr(x), _ptr(q), _ptr(scale), batch, n_kv_heads,
                                                seqlen, head_dim, _stream(x)))
    return q, scale


def quantize_k_per_channel_groupwise_int4(x: torch.Tensor, group_size: int
                                          ) -> Tuple[torch.Tensor, torch.Tensor]:
    """KIVI K: INT4 per channel, grouped along the sequence
    (bindings/extension.cpp:200-229).

    Returns (q [batch, n_kv_heads, seqlen, 64] packed int4,
    scale [batch, n_kv_heads, ceil(seqlen/group_size), 128] fp16).
    """
    batch, n_kv_heads, seqlen, head_dim = _check_writer_input(x)
    _require(group_size > 0, "group_size must be positive")
    n_groups = (seqlen + group_size - 1) // group_size
    q = torch.empty((batch, n_kv_heads, seqlen, head_dim // 2), dtype=torch.int8, device=x.device)
    scale = torch.empty((batch, n_kv_heads, n_groups, head_dim), dtype=torch.float16,
                        device=x.device)
    with torch.cuda.device(x.device):
        check(lib.llmik_quantize_k_per_channel_groupwise_int4(
            _ptr(x), _ptr(q), _ptr(scale), batch, n_kv_heads, seqlen, head_dim, int(group_size),
            _stream(x)))
    return q, scale


def quantize_v_per_token_int4(x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """KIVI V: INT4 per token, packed (bindings/extension.cpp:235-261).

    Returns (q [batch, n_kv_heads, seqlen, 64] packed int4,
    scale [batch, n_kv_heads, seqlen] fp16).
    """
    batch, n_kv_heads, seqlen, head_dim = _check_writer_input(x)
    q = torch.empty((batch, n_kv_heads, seqlen, head_dim // 2), dtype=torch.int8, device=x.device)
    scale = torch.empty((batch, n_kv_heads, seqlen), dtype=torch.float16, device=x.device)
    with torch.cuda.device(x.device):
        check(lib.llmik_quantize_v_per_token_int4(_ptr(x), _ptr(q), _ptr(scale), batch,
                                                  n_kv_heads, seqlen, head_dim, _stream(x)))
    return q, scale


# ------------------------------------------------------- in-place KV writers

def _token_rows(x: torch.Tensor) -> int:
    """Token stride of x's (batch, kv_head) rows, in tokens. x is either
    contiguous or a token slice x = buf[:, :, a:b] of a contiguous 4-D
    buffer: within a row the tokens are contiguous, rows are equally spaced."""
    batch, n_kv_heads, n_tok, head_dim = x.shape
    _require(x.stride(3) == 1 and (n_tok <= 1 or x.stride(2) == head_dim),
             "x must be contiguous within each (batch, kv_head) row")
    if n_kv_heads > 1:
        row = x.stride(1)
        _require(batch <= 1 or x.stride(0) == n_kv_heads * row,
                 "x rows must be equally spaced (a token slice of a contiguous buffer)")
    elif batch > 1:
        row = x.stride(0)
    else:
        row = n_tok * head_dim
    _require(row % head_dim == 0 and row >= n_tok * head_dim,
             "x rows must be equally spaced (a token slice of a contiguous buffer)")
    return row // head_dim


def _check_into(x: torch.Tensor, q_cache: torch.Tensor, scale_cache: torch.Tensor, offset: int,
                packed: bool) -> Tuple[int, int, int, int, int, int]:
    _require(_is_device(x) and _is_device(q_cache) and _is_device(scale_cache),
             "all inputs must be CUDA tensors")
    _require(x.dtype == torch.float16, "x must be fp16")
    _require(q_cache.dtype == torch.int8 and scale_cache.dtype == torch.float16,
             "q_cache must be int8 and scale_cache fp16")
    _require(x.dim() == 4 and q_cache.dim() == 4,
             "x must be [batch, n_kv_heads, n, head_dim] and q_cache 4-D")
    batch, n_kv_heads, n_tok, head_dim = x.shape
    _require(head_dim == 128, "only head_dim=128 supported")
    _require(q_cache.is_contiguous() and scale_cache.is_contiguous(),
             "q_cache and scale_cache must be contiguous")
    cache_len = q_cache.size(2)
    width = head_dim // 2 if packed else head_dim
    _require(q_cache.size(0) == batch and q_cache.size(1) == n_kv_heads
             and q_cache.size(3) == width, "q_cache must be [batch, n_kv_heads, cache_len, %d]" % width)
    _require(0 <= offset and offset + n_tok <= cache_len, "offset + n exceeds the cache length")
    x_len = _token_rows(x)
    return batch, n_kv_heads, n_tok, head_dim, cache_len, x_len


def quantize_per_token_into(x: torch.Tensor, q_cache: torch.Tensor, scale_cache: torch.Tensor,
                            offset: int) -> None:
    """INT8 per-token quantisation of x [batch, n_kv_heads, n, 128] into
    q_cache [batch, n_kv_heads, cache_len, 128] / scale_cache [batch,
    n_kv_heads, cache_len] at positions offset..offset+n-1, in place. The
    codes and scales equal quantize_per_token(x)'s bit for bit."""
    batch, n_kv_heads, n_tok, head_dim, cache_len, x_len = _check_into(
        x, q_cache, scale_cache, int(offset), packed=False)
    _require(tuple(scale_cache.shape) == (batch, n_kv_heads, cache_len),
             "scale_cache must be [batch, n_kv_heads, cache_len]")
    with torch.cuda.device(x.device):
        check(lib.llmik_quantize_per_token_int8_into(
            _ptr(x), x_len, _ptr(q_cache), _ptr(scale_cache), batch, n_kv_heads, n_tok, head_dim,
            cache_len, int(offset), _stream(x)))


def quantize_v_per_token_int4_into(x: torch.Tensor, q_cache: torch.Tensor,
                                   scale_cache: torch.Tensor, offset: int) -> None:
    """KIVI V (INT4 per token, packed) into a preallocated cache at
    positions offset..offset+n-1; bit-equal to quantize_v_per_token_int4(x)."""
    batch, n_kv_heads, n_tok, head_dim, cache_len, x_len = _check_into(
        x, q_cache, scale_cache, int(offset), packed=True)
    _require(tuple(scale_cache.shape) == (batch, n_kv_heads, cache_len),
             "scale_cache must be [batch, n_kv_heads, cache_len]")
    with torch.cuda.device(x.device):
        check(lib.llmik_quantize_v_per_token_int4_into(
            _ptr(x), x_len, _ptr(q_cache), _ptr(scale_cache), batch, n_kv_heads, n_tok, head_dim,
            cache_len, int(offset), _stream(x)))


def kivi_append_token_int4(k: torch.Tensor, v: torch.Tensor, k_open: torch.Tensor,
                           k_q: torch.Tensor, k_scale: torch.Tensor, v_q: torch.Tensor,
                           v_scale: torch.Tensor, length: int, group_size: int) -> None:
    """Append token 0 of k, v [batch, n_kv_heads, n, 128] fp16 to a KIVI INT4
    cache holding `length` tokens, in one launch: V per token at position
    `length`; K after the open group's fp16 tokens in k_open [batch,
    n_kv_heads, group_size, 128], the open group re-quantised into k_q /
    k_scale. Bit-equal to the writers' path (llmik_cuda.kv_cache)."""
    _require(all(_is_device(t) for t in (k, v, k_open, k_q, k_scale, v_q, v_scale)),
             "all inputs must be CUDA tensors")
    _require(k.dtype == torch.float16 and v.dtype == torch.float16 and k_open.dtype == torch.float16,
             "k, v and k_open must be fp16")
    _require(k.dim() == 4 and k.shape[:2] == v.shape[:2] and k.size(3) == 128 and v.size(3) == 128,
             "k and v must be [batch, n_kv_heads, n, 128]")
    batch, n_kv_heads = k.size(0), k.size(1)
    max_len = k_q.size(2)
    n_groups = (max_len + group_size - 1) // group_size
    _require(tuple(k_q.shape) == (batch, n_kv_heads, max_len, 64) and k_q.shape == v_q.shape
             and k_q.dtype == torch.int8 and v_q.dtype == torch.int8,
             "k_q / v_q must be [batch, n_kv_heads, max_len, 64] int8")
    _require(tuple(k_scale.shape) == (batch, n_kv_heads, n_groups, 128)
             and tuple(v_scale.shape) == (batch, n_kv_heads, max_len)
             and k_scale.dtype == torch.float16 and v_scale.dtype == torch.float16,
             "k_scale / v_scale must be fp16 and match the cache's shape")
    _require(tuple(k_open.shape) == (batch, n_kv_heads, group_size, 128),
             "k_open must be [batch, n_kv_heads, group_size, 128]")
    _require(all(t.is_contiguous() for t in (k_open, k_q, k_scale, v_q, v_scale)),
             "cache tensors must be contiguous")
    with torch.cuda.device(k.device):
        check(lib.llmik_kivi_append_token_int4(
            _ptr(k), _token_rows(k), _ptr(v), _token_rows(v), _ptr(k_open), _ptr(k_q), _ptr(k_scale),
            _ptr(v_q), _ptr(v_scale), batch, n_kv_heads, 128, max_len, int(group_size), int(length),
            _stream(k)))


def quantize_k_per_channel_groupwise_int4_into(x: torch.Tensor, q_cache: torch.Tensor,
                                               scale_cache: torch.Tensor, offset: int,
                                               group_size: int) -> None:
    """KIVI K (INT4 per channel, grouped along the sequence) into a
    preallocated cache. offset is a multiple of group_size; x's n tokens form
    ceil(n / group_size) groups written to scale slots offset/group_size...,
    the last one possibly partial. Bit-equal to
    quantize_k_per_channel_groupwise_int4(x, group_size)."""
    _require(group_size > 0, "group_size must be positive")
    _require(int(offset) % group_size == 0, "offset must be a multiple of group_size")
    batch, n_kv_heads, n_tok, head_dim, cache_len, x_len = _check_into(
        x, q_cache, scale_cache, int(offset), packed=True)
    n_groups = (cache_len + group_size - 1) // group_size
    _require(tuple(scale_cache.shape) == (batch, n_kv_heads, n_groups, head_dim),
             "scale_cache must be [batch, n_kv_heads, ceil(cache_len/group_size), head_dim]")
    with torch.cuda.device(x.device):
        check(lib.llmik_quantize_k_per_channel_groupwise_int4_into(
            _ptr(x), x_len, _ptr(q_cache), _ptr(scale_cache), batch, n_kv_heads, n_tok, head_dim,
            cache_len, int(offset), int(group_size), _stream(x)))


# -------------------------------------------------------------------- W4A16

def _check_gemm(act: torch.Tensor, weight_packed: torch.Tensor, scale: torch.Tensor,
                group_size: int) -> Tuple[int, int, int]:
    _require(_is_device(act) and _is_device(weight_packed) and _is_device(scale),
             "all inputs must be CUDA tensors")
    _require(act.dtype == torch.float16, "act must be fp16")
    _require(weight_packed.dtype == torch.int32, "weight_packed must be int32 (uint32 bit pattern)")
    _require(scale.dtype == torch.float16, "scale must be fp16")
    _require(act.is_contiguous() and weight_packed.is_contiguous() and scale.is_contiguous(),
             "all tensors must be contiguous")
    _require(act.dim() == 2 and weight_packed.dim() == 2 and scale.dim() == 2,
             "all inputs must be 2D")
    M, K = act.shape
    k_packs, N = weight_packed.shape
    n_groups = scale.size(0)
    _require(K == k_packs * 8, "act.K must equal weight_packed.K_packs * 8")
    _require(scale.size(1) == N, "scale and weight_packed N mismatch")
    _require(group_size > 0 and group_size % 8 == 0, "group_size must be a positive multiple of 8")
    _require(K == n_groups * group_size, "K must equal n_groups * group_size")
    return M, N, K


def _gemm(act, weight_packed, scale, group_size, out_dtype, fn):
    M, N, K = _check_gemm(act, weight_packed, scale, group_size)
    out = torch.empty((M, N), dtype=out_dtype, device=act.device)
    if M == 0 or N == 0:
        return out
    if K == 0:
        return out.zero_()
    with torch.cuda.device(act.device):
        stream = _stream(act)
        ws, ws_bytes = _workspace(act.device, stream,
                                  lib.llmik_w4a16_workspace_size(M, N, K, int(group_size)))
        check(fn(_ptr(act), _ptr(weight_packed), _ptr(scale), _ptr(out), M, N, K,
                 int(group_size), ws, ws_bytes, stream))
    return out


def w4a16_gemm(act: torch.Tensor, weight_packed: torch.Tensor, scale: torch.Tensor,
               group_size: int) -> torch.Tensor:
    """out [M, N] fp16 = act [M, K] fp16 @ dequant(weight_packed [K/8, N] int32,
    scale [K/group_size, N] fp16), fp32 accumulation
    (bindings/extension.cpp:322-376)."""
    return _gemm(act, weight_packed, scale, group_size, torch.float16, lib.llmik_w4a16_gemm)


def w4a16_gemm_f32out(act: torch.Tensor, weight_packed: torch.Tensor, scale: torch.Tensor,
                      group_size: int) -> torch.Tensor:
    """w4a16_gemm with the fp32 accumulator returned instead of fp16."""
    return _gemm(act, weight_packed, scale, group_size, torch.float32,
                 lib.llmik_w4a16_gemm_f32out)


def w4a16_dequantize(weight_packed: torch.Tensor, scale: torch.Tensor,
                     group_size: int) -> torch.Tensor:
    """fp16 W [K, N] = fp16(code * scale[k // group_size]) from packed int4
    (bindings/extension.cpp:382-403)."""
    _require(_is_device(weight_packed) and _is_device(scale), "inputs must be CUDA")
    _require(weight_packed.dtype == torch.int32, "weight_packed int32")
    _require(scale.dtype == torch.float16, "scale fp16")
    _require(weight_packed.is_contiguous() and scale.is_contiguous(), "contiguous")
    _require(weight_packed.dim() == 2 and scale.dim() == 2, "weight_packed and scale must be 2D")
    K = weight_packed.size(0) * 8
    N = weight_packed.size(1)
    _require(scale.size(1) == N, "scale/weight N mismatch")
    _require(group_size > 0 and K % group_size == 0, "K must be a multiple of group_size")
    _require(scale.size(0) * group_size == K, "scale must have K / group_size rows")
    out = torch.empty((K, N), dtype=torch.float16, device=scale.device)
    with torch.cuda.device(scale.device):
        check(lib.llmik_w4a16_dequantize(_ptr(weight_packed), _ptr(scale), _ptr(out), K, N,
                                         int(group_size), _stream(scale)))
    return out


# ------------------------------------------------------ W4 weight quantiser

def _check_weight(W: torch.Tensor, group_size: int) -> Tuple[int, int]:
    _require(_is_device(W), "W must be a CUDA tensor")
    _require(W.dtype in (torch.float16, torch.float32), "W must be fp16 or fp32")
    _require(W.dim() == 2, "W must be 2D [K, N]")
    _require(W.is_contiguous(), "W must be contiguous")
    _require(int(group_size) > 0, "group_size must be positive")
    return int(W.shape[0]), int(W.shape[1])


def quantize_weights_int4_groupwise(W: torch.Tensor, group_size: int = 128
                                    ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Symmetric INT4 group-wise quantisation of W [K, N] (fp16 or fp32) on
    the GPU: (q [K, N] int8 in [-7, 7], scale [ceil(K/group_size), N] in
    W's dtype), bit for bit the reference's host-side function
    (reference/quant_matmul_ref.py:39-88), fp16 and fp32 semantics
    included."""
    K, N = _check_weight(W, group_size)
    g = int(group_size)
    n_groups = (K + g - 1) // g
    q = torch.empty((K, N), dtype=torch.int8, device=W.device)
    scale = torch.empty((n_groups, N), dtype=W.dtype, device=W.device)
    with torch.cuda.device(W.device):
        check(lib.llmik_quantize_weights_int4_groupwise(
            _ptr(W), int(W.dtype == torch.float16), K, N, g, _ptr(q), None, _ptr(scale), None,
            _stream(W)))
    return q, scale


def pack_int4_along_k(q_int8: torch.Tensor) -> torch.Tensor:
    """[K, N] int8 -> [K/8, N] int32, bits 4i..4i+3 of word (kp, n) = K
    position 8 kp + i (reference/quant_matmul_ref.py:140-165), on the GPU."""
    _require(_is_device(q_int8), "q must be a CUDA tensor")
    _require(q_int8.dtype == torch.int8 and q_int8.dim() == 2 and q_int8.is_contiguous(),
             "q must be a contiguous 2D int8 tensor")
    K, N = q_int8.shape
    assert K % 8 == 0, f"K={K} must be a multiple of 8 to pack int4 along K"
    packed = torch.empty((K // 8, N), dtype=torch.int32, device=q_int8.device)
    with torch.cuda.device(q_int8.device):
        check(lib.llmik_pack_int4_along_k(_ptr(q_int8), K, N, _ptr(packed), _stream(q_int8)))
    return packed


def quantize_pack_weights_int4(W: torch.Tensor, group_size: int = 128
                               ) -> Tuple[torch.Tensor, torch.Tensor]:
    """The two buffers QuantizedLinear registers for a [K, N] weight
    (integration/w4a16_patch.py:78-84): (pack_int4_along_k(q) [K/8, N]
    int32, scale.to(float16)), with (q, scale) =
    quantize_weights_int4_groupwise(W, group_size). One kernel when K and
    group_size are multiples of 8."""
    K, N = _check_weight(W, group_size)
    g = int(group_size)
    assert K % 8 == 0, f"K={K} must be a multiple of 8 to pack int4 along K"
    n_groups = (K + g - 1) // g
    packed = torch.empty((K // 8, N), dtype=torch.int32, device=W.device)
    scale16 = torch.empty((n_groups, N), dtype=torch.float16, device=W.device)
    with torch.cuda.device(W.device):
        if g % 8 == 0:
            check(lib.llmik_quantize_weights_int4_groupwise(
                _ptr(W), int(W.dtype == torch.float16), K, N, g, None, _ptr(packed), None,
                _ptr(scale16), _stream(W)))
        else:
            q = torch.empty((K, N), dtype=torch.int8, device=W.device)
            check(lib.llmik_quantize_weights_int4_groupwise(
                _ptr(W), int(W.dtype == torch.float16), K, N, g, _ptr(q), None, None,
                _ptr(scale16), _stream(W)))
            check(lib.llmik_pack_int4_along_k(_ptr(q), K, N, _ptr(packed), _stream(W)))
    return packed, scale16


# --------------------------------------------------------- fused elementwise

def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm over the last dim, fp32 math (bindings/extension.cpp:408-424)."""
    _require(_is_device(x) and _is_device(weight), "inputs must be CUDA")
    _require(x.dtype == torch.float16 and weight.dtype == torch.float16, "fp16 only")
    H = x.size(-1)
    _require(weight.numel() == H, "weight length must match x last dim")
    x2 = x.contiguous().reshape(-1, H)
    w = weight.contiguous()
    out = torch.empty_like(x2)
    with torch.cuda.device(x.device):
        check(lib.llmik_rmsnorm(_ptr(x2), _ptr(w), _ptr(out), x2.size(0), H, float(eps),
                                _stream(x)))
    return out.reshape(x.shape)


def silu_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up, elementwise (bindings/extension.cpp:427-441)."""
    _require(_is_device(gate) and _is_device(up), "inputs must be CUDA")
    _require(gate.dtype == torch.float16 and up.dtype == torch.float16, "fp16 only")
    _require(gate.shape == up.shape, "gate and up must have the same shape")
    g = gate.contiguous()
    u = up.contiguous()
    out = torch.empty_like(g)
    with torch.cuda.device(gate.device):
        check(lib.llmik_silu_mul(_ptr(g), _ptr(u), _ptr(out), g.numel(), _stream(gate)))
    return out


def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x * cos + rotate_half(x) * sin; x [B, H, S, D], cos/sin [B, S, D] or
    broadcastable [S, D] / [1, S, D] (bindings/extension.cpp:446-473)."""
    _require(_is_device(x) and _is_device(cos) and _is_device(sin), "inputs must be CUDA")
    _require(x.dtype == torch.float16, "fp16 only")
    _require(x.dim() == 4, "x must be [B, H, S, D]")
    B, H, S, D = x.shape
    _require(D % 2 == 0, "head_dim must be even")
    _require(cos.dtype == torch.float16 and sin.dtype == torch.float16, "fp16 only")
    xc = x.contiguous()

    def norm_cs(t: torch.Tensor) -> torch.Tensor:
        t = t.contiguous()
        if t.numel() == B * S * D:
            return t.reshape(B, S, D)
        _require(t.numel() == S * D, "cos/sin must be [B,S,D] or broadcastable [S,D]/[1,S,D]")
        return t.reshape(1, S, D).expand(B, S, D).contiguous()

    cc = norm_cs(cos)
    sc = norm_cs(sin)
    out = torch.empty_like(xc)
    with torch.cuda.device(x.device):
        check(lib.llmik_rope(_ptr(xc), _ptr(cc), _ptr(sc), _ptr(out), B, H, S, D, _stream(x)))
    return out


# ------------------------------------------------------ decode-step merges
# One launch each for consecutive ops of the reference's patched decode step
# (integration/prealloc_cache.py:61-76,126-133); same results as the ops they
# replace.

def rope_qkv_append(qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                    k_cache: torch.Tensor, v_cache: torch.Tensor, pos: int) -> torch.Tensor:
    """One token's fused q|k|v projection qkv [batch, (n_heads + 2 n_kv_heads)
    * head_dim] fp16: returns rope(q) [batch, n_heads, head_dim] and writes
    rope(k) and v into slot `pos` of k_cache / v_cache [batch, n_kv_heads,
    max_len, head_dim]. cos / sin: the position's [head_dim] rotary row.
    Equals rope(q, cos, sin), rope(k, cos, sin) and the two slot copies."""
    _require(all(_is_device(t) for t in (qkv, cos, sin, k_cache, v_cache)), "inputs must be CUDA")
    _require(all(t.dtype == torch.float16 for t in (qkv, cos, sin, k_cache, v_cache)), "fp16 only")
    _require(k_cache.dim() == 4 and k_cache.shape == v_cache.shape and k_cache.is_contiguous()
             and v_cache.is_contiguous(), "caches must be contiguous [batch, n_kv_heads, max_len, head_dim]")
    B, Hkv, max_len, D = k_cache.shape
    _require(D % 2 == 0, "head_dim must be even")
    _require(cos.numel() == D and sin.numel() == D, "cos/sin must be one [head_dim] row")
    _require(qkv.size(0) == B and qkv.numel() % (B * D) == 0, "qkv must be [batch, heads * head_dim]")
    H = qkv.numel() // (B * D) - 2 * Hkv
    _require(H > 0, "qkv holds fewer than 2 n_kv_heads + 1 heads")
    _require(0 <= pos < max_len, "pos outside the cache")
    x = qkv.contiguous()
    cc, sc = cos.contiguous(), sin.contiguous()
    q = torch.empty((B, H, D), dtype=torch.float16, device=qkv.device)
    with torch.cuda.device(qkv.device):
        check(lib.llmik_rope_qkv_append_f16(_ptr(x), _ptr(cc), _ptr(sc), _ptr(q), _ptr(k_cache),
                                            _ptr(v_cache), B, H, Hkv, D, max_len, int(pos),
                                            _stream(qkv)))
    return q


def add_rmsnorm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                eps: float) -> Tuple[torch.Tensor, torch.Tensor]:
    """h = x + residual (fp16) and rmsnorm(h, weight, eps) in one launch;
    returns (h, normed). The last dim is at most 8192, a multiple of 8."""
    _require(all(_is_device(t) for t in (x, residual, weight)), "inputs must be CUDA")
    _require(all(t.dtype == torch.float16 for t in (x, residual, weight)), "fp16 only")
    _require(x.shape == residual.shape, "x and residual must have the same shape")
    Hd = x.size(-1)
    _require(weight.numel() == Hd, "weight length must match x last dim")
    x2 = x.contiguous().reshape(-1, Hd)
    r2 = residual.contiguous().reshape(-1, Hd)
    w = weight.contiguous()
    h = torch.empty_like(x2)
    out = torch.empty_like(x2)
    with torch.cuda.device(x.device):
        check(lib.llmik_add_rmsnorm(_ptr(x2), _ptr(r2), _ptr(w), _ptr(h), _ptr(out), x2.size(0), Hd,
                                    float(eps), _stream(x)))
    return h.reshape(x.shape), out.reshape(x.shape)


def silu_mul_halves(gate_up: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up over a fused gate|up projection [..., 2 * cols]
    (gate = the first half of the last dim): silu_mul of the two halves."""
    _require(_is_device(gate_up), "inputs must be CUDA")
    _require(gate_up.dtype == torch.float16, "fp16 only")
    _require(gate_up.size(-1) % 16 == 0, "the last dim must be 2 * cols with cols a multiple of 8")
    cols = gate_up.size(-1) // 2
    gu = gate_up.contiguous()
    rows = gu.numel() // (2 * cols) if cols else 0
    out = torch.empty(gu.shape[:-1] + (cols,), dtype=torch.float16, device=gu.device)
    with torch.cuda.device(gate_up.device):
        check(lib.llmik_silu_mul_halves(_ptr(gu), _ptr(out), rows, cols, _stream(gate_up)))
    return out
