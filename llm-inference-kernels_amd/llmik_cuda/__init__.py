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

from collections.abc import Mapping
from typing import Iterator, Tuple

import torch

from ._lib import LIB_PATH, check, lib

try:
    from . import _C
except ImportError as e:   # the module is unusable without its native half
    raise ImportError(f"llmik_cuda: the torch extension llmik_cuda/_C is missing or broken ({e}); "
                      "build it with `python llm-inference-kernels_amd/build_lib.py`") from e

__all__ = [
    "decode_attention", "decode_attention_v3", "quantize_per_token", "decode_attention_int8",
    "quantize_k_per_channel_groupwise_int4", "quantize_v_per_token_int4",
    "decode_attention_int4", "w4a16_gemm", "w4a16_dequantize", "rmsnorm", "silu_mul", "rope",
    "w4a16_gemm_f32out", "quantize_per_token_into", "quantize_v_per_token_int4_into",
    "quantize_k_per_channel_groupwise_int4_into", "quantize_weights_int4_groupwise",
    "pack_int4_along_k", "quantize_pack_weights_int4", "kivi_append_token_int4", "rope_qkv_append", "add_rmsnorm", "silu_mul_halves",
    "w4a16_gemm_swiglu", "interleave_gate_up", "w4a16_gemm_qkv_rope", "interleave_head_halves", "LIB_PATH",
]


def _is_device(t: torch.Tensor) -> bool:
    return t.is_cuda


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


class _WorkspaceView(Mapping):
    """Read-only view of the split-K workspaces the ops cache in _C, one
    zero-filled buffer per (device index, stream handle). The kernels leave
    the completion counters at the start of a workspace zeroed, so a
    workspace is reused by later calls on the same stream (stream order
    serialises them). A buffer replaced by a larger one is kept alive, not
    freed: a HIP graph captured earlier on that stream still addresses it."""

    def __getitem__(self, key: Tuple[int, int]) -> torch.Tensor:
        return _C.workspaces()[key]

    def __iter__(self) -> Iterator[Tuple[int, int]]:
        return iter(_C.workspaces())

    def __len__(self) -> int:
        return len(_C.workspaces())


_WORKSPACES = _WorkspaceView()
_token_rows = _C.token_rows


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
    return _C.decode_attention(q, k, v, float(softmax_scale), int(seqlen))


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
    return _C.decode_attention_int8(q, k_q, k_scale, v_q, v_scale, float(softmax_scale), int(seqlen))


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
    return _C.decode_attention_int4(q, k_q, k_scale, v_q, v_scale, int(group_size),
                                        float(softmax_scale), int(seqlen))


# ---------------------------------------------------------------- KV writers

def quantize_per_token(x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """INT8 symmetric per-token quantisation (bindings/extension.cpp:120-146).

    x [batch, n_kv_heads, seqlen, 128] fp16 -> (q int8 same shape,
    scale [batch, n_kv_heads, seqlen] fp16), bit-exact with
    reference/kv_cache_ref.py quantize_per_token(x.float(), bits=8).
    """
    _require(_is_device(x), "x must be CUDA")
    return _C.quantize_per_token(x)


def quantize_k_per_channel_groupwise_int4(x: torch.Tensor, group_size: int
                                          ) -> Tuple[torch.Tensor, torch.Tensor]:
    """KIVI K: INT4 per channel, grouped along the sequence
    (bindings/extension.cpp:200-229).

    Returns (q [batch, n_kv_heads, seqlen, 64] packed int4,
    scale [batch, n_kv_heads, ceil(seqlen/group_size), 128] fp16).
    """
    _require(_is_device(x), "x must be CUDA")
    return _C.quantize_k_per_channel_groupwise_int4(x, int(group_size))


def quantize_v_per_token_int4(x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """KIVI V: INT4 per token, packed (bindings/extension.cpp:235-261).

    Returns (q [batch, n_kv_heads, seqlen, 64] packed int4,
    scale [batch, n_kv_heads, seqlen] fp16).
    """
    _require(_is_device(x), "x must be CUDA")
    return _C.quantize_v_per_token_int4(x)


# ------------------------------------------------------- in-place KV writers

def quantize_per_token_into(x: torch.Tensor, q_cache: torch.Tensor, scale_cache: torch.Tensor,
                            offset: int) -> None:
    """INT8 per-token quantisation of x [batch, n_kv_heads, n, 128] into
    q_cache [batch, n_kv_heads, cache_len, 128] / scale_cache [batch,
    n_kv_heads, cache_len] at positions offset..offset+n-1, in place. The
    codes and scales equal quantize_per_token(x)'s bit for bit."""
    _require(_is_device(x) and _is_device(q_cache) and _is_device(scale_cache),
                 "all inputs must be CUDA tensors")
    _C.quantize_per_token_into(x, q_cache, scale_cache, int(offset))


def quantize_v_per_token_int4_into(x: torch.Tensor, q_cache: torch.Tensor,
                                   scale_cache: torch.Tensor, offset: int) -> None:
    """KIVI V (INT4 per token, packed) into a preallocated cache at
    positions offset..offset+n-1; bit-equal to quantize_v_per_token_int4(x)."""
    _require(_is_device(x) and _is_device(q_cache) and _is_device(scale_cache),
                 "all inputs must be CUDA tensors")
    _C.quantize_v_per_token_int4_into(x, q_cache, scale_cache, int(offset))


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
    _C.kivi_append_token_int4(k, v, k_open, k_q, k_scale, v_q, v_scale, int(length), int(group_size))


def quantize_k_per_channel_groupwise_int4_into(x: torch.Tensor, q_cache: torch.Tensor,
                                               scale_cache: torch.Tensor, offset: int,
                                               group_size: int) -> None:
    """KIVI K (INT4 per channel, grouped along the sequence) into a
    preallocated cache. offset is a multiple of group_size; x's n tokens form
    ceil(n / group_size) groups written to scale slots offset/group_size...,
    the last one possibly partial. Bit-equal to
    quantize_k_per_channel_groupwise_int4(x, group_size)."""
    _require(_is_device(x) and _is_device(q_cache) and _is_device(scale_cache),
                 "all inputs must be CUDA tensors")
    _C.quantize_k_per_channel_groupwise_int4_into(x, q_cache, scale_cache, int(offset), int(group_size))


# -------------------------------------------------------------------- W4A16

def w4a16_gemm(act: torch.Tensor, weight_packed: torch.Tensor, scale: torch.Tensor,
               group_size: int) -> torch.Tensor:
    """out [M, N] fp16 = act [M, K] fp16 @ dequant(weight_packed [K/8, N] int32,
    scale [K/group_size, N] fp16), fp32 accumulation
    (bindings/extension.cpp:322-376)."""
    _require(_is_device(act) and _is_device(weight_packed) and _is_device(scale),
                 "all inputs must be CUDA tensors")
    return _C.w4a16_gemm(act, weight_packed, scale, int(group_size))


def w4a16_gemm_f32out(act: torch.Tensor, weight_packed: torch.Tensor, scale: torch.Tensor,
                      group_size: int) -> torch.Tensor:
    """w4a16_gemm with the fp32 accumulator returned instead of fp16."""
    _require(_is_device(act) and _is_device(weight_packed) and _is_device(scale),
                 "all inputs must be CUDA tensors")
    return _C.w4a16_gemm_f32out(act, weight_packed, scale, int(group_size))


def interleave_gate_up(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """The column order `w4a16_gemm_swiglu` expects, from the gate and up
    weights [K, I] (any dtype, I % 32 == 0): [K, 2 I] in 64-column tiles of
    32 gate columns followed by the same 32 up columns. Quantising it column
    by column gives each column the codes and scales it has in the separate
    weights."""
    _require(gate.shape == up.shape and gate.dim() == 2 and gate.shape[1] % 32 == 0,
             "gate and up must be [K, I] with I % 32 == 0")
    K, inter = gate.shape
    return torch.stack((gate.reshape(K, inter // 32, 32), up.reshape(K, inter // 32, 32)),
                       dim=2).reshape(K, 2 * inter)


def w4a16_gemm_swiglu(act: torch.Tensor, weight_packed: torch.Tensor, scale: torch.Tensor,
                      group_size: int) -> torch.Tensor:
    """The decode step's gate|up projection and SwiGLU in one launch:
    out [M, N/2] fp16 = silu(g) * up for a weight whose columns are
    `interleave_gate_up(gate, up)` (packed [K/8, N], scale [K/g, N]), with
    g and up the fp16 products (prealloc_cache.py:129-130: silu_mul of the
    gate and up projections). 1 <= M <= 16, N % 64 == 0."""
    _require(_is_device(act) and _is_device(weight_packed) and _is_device(scale),
             "all inputs must be CUDA tensors")
    return _C.w4a16_gemm_swiglu(act, weight_packed, scale, int(group_size))


def interleave_head_halves(w: torch.Tensor) -> torch.Tensor:
    """The column order `w4a16_gemm_qkv_rope` expects, from a concatenated
    q | k | v weight [K, n_heads_total * 128]: each head's columns become
    dimensions 0..31, 64..95, 32..63, 96..127 (its two halves interleaved in
    32-column blocks). Quantising it column by column gives each column the
    codes and scales it has in the concatenated weight."""
    _require(w.dim() == 2 and w.shape[1] % 128 == 0, "w must be [K, n_heads_total * 128]")
    K, n = w.shape
    return w.reshape(K, n // 128, 2, 2, 32).transpose(2, 3).reshape(K, n)


def w4a16_gemm_qkv_rope(act: torch.Tensor, weight_packed: torch.Tensor, scale: torch.Tensor,
                        cos: torch.Tensor, sin: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                        pos: int, n_heads: int, group_size: int) -> torch.Tensor:
    """The decode step's q|k|v projection, rope and cache append in one
    launch (head_dim 128): returns the roped q [batch, n_heads, 128] and
    writes slot `pos` of k_cache / v_cache [batch, n_kv_heads, max_len, 128],
    for a weight whose columns are `interleave_head_halves(W_q | W_k | W_v)`
    (prealloc_cache.py:42-110,132-133: the q/k/v projections, rope and the
    cache update). The bits of `w4a16_gemm` on the concatenated weight and
    `rope_qkv_append`. 1 <= batch <= 16."""
    _require(all(_is_device(t) for t in (act, weight_packed, scale, cos, sin, k_cache, v_cache)),
             "all inputs must be CUDA tensors")
    return _C.w4a16_gemm_qkv_rope(act, weight_packed, scale, cos, sin, k_cache, v_cache, int(pos),
                                  int(n_heads), int(group_size))


def w4a16_dequantize(weight_packed: torch.Tensor, scale: torch.Tensor,
                     group_size: int) -> torch.Tensor:
    """fp16 W [K, N] = fp16(code * scale[k // group_size]) from packed int4
    (bindings/extension.cpp:382-403)."""
    _require(_is_device(weight_packed) and _is_device(scale), "inputs must be CUDA")
    return _C.w4a16_dequantize(weight_packed, scale, int(group_size))


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
    return _C.rmsnorm(x, weight, float(eps))


def silu_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up, elementwise (bindings/extension.cpp:427-441)."""
    _require(_is_device(gate) and _is_device(up), "inputs must be CUDA")
    return _C.silu_mul(gate, up)


def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x * cos + rotate_half(x) * sin; x [B, H, S, D], cos/sin [B, S, D] or
    broadcastable [S, D] / [1, S, D] (bindings/extension.cpp:446-473)."""
    _require(_is_device(x) and _is_device(cos) and _is_device(sin), "inputs must be CUDA")
    return _C.rope(x, cos, sin)


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
    return _C.rope_qkv_append(qkv, cos, sin, k_cache, v_cache, int(pos))


def add_rmsnorm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                eps: float) -> Tuple[torch.Tensor, torch.Tensor]:
    """h = x + residual (fp16) and rmsnorm(h, weight, eps) in one launch;
    returns (h, normed). The last dim is at most 8192, a multiple of 8."""
    _require(all(_is_device(t) for t in (x, residual, weight)), "inputs must be CUDA")
    return _C.add_rmsnorm(x, residual, weight, float(eps))


def silu_mul_halves(gate_up: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up over a fused gate|up projection [..., 2 * cols]
    (gate = the first half of the last dim): silu_mul of the two halves."""
    _require(_is_device(gate_up), "inputs must be CUDA")
    return _C.silu_mul_halves(gate_up)
