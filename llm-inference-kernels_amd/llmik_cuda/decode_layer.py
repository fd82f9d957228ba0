"""One decoder layer's decode step on llmik ops, and its capture in a HIP graph.

The reference runs a Llama decode step on these ops by patching transformers:
RMSNorm, SwiGLU and RoPE become `rmsnorm`, `silu_mul` and `rope`
(integration/prealloc_cache.py:113-144), each new token's K and V are written
in place into a preallocated `[B, Hkv, max_len, D]` cache whose live prefix
`decode_attention(q, kbuf, vbuf, scale, seqlen)` reads (:42-110), and the
projections are W4A16 `QuantizedLinear`s (integration/w4a16_patch.py:67-116).
`DecodeLayer` is that sequence for one layer, without the model around it:

    n1 = rmsnorm(x);  q, k, v = q_proj(n1), k_proj(n1), v_proj(n1)
    q, k = rope(q), rope(k);  kbuf[:, :, pos] = k;  vbuf[:, :, pos] = v
    h = x + o_proj(decode_attention(q, kbuf, vbuf, scale, pos + 1))
    out = h + down_proj(silu_mul(gate_proj(n2), up_proj(n2))),  n2 = rmsnorm(h)

With `fused=True` (the default) the step makes 8 launches instead of 17:
the q|k|v projection, rope of q and k and the cache-slot writes are one
launch (`w4a16_gemm_qkv_rope` over the concatenated weight with each head's
halves interleaved), `add_rmsnorm` takes the residual add and the second
norm, and gate|up with its SwiGLU is one launch (`w4a16_gemm_swiglu` over the
gate and up columns interleaved in 64-column tiles). Codes and scales per
column are those of the separate matrices. Where those launches do not apply
(a batch above 16, another head_dim) the step runs a column-concatenated
projection followed by `rope_qkv_append` / `silu_mul_halves`. `fused=False`
runs the op-by-op sequence above.
`DecodeStack` runs merged layers in sequence with each layer's last residual
add carried into the next layer's first RMSNorm launch.

Every op enqueues on the current stream without a host synchronisation, the
split-K reductions are deterministic and the per-stream workspace is reused,
so `capture(x, pos)` records one step in a `torch.cuda.CUDAGraph` whose
replays reproduce the eager step bit for bit. A graph holds one position (the
cache slot and the live length are baked into its launches): a serving loop
captures one graph per position, or per bucket of positions, and replays it.
"""
from __future__ import annotations

import math
from typing import Dict, Optional, Tuple

import torch

from . import (add_rmsnorm, decode_attention, interleave_gate_up, interleave_head_halves,
               quantize_pack_weights_int4, rmsnorm, rope, rope_qkv_append, silu_mul, silu_mul_halves,
               w4a16_gemm, w4a16_gemm_qkv_rope, w4a16_gemm_swiglu)


class W4Linear:
    """A W4A16 projection: an fp32 or fp16 [K, N] weight quantised on the GPU
    in QuantizedLinear's convention (integration/w4a16_patch.py:78-84: int4
    codes of the fp32 weight, group-wise fp16 scales), applied with
    `w4a16_gemm`."""

    def __init__(self, w_kn: torch.Tensor, group_size: int = 128) -> None:
        self.in_features, self.out_features = w_kn.shape
        self.group_size = group_size
        self.weight_packed, self.scale = quantize_pack_weights_int4(w_kn.float().contiguous(), group_size)

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        return w4a16_gemm(x, self.weight_packed, self.scale, self.group_size)

    def swiglu(self, x: torch.Tensor) -> torch.Tensor:
        """silu(gate) * up of a weight built from `interleave_gate_up`."""
        return w4a16_gemm_swiglu(x, self.weight_packed, self.scale, self.group_size)

    def qkv_rope(self, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, k_cache: torch.Tensor,
                 v_cache: torch.Tensor, pos: int, n_heads: int) -> torch.Tensor:
        """Roped q of a weight built from `interleave_head_halves`; k and v
        into cache slot `pos`."""
        return w4a16_gemm_qkv_rope(x, self.weight_packed, self.scale, cos, sin, k_cache, v_cache, pos,
                                   n_heads, self.group_size)


def rope_tables(max_len: int, head_dim: int, theta: float, device: torch.device) -> Tuple[torch.Tensor, torch.Tensor]:
    """cos / sin of the rotary embedding, [max_len, head_dim] fp16, in the
    half-split layout `rope` rotates (frequencies repeated over both halves)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float64) / head_dim))
    ang = torch.arange(max_len, dtype=torch.float64)[:, None] * inv_freq[None, :]
    ang = torch.cat([ang, ang], dim=1)
    return ang.cos().half().to(device), ang.sin().half().to(device)


class DecodeLayer:
    """A Llama-style layer (GQA attention, SwiGLU MLP, W4A16 projections) with
    a preallocated fp16 KV cache of `max_len` positions for `batch` sequences.

    `weights` maps q, k, v, o, gate, up, down to [in, out] fp32 matrices and
    ln1, ln2 to [hidden] fp16 vectors; missing entries are drawn from a seeded
    generator (N(0, 0.02) matrices, N(1, 0.1) norm weights). Only the packed
    codes and fp16 scales of the matrices are kept: in `proj` under their
    names, or with `fused=True` as "qkv" and "gate_up" column concatenations
    (gate|up interleaved in 64-column tiles when the SwiGLU launch applies);
    `columns[name]` gives (key in `proj`, the indices of the columns of that
    projection's output, in order). `merge_swiglu=False` keeps the merged
    step's gate|up projection and `silu_mul_halves` as two launches,
    `merge_rope=False` its q|k|v projection and `rope_qkv_append`."""

    NAMES = ("q", "k", "v", "o", "gate", "up", "down")

    def __init__(self, hidden: int, n_heads: int, n_kv_heads: int, intermediate: int, batch: int,
                 max_len: int, device: Optional[torch.device] = None, head_dim: int = 128,
                 group_size: int = 128, eps: float = 1e-5, rope_theta: float = 500000.0,
                 weights: Optional[Dict[str, torch.Tensor]] = None, seed: int = 0,
                 fused: bool = True, merge_swiglu: bool = True, merge_rope: bool = True) -> None:
        if n_heads * head_dim != hidden or n_heads % n_kv_heads != 0:
            raise RuntimeError("hidden must be n_heads * head_dim and n_heads a multiple of n_kv_heads")
        dev = torch.device("cuda") if device is None else torch.device(device)
        self.hidden, self.n_heads, self.n_kv_heads = hidden, n_heads, n_kv_heads
        self.head_dim, self.intermediate, self.batch, self.max_len = head_dim, intermediate, batch, max_len
        self.eps = eps
        self.scale = 1.0 / math.sqrt(head_dim)
        kv = n_kv_heads * head_dim
        shapes = {"q": (hidden, hidden), "k": (hidden, kv), "v": (hidden, kv), "o": (hidden, hidden),
                  "gate": (hidden, intermediate), "up": (hidden, intermediate), "down": (intermediate, hidden)}
        weights = dict(weights or {})
        gen = torch.Generator(device=dev).manual_seed(seed)
        for name in self.NAMES:
            if name not in weights:
                weights[name] = torch.randn(shapes[name], generator=gen, device=dev) * 0.02
        for name in ("ln1", "ln2"):
            if name not in weights:
                weights[name] = (1.0 + 0.1 * torch.randn(hidden, generator=gen, device=dev)).half()
        # the merged kernels' limits: add_rmsnorm rows of at most 8192, 16-byte vectors
        self.fused = fused and hidden % 8 == 0 and hidden <= 8192 and intermediate % 8 == 0
        # gate|up + SwiGLU in one launch: the streaming GEMV's rows and tiles
        stream_ok = batch <= 16 and group_size >= 32 and group_size & (group_size - 1) == 0 and hidden % 32 == 0
        self.swiglu = self.fused and merge_swiglu and stream_ok and intermediate % 32 == 0
        # q|k|v + rope + cache append in one launch: the same, and 128-wide heads
        self.qkv_rope = self.fused and merge_rope and stream_ok and head_dim == 128
        span = lambda a, b: torch.arange(a, b)  # noqa: E731
        if self.fused:
            cat = lambda *ns: torch.cat([weights.pop(n) for n in ns], dim=1)  # noqa: E731
            qkv = cat("q", "k", "v")
            n_qkv = hidden + 2 * kv
            if self.qkv_rope:
                qkv = interleave_head_halves(qkv)
                c = span(0, n_qkv)
                dd = c % 128
                order = (c // 128) * 128 + (dd % 64 // 32) * 64 + (dd // 64) * 32 + dd % 32
            else:
                order = span(0, n_qkv)
            self.proj = {"qkv": W4Linear(qkv, group_size), "o": W4Linear(weights.pop("o"), group_size),
                         "down": W4Linear(weights.pop("down"), group_size)}
            self.columns = {"q": ("qkv", order[:hidden]), "k": ("qkv", order[hidden:hidden + kv]),
                            "v": ("qkv", order[hidden + kv:]), "o": ("o", span(0, hidden)),
                            "down": ("down", span(0, hidden))}
            if self.swiglu:
                self.proj["gate_up"] = W4Linear(interleave_gate_up(weights.pop("gate"), weights.pop("up")),
                                                group_size)
                gate_cols = (span(0, intermediate) // 32) * 64 + span(0, intermediate) % 32
                self.columns["gate"] = ("gate_up", gate_cols)
                self.columns["up"] = ("gate_up", gate_cols + 32)
            else:
                self.proj["gate_up"] = W4Linear(cat("gate", "up"), group_size)
                self.columns["gate"] = ("gate_up", span(0, intermediate))
                self.columns["up"] = ("gate_up", span(intermediate, 2 * intermediate))
        else:
            self.proj = {name: W4Linear(weights.pop(name), group_size) for name in self.NAMES}
            self.columns = {name: (name, span(0, shapes[name][1])) for name in self.NAMES}
        self.ln1 = weights["ln1"].to(dev, torch.float16).contiguous()
        self.ln2 = weights["ln2"].to(dev, torch.float16).contiguous()
        self.cos, self.sin = rope_tables(max_len, head_dim, rope_theta, dev)
        if not self.fused:
            # Per-position tables already broadcast over the batch ([max_len,
            # batch, D]): rope takes a position's [batch, 1, D] slice as is,
            # where a [1, D] slice would be expanded by a copy on every call.
            self.cos_b = self.cos[:, None, :].expand(max_len, batch, head_dim).contiguous()
            self.sin_b = self.sin[:, None, :].expand(max_len, batch, head_dim).contiguous()
        shape = (batch, n_kv_heads, max_len, head_dim)
        self.kbuf = torch.zeros(shape, dtype=torch.float16, device=dev)
        self.vbuf = torch.zeros(shape, dtype=torch.float16, device=dev)

    def step(self, x: torch.Tensor, pos: int) -> torch.Tensor:
        """One decode step for the token at position `pos` (0-based) of every
        sequence: x [batch, hidden] fp16 -> [batch, hidden] fp16. Writes the
        token's K and V at cache slot `pos` and attends over positions
        0..pos."""
        if not 0 <= pos < self.max_len:
            raise RuntimeError(f"position {pos} outside the cache (max_len {self.max_len})")
        if self.fused:
            h, mlp = self.step_parts(x, pos)
            return h + mlp
        B, H, Hkv, D = self.batch, self.n_heads, self.n_kv_heads, self.head_dim
        p = self.proj
        n1 = rmsnorm(x, self.ln1, self.eps)
        cos, sin = self.cos_b[pos].view(B, 1, D), self.sin_b[pos].view(B, 1, D)
        q = rope(p["q"](n1).view(B, H, 1, D), cos, sin)
        k = rope(p["k"](n1).view(B, Hkv, 1, D), cos, sin)
        self.kbuf[:, :, pos:pos + 1].copy_(k)
        self.vbuf[:, :, pos:pos + 1].copy_(p["v"](n1).view(B, Hkv, 1, D))
        attn = decode_attention(q.view(B, H, D), self.kbuf, self.vbuf, self.scale, pos + 1)
        h = x + p["o"](attn.view(B, H * D))
        n2 = rmsnorm(h, self.ln2, self.eps)
        return h + p["down"](silu_mul(p["gate"](n2), p["up"](n2)))

    def step_parts(self, x: torch.Tensor, pos: int,
                   residual: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
        """The merged step without its last residual add: returns (h, mlp)
        with step(x, pos) == h + mlp. With `residual`, the layer's input is
        x + residual, added by the first RMSNorm's launch (add_rmsnorm), so
        a stack of layers hands (h, mlp) on without a separate add."""
        if not self.fused:
            raise RuntimeError("step_parts needs a layer built with fused=True")
        if not 0 <= pos < self.max_len:
            raise RuntimeError(f"position {pos} outside the cache (max_len {self.max_len})")
        B, H, D = self.batch, self.n_heads, self.head_dim
        p = self.proj
        if residual is None:
            n1 = rmsnorm(x, self.ln1, self.eps)
        else:
            x, n1 = add_rmsnorm(x, residual, self.ln1, self.eps)
        if self.qkv_rope:
            q = p["qkv"].qkv_rope(n1, self.cos[pos], self.sin[pos], self.kbuf, self.vbuf, pos, H)
        else:
            q = rope_qkv_append(p["qkv"](n1), self.cos[pos], self.sin[pos], self.kbuf, self.vbuf, pos)
        attn = decode_attention(q, self.kbuf, self.vbuf, self.scale, pos + 1)
        h, n2 = add_rmsnorm(x, p["o"](attn.view(B, H * D)), self.ln2, self.eps)
        act = p["gate_up"].swiglu(n2) if self.swiglu else silu_mul_halves(p["gate_up"](n2))
        return h, p["down"](act)

    def capture(self, x: torch.Tensor, pos: int, warmup: int = 2) -> Tuple[torch.cuda.CUDAGraph, torch.Tensor]:
        """Record `step(x, pos)` in a CUDA (HIP) graph. Returns the graph and
        its output tensor; `graph.replay()` reruns the step on whatever `x`
        holds then. Every capture of this layer runs on the layer's own
        capture stream, whose split-K workspace the warm-up steps set up
        before the first capture; all of the layer's graphs share that
        workspace, so their replays must not overlap (replay them on one
        stream, or order them)."""
        self._capture_stream = _capture_stream(self, x.device)
        return _capture(self.step, x, pos, warmup, self._capture_stream)


class DecodeStack:
    """Merged-step layers run in sequence for one token. Layer i's last
    residual add goes into layer i + 1's first RMSNorm launch
    (`step_parts(..., residual=)`), so n layers make 7 n + 1 launches (one
    more per layer for each merged projection that does not apply); the
    output equals chaining `layer.step` bit for bit (the merged norm rounds
    x + residual exactly as the add it replaces)."""

    def __init__(self, layers) -> None:
        self.layers = list(layers)
        if not self.layers or not all(layer.fused for layer in self.layers):
            raise RuntimeError("DecodeStack needs one or more layers built with fused=True")

    def step(self, x: torch.Tensor, pos: int) -> torch.Tensor:
        h, r = x, None
        for layer in self.layers:
            h, r = layer.step_parts(h, pos, r)
        return h + r

    def capture(self, x: torch.Tensor, pos: int, warmup: int = 2) -> Tuple[torch.cuda.CUDAGraph, torch.Tensor]:
        """As DecodeLayer.capture, for the whole stack (one capture stream
        per stack)."""
        self._capture_stream = _capture_stream(self, x.device)
        return _capture(self.step, x, pos, warmup, self._capture_stream)


def _capture_stream(module, device: torch.device) -> torch.cuda.Stream:
    """The module's capture stream, created on its first capture. The ops
    cache their split-K workspace per stream, so graphs captured on one
    stream share it. torch hands out streams from a pool of 32 per device,
    so modules beyond that may share a stream handle; graphs whose capture
    streams share a handle must likewise be replayed in one stream order."""
    s = getattr(module, "_capture_stream", None)
    if s is None or s.device != device:
        s = torch.cuda.Stream(device=device)
    return s


def _capture(step, x: torch.Tensor, pos: int, warmup: int,
             stream: torch.cuda.Stream) -> Tuple[torch.cuda.CUDAGraph, torch.Tensor]:
    stream.wait_stream(torch.cuda.current_stream(x.device))
    with torch.cuda.stream(stream):
        for _ in range(warmup):
            step(x, pos)
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        out = step(x, pos)
    return graph, out
