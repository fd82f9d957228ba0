"""Fused decode-path elementwise ops (test infrastructure; see
oracle/__init__.py).

The reference has no Python oracle for these; its CUDA kernels
(kernels/fused/fused_ops.cu:31-86) define them and its tests compare to the
PyTorch formulas in tests/test_fused.py:54-62. Restated here in fp32 with
one fp16 rounding per output, as the kernels compute them.
"""
from __future__ import annotations

import numpy as np


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """fp32 x * rsqrt(mean(x^2) + eps) * w (fused_ops.cu:31-52), not rounded."""
    xf = x.astype(np.float32)
    var = (xf.astype(np.float64) ** 2).mean(axis=-1, keepdims=True)
    inv = (1.0 / np.sqrt(var + eps)).astype(np.float32)
    return xf * inv * w.astype(np.float32)


def rmsnorm_hf(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """The reference test's formula w * fp16(x * rsqrt(var + eps))
    (tests/test_fused.py:54-57)."""
    xf = x.astype(np.float32)
    var = (xf ** 2).mean(axis=-1, keepdims=True)
    y = (xf / np.sqrt(var + np.float32(eps))).astype(np.float16)
    return (w.astype(np.float16) * y).astype(np.float16)


def silu_mul(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    """silu(g) * u in fp32 (fused_ops.cu:55-63), not rounded."""
    gf = g.astype(np.float32)
    return gf / (1.0 + np.exp(-gf)) * u.astype(np.float32)


def rotate_half(x: np.ndarray) -> np.ndarray:
    h = x.shape[-1] // 2
    return np.concatenate([-x[..., h:], x[..., :h]], axis=-1)


def rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """x [B,H,S,D] * cos + rotate_half(x) * sin with cos/sin [B,S,D]
    broadcast over heads (fused_ops.cu:68-86), fp32, not rounded."""
    xf = x.astype(np.float32)
    c = cos.astype(np.float32)[:, None]
    s = sin.astype(np.float32)[:, None]
    return xf * c + rotate_half(xf) * s
