"""Symmetric KV-cache quantisers and INT4 packing (test infrastructure; see
oracle/__init__.py).

Restates reference/kv_cache_ref.py with torch's dtype semantics:
  _qmax                            (:32-43)
  quantize_per_token               (:46-62)
  dequantize_per_token             (:65-70)
  quantize_per_channel_groupwise   (:73-112)
  dequantize_per_channel_groupwise (:115-129)
  kivi / int8 presets              (:136-180)

dtype semantics (torch CPU, confirmed by the golden vectors): absmax, the
division by qmax and the clamp run in x's dtype — for fp16 input the scale
is rounded to fp16 BEFORE the codes are computed, and clamp(min=1e-8)
rounds its bound to fp16 (0), so it never lifts a scale. The codes are
round_half_even(fp32(x) / fp32(scale)) clamped to +-qmax; a NaN quotient
(an all-zero row in fp16) converts to code 0 as torch does on x86. The
KV kernels of this build follow the fp32 convention (the reference tests
call the oracle on x.float(), tests/test_kv_cache.py:234,333,360).

INT4 packing is the reference CUDA writers' storage format
(kernels/kv_cache/kv_compress.cuh:25-28, kv_compress.cu:150-155): byte i of
a token row holds channel 2i in the low nibble and channel 2i+1 in the high
nibble, two's complement; tests/test_kv_cache.py:295-314 is its inverse.
"""
from __future__ import annotations

from typing import Tuple

import numpy as np


def qmax(bits: int) -> int:
    """2^(bits-1) - 1 (kv_cache_ref.py:32-43)."""
    assert bits in (4, 8), bits
    return (1 << (bits - 1)) - 1


def _to_int8(qf: np.ndarray) -> np.ndarray:
    qf = np.where(np.isnan(qf), 0.0, qf)
    return qf.astype(np.int8)


def _clamp_scale(scale: np.ndarray) -> np.ndarray:
    # torch: (absmax / qmax).clamp(min=1e-8) in the tensor's dtype.
    return np.maximum(scale, scale.dtype.type(1e-8))


def quantize_per_token(x: np.ndarray, bits: int) -> Tuple[np.ndarray, np.ndarray]:
    """x [B, Hkv, S, D] -> (q int8 [B, Hkv, S, D], scale [B, Hkv, S] in x.dtype)."""
    qm = qmax(bits)
    absmax = np.abs(x).max(axis=-1, keepdims=True)
    scale = _clamp_scale((absmax / x.dtype.type(qm)).astype(x.dtype))
    with np.errstate(invalid="ignore", divide="ignore"):
        qf = np.rint(x.astype(np.float32) / scale.astype(np.float32))
    qf = np.clip(qf, -qm, qm)
    return _to_int8(qf), scale[..., 0].astype(x.dtype)


def dequantize_per_token(q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """fp32 q * scale (kv_cache_ref.py:65-70)."""
    return q.astype(np.float32) * scale.astype(np.float32)[..., None]


def quantize_per_channel_groupwise(x: np.ndarray, bits: int, group_size: int
                                   ) -> Tuple[np.ndarray, np.ndarray]:
    """x [B, Hkv, S, D] -> (q int8 [B, Hkv, S, D],
    scale [B, Hkv, ceil(S/g), D] in x.dtype). Zero padding of the short last
    group does not change its absmax (kv_cache_ref.py:94-106)."""
    qm = qmax(bits)
    B, H, S, D = x.shape
    ng = (S + group_size - 1) // group_size
    pad = ng * group_size - S
    xp = np.concatenate([x, np.zeros((B, H, pad, D), dtype=x.dtype)], axis=2) if pad else x
    xg = xp.reshape(B, H, ng, group_size, D)
    absmax = np.abs(xg).max(axis=3)
    scale = _clamp_scale((absmax / x.dtype.type(qm)).astype(x.dtype))
    with np.errstate(invalid="ignore", divide="ignore"):
        qf = np.rint(xg.astype(np.float32) / scale.astype(np.float32)[:, :, :, None, :])
    qf = np.clip(qf, -qm, qm)
    q = _to_int8(qf).reshape(B, H, ng * group_size, D)[:, :, :S, :]
    return q, scale.astype(x.dtype)


def dequantize_per_channel_groupwise(q: np.ndarray, scale: np.ndarray, group_size: int
                                     ) -> np.ndarray:
    """fp32 q * scale[token // group_size] (kv_cache_ref.py:115-129)."""
    S = q.shape[2]
    idx = np.arange(S) // group_size
    return q.astype(np.float32) * scale.astype(np.float32)[:, :, idx, :]


def pack_kv_int4(q: np.ndarray) -> np.ndarray:
    """[..., D] int8 codes in [-8, 7] -> [..., D/2] int8 packed bytes."""
    lo = q[..., 0::2].astype(np.int32) & 0xF
    hi = q[..., 1::2].astype(np.int32) & 0xF
    return (lo | (hi << 4)).astype(np.uint8).view(np.int8)


def unpack_kv_int4(packed: np.ndarray) -> np.ndarray:
    """Inverse of pack_kv_int4 (tests/test_kv_cache.py:295-314)."""
    p = packed.view(np.uint8).astype(np.int32)
    lo = ((p & 0x0F) << 4).astype(np.uint8).view(np.int8) >> 4
    hi = (p & 0xF0).astype(np.uint8).view(np.int8) >> 4
    out = np.stack([lo, hi], axis=-1).reshape(*packed.shape[:-1], 2 * packed.shape[-1])
    return out.astype(np.int8)


def quantize_kv_int8_per_token(k: np.ndarray, v: np.ndarray):
    """INT8 preset (kv_cache_ref.py:136-145)."""
    return (*quantize_per_token(k, 8), *quantize_per_token(v, 8))


def quantize_kv_kivi_int4(k: np.ndarray, v: np.ndarray, group_size: int = 32):
    """KIVI preset (kv_cache_ref.py:158-169): K per channel groupwise, V per token."""
    return (*quantize_per_channel_groupwise(k, 4, group_size), *quantize_per_token(v, 4))
