"""W4A16 group-wise INT4 weight quantisation, packing and matmul (test
infrastructure; see oracle/__init__.py).

Restates reference/quant_matmul_ref.py:
  quantize_weights_int4_groupwise   (:39-88)  dtype semantics as in
                                    oracle/kv_quant.py: for fp16 W the scale
                                    is rounded to fp16 before the codes
  dequantize_weights_int4_groupwise (:91-109)
  quantized_matmul_ref              (:112-135) fp32 act @ fp32 W_hat
  pack_int4_along_k                 (:140-165) [K, N] -> [K/8, N] int32,
                                    bits 4i..4i+3 = K position 8*k_pack + i
and the dequantise kernel's output convention fp16(code * scale)
(kernels/quant/quant_matmul.cu:612-627).
"""
from __future__ import annotations

from typing import Tuple

import numpy as np

QMAX_INT4 = 7


def quantize_weights_int4_groupwise(W: np.ndarray, group_size: int = 128
                                    ) -> Tuple[np.ndarray, np.ndarray]:
    """W [K, N] fp16/fp32 -> (q int8 [K, N] in [-7, 7], scale [ceil(K/g), N] in W.dtype)."""
    K, N = W.shape
    ng = (K + group_size - 1) // group_size
    pad = ng * group_size - K
    Wp = np.concatenate([W, np.zeros((pad, N), dtype=W.dtype)], axis=0) if pad else W
    Wg = Wp.reshape(ng, group_size, N)
    absmax = np.abs(Wg).max(axis=1)
    scale = (absmax / W.dtype.type(QMAX_INT4)).astype(W.dtype)
    scale = np.maximum(scale, scale.dtype.type(1e-8))
    with np.errstate(invalid="ignore", divide="ignore"):
        qf = np.rint(Wg.astype(np.float32) / scale.astype(np.float32)[:, None, :])
    qf = np.clip(qf, -QMAX_INT4, QMAX_INT4)
    qf = np.where(np.isnan(qf), 0.0, qf)
    q = qf.astype(np.int8).reshape(ng * group_size, N)[:K]
    return q, scale.astype(W.dtype)


def dequantize_weights_int4_groupwise(q: np.ndarray, scale: np.ndarray, group_size: int
                                      ) -> np.ndarray:
    """fp32 W_hat[k, n] = q[k, n] * scale[k // g, n]."""
    idx = np.arange(q.shape[0]) // group_size
    return q.astype(np.float32) * scale.astype(np.float32)[idx, :]


def quantized_matmul_ref(act: np.ndarray, q: np.ndarray, scale: np.ndarray, group_size: int,
                         acc_dtype=np.float32) -> np.ndarray:
    """act [M, K] @ W_hat [K, N] accumulated in acc_dtype, not cast back
    (the reference casts to act.dtype at quant_matmul_ref.py:135)."""
    w_hat = dequantize_weights_int4_groupwise(q, scale, group_size).astype(acc_dtype)
    return act.astype(acc_dtype) @ w_hat


def pack_int4_along_k(q: np.ndarray) -> np.ndarray:
    """[K, N] int8 -> [K/8, N] int32 (quant_matmul_ref.py:140-165)."""
    K, N = q.shape
    assert K % 8 == 0, K
    g = (q.reshape(K // 8, 8, N).astype(np.int64) & 0xF)
    packed = np.zeros((K // 8, N), dtype=np.int64)
    for i in range(8):
        packed |= g[:, i, :] << (4 * i)
    return packed.astype(np.uint32).view(np.int32)


def unpack_int4_along_k(packed: np.ndarray) -> np.ndarray:
    """[K/8, N] int32 -> [K, N] int8 via the kernel's sign-extending shift
    `(w << (28 - 4i)) >> 28` (kernels/quant/quant_matmul.cu:66)."""
    kp, N = packed.shape
    w = packed.astype(np.int32)
    out = np.empty((kp, 8, N), dtype=np.int8)
    for i in range(8):
        out[:, i, :] = ((w << np.int32(28 - 4 * i)) >> np.int32(28)).astype(np.int8)
    return out.reshape(kp * 8, N)


def w4a16_dequantize_fp16(packed: np.ndarray, scale: np.ndarray, group_size: int) -> np.ndarray:
    """fp16 W [K, N] = fp16(code * scale[k // g]) (the code * fp16-scale product
    is exact in fp32, so this is one round-to-nearest-even)."""
    q = unpack_int4_along_k(packed)
    idx = np.arange(q.shape[0]) // group_size
    return (q.astype(np.float32) * scale.astype(np.float32)[idx, :]).astype(np.float16)
