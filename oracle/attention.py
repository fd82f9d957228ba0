"""Eager GQA decode attention (test infrastructure; see oracle/__init__.py).

Restates reference/attention_ref.py:
  _expand_gqa       (:15-40)  repeat each kv head n_heads/n_kv_heads times
                              (repeat_interleave along the head axis)
  eager_attention   (:43-80)  scores = (q @ k^T) * scale in fp32, softmax,
                              probs @ v, result cast to q.dtype
  decode_attention  (:108-123) one query token per sequence

`decode_attention` evaluates the same sums batch by batch with the query
heads of a kv head grouped against that kv head, instead of materialising
the expanded cache; `decode_attention_expanded` is the literal
repeat_interleave form, and the tests pin the two against each other.
"""
from __future__ import annotations

import math
from typing import Optional

import numpy as np


def expand_gqa(k: np.ndarray, n_heads: int) -> np.ndarray:
    """[B, Hkv, S, D] -> [B, n_heads, S, D] (attention_ref.py:15-40)."""
    n_kv = k.shape[1]
    if n_kv == n_heads:
        return k
    return np.repeat(k, n_heads // n_kv, axis=1)


def _softmax_rows(scores: np.ndarray) -> np.ndarray:
    m = scores.max(axis=-1, keepdims=True)
    e = np.exp(scores - m)
    return e / e.sum(axis=-1, keepdims=True)


def decode_attention_expanded(q: np.ndarray, k: np.ndarray, v: np.ndarray,
                              scale: Optional[float] = None, acc_dtype=np.float32) -> np.ndarray:
    """Literal attention_ref.py:65-80 with q_len == 1, not cast back."""
    B, H, D = q.shape
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    kk = expand_gqa(k.astype(acc_dtype), H)
    vv = expand_gqa(v.astype(acc_dtype), H)
    qq = q.astype(acc_dtype)[:, :, None, :]
    scores = np.matmul(qq, np.swapaxes(kk, -1, -2)) * acc_dtype(scale)     # [B, H, 1, S]
    return np.matmul(_softmax_rows(scores), vv)[:, :, 0, :].astype(acc_dtype)


def decode_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray,
                     scale: Optional[float] = None, seqlen: Optional[int] = None,
                     acc_dtype=np.float32) -> np.ndarray:
    """One-token GQA decode attention computed in `acc_dtype`, not cast back.

    q [B, H, D]; k, v [B, Hkv, L, D] (any float dtype, or int codes already
    dequantised by the caller). Only the first `seqlen` positions are
    attended (default: all L). Returns [B, H, D] in acc_dtype; the
    reference's `.to(q.dtype)` (attention_ref.py:80) is left to the caller
    so the unrounded value can be the parity target. An empty cache gives
    zeros, as torch's softmax over an empty axis followed by matmul does.
    """
    B, H, D = q.shape
    Hkv = k.shape[1]
    G = H // Hkv
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    S = k.shape[2] if seqlen is None else seqlen
    out = np.zeros((B, H, D), dtype=acc_dtype)
    if S == 0:
        return out
    sc = acc_dtype(scale)
    for b in range(B):
        kb = k[b, :, :S].astype(acc_dtype)                          # [Hkv, S, D]
        vb = v[b, :, :S].astype(acc_dtype)
        qb = q[b].astype(acc_dtype).reshape(Hkv, G, D)              # heads h = kv*G + g
        scores = np.matmul(qb, np.swapaxes(kb, -1, -2)) * sc        # [Hkv, G, S]
        out[b] = np.matmul(_softmax_rows(scores), vb).reshape(H, D)
    return out
