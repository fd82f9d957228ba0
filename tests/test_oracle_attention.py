"""Pins for oracle/attention.py (CPU): float64 brute force with explicit
loops on tiny shapes, closed forms, and the invariants the math fixes.

A plausible mistake — a dropped scale, softmax over the wrong axis, a wrong
head-to-kv-head map (h % Hkv instead of h // G), a transposed operand —
fails at least one of these.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import attention as oa
from tests.helpers import randn


def brute_force(q, k, v, scale):
    """Scalar-loop float64 attention: out[b,h] = sum_t p_t v_t."""
    B, H, D = q.shape
    Hkv, S = k.shape[1], k.shape[2]
    G = H // Hkv
    out = np.zeros((B, H, D))
    for b in range(B):
        for h in range(H):
            kvh = h // G
            s = [scale * sum(float(q[b, h, d]) * float(k[b, kvh, t, d]) for d in range(D))
                 for t in range(S)]
            m = max(s)
            w = [math.exp(x - m) for x in s]
            z = sum(w)
            for d in range(D):
                out[b, h, d] = sum(w[t] * float(v[b, kvh, t, d]) for t in range(S)) / z
    return out


@pytest.mark.parametrize("B,H,Hkv,S,D", [(1, 4, 2, 5, 8), (2, 6, 3, 7, 4), (1, 2, 2, 3, 16)])
def test_matches_float64_brute_force(B, H, Hkv, S, D):
    q, k, v = randn((B, H, D), 1), randn((B, Hkv, S, D), 2), randn((B, Hkv, S, D), 3)
    scale = 1.0 / math.sqrt(D)
    ref = brute_force(q, k, v, scale)
    assert np.abs(oa.decode_attention(q, k, v, scale, acc_dtype=np.float64) - ref).max() < 1e-12
    assert np.abs(oa.decode_attention(q, k, v, scale) - ref).max() < 1e-5


def test_grouped_equals_repeat_interleave_form():
    q, k, v = randn((2, 32, 128), 4), randn((2, 8, 300, 128), 5), randn((2, 8, 300, 128), 6)
    a = oa.decode_attention(q, k, v, acc_dtype=np.float64)
    b = oa.decode_attention_expanded(q, k, v, acc_dtype=np.float64)
    assert np.abs(a - b).max() < 1e-12


def test_single_token_returns_its_value():
    q, k, v = randn((1, 8, 128), 7), randn((1, 2, 1, 128), 8), randn((1, 2, 1, 128), 9)
    out = oa.decode_attention(q, k, v, acc_dtype=np.float64)
    for h in range(8):
        assert np.allclose(out[0, h], v[0, h // 4, 0], atol=1e-12)


def test_constant_keys_give_mean_of_values():
    k = np.ones((1, 1, 50, 16), dtype=np.float32)
    v = randn((1, 1, 50, 16), 10)
    q = randn((1, 3, 16), 11)
    out = oa.decode_attention(q, k, v, acc_dtype=np.float64)
    assert np.allclose(out[0], v[0, 0].mean(axis=0), atol=1e-12)


def test_dominant_score_selects_its_row():
    D = 16
    k = np.zeros((1, 1, 9, D), dtype=np.float32)
    k[0, 0, 4, 0] = 1000.0
    q = np.zeros((1, 1, D), dtype=np.float32)
    q[0, 0, 0] = 1.0
    v = randn((1, 1, 9, D), 12)
    out = oa.decode_attention(q, k, v, scale=1.0, acc_dtype=np.float64)
    assert np.allclose(out[0, 0], v[0, 0, 4], atol=1e-12)


def test_token_permutation_invariance_and_convexity():
    q, k, v = randn((1, 4, 32), 13), randn((1, 1, 64, 32), 14), randn((1, 1, 64, 32), 15)
    perm = np.random.default_rng(0).permutation(64)
    a = oa.decode_attention(q, k, v, acc_dtype=np.float64)
    b = oa.decode_attention(q, k[:, :, perm], v[:, :, perm], acc_dtype=np.float64)
    assert np.abs(a - b).max() < 1e-12
    assert (a <= v.max(axis=2)[:, :, None, :].max(axis=1) + 1e-12).all()
    assert (a >= v.min(axis=2)[:, :, None, :].min(axis=1) - 1e-12).all()


def test_seqlen_prefix_and_empty():
    q, k, v = randn((1, 4, 16), 16), randn((1, 2, 40, 16), 17), randn((1, 2, 40, 16), 18)
    a = oa.decode_attention(q, k, v, seqlen=25, acc_dtype=np.float64)
    b = oa.decode_attention(q, k[:, :, :25], v[:, :, :25], acc_dtype=np.float64)
    assert np.array_equal(a, b)
    assert not np.any(oa.decode_attention(q, k, v, seqlen=0))


def test_planted_wrong_head_map_is_caught():
    q, k, v = randn((1, 4, 8), 19), randn((1, 2, 6, 8), 20), randn((1, 2, 6, 8), 21)
    ref = brute_force(q, k, v, 1 / math.sqrt(8))
    # a mistaken oracle mapping head h to kv head h % Hkv
    wrong = np.stack([oa.decode_attention(q[:, h:h + 1], k[:, h % 2:h % 2 + 1],
                                          v[:, h % 2:h % 2 + 1], acc_dtype=np.float64)[:, 0]
                      for h in range(4)], axis=1)
    assert np.abs(wrong - ref).max() > 1e-3
