"""CPU: the torch restatements that bench.py times as the host baseline
(oracle/torch_ref.py) agree with the pinned numpy oracle: attention within
fp32 rounding before the cast and bit for bit after it on these inputs up to
one fp16 ulp, the quantisers bit for bit, the W4A16 reference matmul within
one fp16 ulp."""
from __future__ import annotations

import math

import numpy as np
import torch

from oracle import attention as oa
from oracle import kv_quant as kq
from oracle import torch_ref as tr
from oracle import w4a16 as ow
from tests.helpers import kv_with_outliers, randn


def _ulps_f16(a: np.ndarray, b: np.ndarray) -> int:
    ia = a.astype(np.float16).view(np.int16).astype(np.int32)
    ib = b.astype(np.float16).view(np.int16).astype(np.int32)
    return int(np.abs(ia - ib).max())


def test_attention_matches_numpy_oracle():
    q = randn((2, 32, 128), 1).astype(np.float16)
    k = randn((2, 8, 300, 128), 2).astype(np.float16)
    v = randn((2, 8, 300, 128), 3).astype(np.float16)
    got = tr.eager_decode_attention(torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v),
                                    1 / math.sqrt(128))
    assert got.dtype == torch.float16 and got.shape == (2, 32, 128)
    ref = oa.decode_attention(q, k, v, 1 / math.sqrt(128), acc_dtype=np.float64)
    assert float(np.abs(got.double().numpy() - ref).max()) <= 1e-3
    assert _ulps_f16(got.numpy(), ref) <= 1


def test_attention_gqa_is_repeat_interleave():
    """A wrong head mapping (kv head h % Hkv instead of h // G) is caught."""
    q = randn((1, 8, 128), 4).astype(np.float16)
    k = randn((1, 2, 50, 128), 5).astype(np.float16)
    v = randn((1, 2, 50, 128), 6).astype(np.float16)
    got = tr.eager_decode_attention(torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v))
    wrong = oa.decode_attention_expanded(q, np.tile(k, (1, 4, 1, 1)), np.tile(v, (1, 4, 1, 1)))
    right = oa.decode_attention_expanded(q, np.repeat(k, 4, axis=1), np.repeat(v, 4, axis=1))
    assert float(np.abs(got.float().numpy() - right).max()) <= 2e-3
    assert float(np.abs(got.float().numpy() - wrong).max()) > 1e-2


def test_quantisers_match_numpy_oracle_bit_for_bit():
    x = kv_with_outliers((2, 8, 200, 128), 7).astype(np.float16).astype(np.float32)
    for bits in (8, 4):
        q, s = tr.quantize_per_token(torch.from_numpy(x), bits)
        rq, rs = kq.quantize_per_token(x, bits)
        assert np.array_equal(q.numpy(), rq) and np.array_equal(s.numpy(), rs)
    for gs in (32, 128):
        q, s = tr.quantize_per_channel_groupwise(torch.from_numpy(x), 4, gs)
        rq, rs = kq.quantize_per_channel_groupwise(x, 4, gs)
        assert np.array_equal(q.numpy(), rq) and np.array_equal(s.numpy(), rs)


def test_quantized_matmul_matches_numpy_oracle():
    W = randn((512, 256), 8, scale=0.02)
    q, s = ow.quantize_weights_int4_groupwise(W, 128)
    s = s.astype(np.float16)
    act = randn((3, 512), 9).astype(np.float16)
    got = tr.quantized_matmul_ref(torch.from_numpy(act), torch.from_numpy(q), torch.from_numpy(s), 128)
    ref = ow.quantized_matmul_ref(act, q, s, 128, acc_dtype=np.float64)
    assert got.dtype == torch.float16
    assert _ulps_f16(got.numpy(), ref) <= 1


def test_host_threads_respects_affinity():
    import os
    n = tr.host_threads()
    assert 1 <= n <= len(os.sched_getaffinity(0))
