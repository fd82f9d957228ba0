"""GPU parity: quantize-on-append KV writers, bit-exact codes, packing and
fp16 scales vs the oracle applied to x.float() (the reference tests' call
convention, tests/test_kv_cache.py:234,333,360)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kv_quant as kq
from tests.helpers import GOLDEN, kv_with_outliers

pytestmark = pytest.mark.gpu

GOLD = np.load(GOLDEN / "kv_quant_golden.npz")


def _dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _bits_equal(t: torch.Tensor, a: np.ndarray) -> bool:
    got = t.cpu().numpy()
    return got.shape == a.shape and np.array_equal(got.view(np.uint8), a.view(np.uint8))


def _special(x: np.ndarray) -> np.ndarray:
    x = x.copy()
    x[0, 0, 0] = 0.0
    x[0, 0, min(1, x.shape[2] - 1)] *= np.float16(1e-4)
    return x


SHAPES = [(1, 8, 1, 128), (2, 8, 17, 128), (1, 8, 128, 128), (4, 8, 1000, 128), (8, 8, 4096, 128)]


@pytest.mark.parametrize("shape", SHAPES)
def test_int8_per_token_bit_exact(llmik, cuda, shape):
    x = _special(kv_with_outliers(shape, seed=shape[2]).astype(np.float16))
    q, s = llmik.quantize_per_token(_dev(x, cuda))
    rq, rs = kq.quantize_per_token(x.astype(np.float32), 8)
    assert q.dtype == torch.int8 and s.dtype == torch.float16
    assert _bits_equal(q, rq)
    assert _bits_equal(s, rs.astype(np.float16))


@pytest.mark.parametrize("shape", SHAPES)
def test_int4_v_per_token_bit_exact(llmik, cuda, shape):
    x = _special(kv_with_outliers(shape, seed=shape[2] + 1).astype(np.float16))
    q, s = llmik.quantize_v_per_token_int4(_dev(x, cuda))
    rq, rs = kq.quantize_per_token(x.astype(np.float32), 4)
    assert q.shape == (*shape[:3], 64)
    assert _bits_equal(q, kq.pack_kv_int4(rq))
    assert _bits_equal(s, rs.astype(np.float16))


@pytest.mark.parametrize("shape", SHAPES + [(2, 8, 100, 128), (1, 2, 37, 128)])
@pytest.mark.parametrize("gs", [32, 128, 64])
def test_int4_k_groupwise_bit_exact(llmik, cuda, shape, gs):
    _check_k_groupwise(llmik, cuda, shape, gs)


# Group sizes that take the other register-resident widths (<= 16 tokens,
# a group that does not fill its rows) and the two-pass path (> 128).
@pytest.mark.parametrize("shape,gs", [((1, 8, 100, 128), 8), ((2, 4, 70, 128), 16),
                                      ((1, 8, 300, 128), 96), ((2, 8, 600, 128), 256),
                                      ((1, 2, 37, 128), 512)])
def test_int4_k_groupwise_other_group_sizes(llmik, cuda, shape, gs):
    _check_k_groupwise(llmik, cuda, shape, gs)


def _check_k_groupwise(llmik, cuda, shape, gs):
    x = _special(kv_with_outliers(shape, seed=shape[2] + gs).astype(np.float16))
    q, s = llmik.quantize_k_per_channel_groupwise_int4(_dev(x, cuda), gs)
    rq, rs = kq.quantize_per_channel_groupwise(x.astype(np.float32), 4, gs)
    assert s.shape == (*shape[:2], (shape[2] + gs - 1) // gs, 128)
    assert _bits_equal(q, kq.pack_kv_int4(rq))
    assert _bits_equal(s, rs.astype(np.float16))


def test_golden_inputs_bit_exact(llmik, cuda):
    """The golden rows (zeros, subnormal scales, exact ties, near-tie rows
    that separate true division from reciprocal multiplication), rounded to
    fp16 as the kernels take them."""
    x16 = GOLD["pt_x32"].astype(np.float16)
    xd = _dev(x16, cuda)
    q8, s8 = llmik.quantize_per_token(xd)
    rq8, rs8 = kq.quantize_per_token(x16.astype(np.float32), 8)
    assert _bits_equal(q8, rq8) and _bits_equal(s8, rs8.astype(np.float16))
    q4, s4 = llmik.quantize_v_per_token_int4(xd)
    rq4, rs4 = kq.quantize_per_token(x16.astype(np.float32), 4)
    assert _bits_equal(q4, kq.pack_kv_int4(rq4)) and _bits_equal(s4, rs4.astype(np.float16))
    g16 = GOLD["gw_x32"].astype(np.float16)
    for gs in (32, 128):
        qk, sk = llmik.quantize_k_per_channel_groupwise_int4(_dev(g16, cuda), gs)
        rqk, rsk = kq.quantize_per_channel_groupwise(g16.astype(np.float32), 4, gs)
        assert _bits_equal(qk, kq.pack_kv_int4(rqk)) and _bits_equal(sk, rsk.astype(np.float16))


def test_fp32_golden_rows_at_fp16_exact_values(llmik, cuda):
    """Near-tie rows built in fp32 lose their tie when rounded to fp16; build
    fp16-exact near-ties directly: x = fp16 values whose fp32 quotient by an
    fp32 scale lands within an ulp of a half-integer."""
    rng = np.random.default_rng(11)
    rows = []
    while len(rows) < 64:
        amax = np.float16(rng.uniform(0.5, 8.0))
        s = np.float32(np.float32(amax) / np.float32(127))
        r = np.float32(np.float32(1.0) / s)
        row = np.zeros(128, dtype=np.float16)
        row[0] = amax
        n = 1
        for k in rng.integers(-126, 126, size=4000):
            if n == 128:
                break
            c = np.float16((k + 0.5) * float(s))
            for cand in (c, np.nextafter(c, np.float16(np.inf)), np.nextafter(c, np.float16(-np.inf))):
                cf = np.float32(cand)
                if abs(cf) < np.float32(amax) and np.rint(cf / s) != np.rint(np.float32(cf * r)):
                    row[n] = cand
                    n += 1
                    break
        rows.append(row)
    x = np.stack(rows).reshape(1, 1, 64, 128)
    q, s_ = llmik.quantize_per_token(_dev(x, cuda))
    rq, rs = kq.quantize_per_token(x.astype(np.float32), 8)
    assert _bits_equal(q, rq) and _bits_equal(s_, rs.astype(np.float16))
