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


def _bits_equal_nan(t: torch.Tensor, a: np.ndarray) -> bool:
    """Bit-exact, except that a NaN matches any NaN (torch's own NaN payload
    depends on its reduction path, so it is no pin)."""
    got = t.cpu().numpy()
    if got.shape != a.shape or got.dtype != a.dtype:
        return False
    ng, na = np.isnan(got), np.isnan(a)
    return bool((ng == na).all()) and np.array_equal(got[~ng].view(np.uint8), a[~na].view(np.uint8))


def _nonfinite16(key: str) -> np.ndarray:
    with np.errstate(over="ignore"):
        return GOLD[key].astype(np.float16)


def test_nonfinite_golden_rows(llmik, cuda):
    """Rows holding NaN, +-inf and fp16 overflow, against the reference's
    own quantisers on x.float() (tests/golden, kv_cache_ref.py:59-61): a row
    (or group channel) with a NaN stores scale NaN and codes 0, one with an
    inf stores +inf and codes 0, and every other row is unchanged."""
    x16 = _nonfinite16("nf_pt_x32")
    xd = _dev(x16, cuda)
    q8, s8 = llmik.quantize_per_token(xd)
    assert _bits_equal(q8, GOLD["nf_pt_x16f_b8_q"])
    assert _bits_equal_nan(s8, GOLD["nf_pt_x16f_b8_s"].astype(np.float16))
    q4, s4 = llmik.quantize_v_per_token_int4(xd)
    assert _bits_equal(q4, kq.pack_kv_int4(GOLD["nf_pt_x16f_b4_q"]))
    assert _bits_equal_nan(s4, GOLD["nf_pt_x16f_b4_s"].astype(np.float16))
    assert torch.isnan(s8[0, 0, 3]) and torch.isinf(s8[0, 0, 1]) and not q8[0, 0, :6].any()
    g16 = _dev(_nonfinite16("nf_gw_x32"), cuda)
    for gs in (32, 128):
        qk, sk = llmik.quantize_k_per_channel_groupwise_int4(g16, gs)
        assert _bits_equal(qk, kq.pack_kv_int4(GOLD[f"nf_gw_x16f_b4_g{gs}_q"]))
        assert _bits_equal_nan(sk, GOLD[f"nf_gw_x16f_b4_g{gs}_s"].astype(np.float16))
    # The in-place forms (mapped token positions) and the one-launch KIVI
    # append share the arithmetic; check them on the same rows.
    qc = torch.full((1, 2, 12, 128), 0x5A, dtype=torch.int8, device=cuda)
    sc = torch.full((1, 2, 12), 1234.0, dtype=torch.float16, device=cuda)
    llmik.quantize_per_token_into(xd, qc, sc, 3)
    assert torch.equal(qc[:, :, 3:11], q8)
    assert torch.equal(torch.isnan(sc[:, :, 3:11]), torch.isnan(s8))
    assert torch.equal(torch.nan_to_num(sc[:, :, 3:11]).view(torch.int16),
                       torch.nan_to_num(s8).view(torch.int16))


def test_nonfinite_kivi_append(llmik, cuda):
    """Single-token appends through Int4KIVICache's one-launch path, where
    the open K group and the V token hold NaN and inf: the cache holds what
    the oracle quantisers give for the same fp16 tokens."""
    from llmik_cuda.kv_cache import Int4KIVICache
    g = 32
    k_all = _nonfinite16("nf_gw_x32")[:, :, :40]          # NaN at token 5, inf at token 10/11
    v_all = np.concatenate([_nonfinite16("nf_pt_x32")] * 5, axis=2)   # 40 tokens
    cache = Int4KIVICache(1, 2, max_len=64, group_size=g, device=cuda)
    for t in range(40):
        cache.append(_dev(k_all[:, :, t:t + 1], cuda), _dev(v_all[:, :, t:t + 1], cuda))
    k_q, k_s, v_q, v_s, L = cache.get_quantized_for_attention()
    rq0, rs0 = kq.quantize_per_channel_groupwise(k_all[:, :, :32].astype(np.float32), 4, g)
    rq1, rs1 = kq.quantize_per_channel_groupwise(k_all[:, :, 32:].astype(np.float32), 4, g)
    rvq, rvs = kq.quantize_per_token(v_all.astype(np.float32), 4)
    assert _bits_equal(k_q[:, :, :L], kq.pack_kv_int4(np.concatenate([rq0, rq1], axis=2)))
    assert _bits_equal_nan(k_s[:, :, :2], np.concatenate([rs0, rs1], axis=2).astype(np.float16))
    assert _bits_equal(v_q[:, :, :L], kq.pack_kv_int4(rvq))
    assert _bits_equal_nan(v_s[:, :, :L], rvs.astype(np.float16))
