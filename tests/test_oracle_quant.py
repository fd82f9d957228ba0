"""Pins for oracle/kv_quant.py (CPU).

* golden vectors written by the reference's own kv_cache_ref.py
  (tests/golden/make_golden.py), fp32 and fp16 inputs, bits 4/8,
  groups 32/128, a short final group (S=100), zero / tiny / tie rows;
* hand-computed half-to-even ties;
* round-trip bound |x - dequant(quant(x))| <= absmax/qmax
  (the reference's tests/test_kv_cache.py:57-116);
* packing <-> unpacking inverse and the byte layout;
* golden rows holding NaN, +-inf and fp16 overflow (reference-written):
  torch's amax propagates NaN, so such a row stores scale NaN / +inf and
  codes 0, in all three conventions (fp32, fp16, and fp16 input .float());
* plant-a-mistake: oracle variants with a plausible error (reciprocal
  multiply, round-half-away, no clamp floor, fp16 scale before the
  division for fp32 inputs, a NaN-dropping absmax) must fail the golden
  vectors.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import kv_quant as kq
from tests.helpers import GOLDEN

GOLD = np.load(GOLDEN / "kv_quant_golden.npz")


def _inputs(prefix: str):
    x32 = GOLD[f"{prefix}_x32"]
    return {f"{prefix}_x32": x32, f"{prefix}_x16": x32.astype(np.float16)}


def _same_bits(a: np.ndarray, b: np.ndarray) -> bool:
    return a.dtype == b.dtype and a.shape == b.shape and np.array_equal(
        a.view(np.uint8), b.view(np.uint8))


@pytest.mark.parametrize("name", ["pt_x32", "pt_x16"])
@pytest.mark.parametrize("bits", [8, 4])
def test_per_token_matches_reference_golden(name, bits):
    x = _inputs("pt")[name]
    q, s = kq.quantize_per_token(x, bits)
    assert _same_bits(q, GOLD[f"{name}_b{bits}_q"])
    assert _same_bits(s, GOLD[f"{name}_b{bits}_s"])


@pytest.mark.parametrize("name", ["gw_x32", "gw_x16"])
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 128])
def test_groupwise_matches_reference_golden(name, bits, gs):
    x = _inputs("gw")[name]
    q, s = kq.quantize_per_channel_groupwise(x, bits, gs)
    assert _same_bits(q, GOLD[f"{name}_b{bits}_g{gs}_q"])
    assert _same_bits(s, GOLD[f"{name}_b{bits}_g{gs}_s"])


def _same_bits_nan(a: np.ndarray, b: np.ndarray) -> bool:
    """Bit-exact, except that a NaN matches any NaN: torch's own NaN payload
    depends on its reduction path (0x7FC00000 from the per-token reduction,
    0xFFFFFFFF from the group-axis one on this CPU), so it pins nothing."""
    if a.dtype != b.dtype or a.shape != b.shape:
        return False
    na, nb = np.isnan(a), np.isnan(b)
    return bool((na == nb).all()) and np.array_equal(a[~na].view(np.uint8), b[~nb].view(np.uint8))


def _nonfinite_inputs(prefix: str):
    x32 = GOLD[f"{prefix}_x32"]
    with np.errstate(over="ignore"):
        x16 = x32.astype(np.float16)
    return {f"{prefix}_x32": x32, f"{prefix}_x16": x16, f"{prefix}_x16f": x16.astype(np.float32)}


@pytest.mark.parametrize("name", ["nf_pt_x32", "nf_pt_x16", "nf_pt_x16f"])
@pytest.mark.parametrize("bits", [8, 4])
def test_per_token_nonfinite_rows_match_reference_golden(name, bits):
    x = _nonfinite_inputs("nf_pt")[name]
    q, s = kq.quantize_per_token(x, bits)
    assert _same_bits(q, GOLD[f"{name}_b{bits}_q"])
    assert _same_bits_nan(s, GOLD[f"{name}_b{bits}_s"])
    # The closed form behind those bits: a NaN row -> scale NaN, an inf row
    # (no NaN) -> scale +inf, and all codes 0 in both.
    bad = ~np.isfinite(x).all(axis=-1)
    assert (q[bad] == 0).all() and not np.isfinite(s[bad]).any()


@pytest.mark.parametrize("name", ["nf_gw_x32", "nf_gw_x16", "nf_gw_x16f"])
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 128])
def test_groupwise_nonfinite_rows_match_reference_golden(name, bits, gs):
    x = _nonfinite_inputs("nf_gw")[name]
    q, s = kq.quantize_per_channel_groupwise(x, bits, gs)
    assert _same_bits(q, GOLD[f"{name}_b{bits}_g{gs}_q"])
    assert _same_bits_nan(s, GOLD[f"{name}_b{bits}_g{gs}_s"])
    assert np.isnan(s).any() and np.isinf(s).any()


def test_nan_dropping_absmax_fails_nonfinite_golden():
    """Plant: an absmax that skips NaN (as fmaxf does) stores a
    finite scale for a row holding a NaN, and the golden rows catch it."""
    x = _nonfinite_inputs("nf_pt")["nf_pt_x16f"]
    absmax = np.where(np.isnan(x), 0.0, np.abs(x)).max(axis=-1, keepdims=True)
    s = np.maximum(absmax / np.float32(127), np.float32(1e-8))
    assert not _same_bits_nan(s[..., 0], GOLD["nf_pt_x16f_b8_s"])


def test_half_even_ties_by_hand():
    x = np.zeros((1, 1, 2, 128), dtype=np.float32)
    x[0, 0, 0, :8] = [127.0, 0.5, 1.5, 2.5, -0.5, -2.5, 63.5, -126.5]   # scale exactly 1
    x[0, 0, 1, :6] = [7.0, 0.5, 1.5, 2.5, 3.5, -3.5]
    q8, s8 = kq.quantize_per_token(x[:, :, :1], 8)
    assert s8[0, 0, 0] == 1.0
    assert q8[0, 0, 0, :8].tolist() == [127, 0, 2, 2, 0, -2, 64, -126]
    q4, s4 = kq.quantize_per_token(x[:, :, 1:], 4)
    assert s4[0, 0, 0] == 1.0
    assert q4[0, 0, 0, :6].tolist() == [7, 0, 2, 2, 4, -4]


def test_zero_row_fp32_convention():
    x = np.zeros((1, 1, 1, 128), dtype=np.float32)
    q, s = kq.quantize_per_token(x, 8)
    assert (q == 0).all() and s[0, 0, 0] == np.float32(1e-8)
    assert np.float16(s[0, 0, 0]) == 0.0   # stored as fp16 it underflows to 0


@pytest.mark.parametrize("bits", [4, 8])
def test_round_trip_bound(bits):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((2, 8, 64, 128)).astype(np.float32)
    x[..., ::17] *= 3.5
    qm = kq.qmax(bits)
    q, s = kq.quantize_per_token(x, bits)
    err = np.abs(kq.dequantize_per_token(q, s) - x)
    tol = np.abs(x).max(axis=-1, keepdims=True) / qm
    assert (err <= tol * 1.001).all()
    assert q.min() >= -qm and q.max() <= qm
    qg, sg = kq.quantize_per_channel_groupwise(x, bits, 32)
    errg = np.abs(kq.dequantize_per_channel_groupwise(qg, sg, 32) - x)
    assert errg.max() <= np.abs(x).max() / qm * 1.001


def test_pack_layout_and_inverse():
    codes = np.array([[1, -1, 7, -7, 0, -8, 3, 4]], dtype=np.int8)
    packed = kq.pack_kv_int4(codes)
    # byte i = (code[2i] & 0xF) | (code[2i+1] & 0xF) << 4
    assert packed.view(np.uint8).tolist() == [[0xF1, 0x97, 0x80, 0x43]]
    rng = np.random.default_rng(1)
    c = rng.integers(-8, 8, size=(3, 5, 128)).astype(np.int8)
    assert np.array_equal(kq.unpack_kv_int4(kq.pack_kv_int4(c)), c)


# ---- plant-a-mistake: each variant must be caught by the golden vectors ----

def _recip_variant(x, bits):
    qm = kq.qmax(bits)
    absmax = np.abs(x).max(axis=-1, keepdims=True)
    s = np.maximum((absmax / x.dtype.type(qm)).astype(x.dtype), x.dtype.type(1e-8))
    r = (np.float32(1.0) / s.astype(np.float32))
    q = np.clip(np.rint(x.astype(np.float32) * r), -qm, qm)
    return np.where(np.isnan(q), 0, q).astype(np.int8), s[..., 0]


def _half_away_variant(x, bits):
    qm = kq.qmax(bits)
    absmax = np.abs(x).max(axis=-1, keepdims=True)
    s = np.maximum((absmax / x.dtype.type(qm)).astype(x.dtype), x.dtype.type(1e-8))
    y = x.astype(np.float32) / s.astype(np.float32)
    q = np.clip(np.sign(y) * np.floor(np.abs(y) + 0.5), -qm, qm)
    return np.where(np.isnan(q), 0, q).astype(np.int8), s[..., 0]


def _fp16_scale_for_fp32_variant(x, bits):
    qm = kq.qmax(bits)
    absmax = np.abs(x).max(axis=-1, keepdims=True)
    s = np.maximum((absmax / x.dtype.type(qm)).astype(np.float16), np.float16(0))
    with np.errstate(invalid="ignore", divide="ignore"):
        q = np.clip(np.rint(x.astype(np.float32) / s.astype(np.float32)), -qm, qm)
    return np.where(np.isnan(q), 0, q).astype(np.int8), s[..., 0].astype(x.dtype)


@pytest.mark.parametrize("variant", [_recip_variant, _half_away_variant,
                                     _fp16_scale_for_fp32_variant])
def test_planted_mistakes_fail_golden(variant):
    x = GOLD["pt_x32"]
    caught = False
    for bits in (8, 4):
        q, s = variant(x, bits)
        if not (np.array_equal(q, GOLD[f"pt_x32_b{bits}_q"])
                and _same_bits(s.astype(np.float32), GOLD[f"pt_x32_b{bits}_s"])):
            caught = True
    assert caught
