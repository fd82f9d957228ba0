"""Pins for oracle/w4a16.py (CPU).

* the reference's literal pack/unpack known-answer matrix
  (tests/test_quant.py:201-219 of the reference), unpacked with the kernel's
  shift trick;
* golden vectors from the reference's quant_matmul_ref.py (fp16 and fp32
  weights, groups 64/128, a partial K group, an all-zero column);
* the matmul against float64 brute force; the dequantise-to-fp16
  convention against the fp32 product.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import w4a16 as ow
from tests.helpers import GOLDEN, randn

GOLD = np.load(GOLDEN / "w4a16_golden.npz")

# Literal KAT matrix from the reference's tests/test_quant.py:202-219 (data).
KAT = np.array([
    [7, -7, 3, -3], [0, 1, -1, 2], [-2, 4, -4, 5], [-5, 6, -6, 7],
    [1, 2, 3, 4], [5, 6, 7, -7], [-6, -5, -4, -3], [-2, -1, 0, 1],
    [2, 3, 4, 5], [6, 7, -7, -6], [-5, -4, -3, -2], [-1, 0, 1, 2],
    [3, 4, 5, 6], [7, -7, -6, -5], [-4, -3, -2, -1], [0, 1, 2, 3],
], dtype=np.int8)


def _kernel_unpack_scalar(word: int, i: int) -> int:
    w = word & 0xFFFFFFFF
    shifted = (w << (28 - 4 * i)) & 0xFFFFFFFF
    if shifted >= 0x80000000:
        shifted -= 0x100000000
    return shifted >> 28


def test_pack_kat_matches_kernel_unpack():
    packed = ow.pack_int4_along_k(KAT)
    assert packed.shape == (2, 4) and packed.dtype == np.int32
    for kp in range(2):
        for n in range(4):
            for i in range(8):
                assert _kernel_unpack_scalar(int(packed[kp, n]), i) == KAT[kp * 8 + i, n]
    assert np.array_equal(ow.unpack_int4_along_k(packed), KAT)


@pytest.mark.parametrize("name", ["W32", "W16", "Wp32", "Wp16"])
@pytest.mark.parametrize("gs", [64, 128])
def test_quantizer_matches_reference_golden(name, gs):
    q, s = ow.quantize_weights_int4_groupwise(GOLD[name], gs)
    assert np.array_equal(q, GOLD[f"{name}_g{gs}_q"])
    assert s.dtype == GOLD[f"{name}_g{gs}_s"].dtype
    assert np.array_equal(s.view(np.uint8), GOLD[f"{name}_g{gs}_s"].view(np.uint8))
    if f"{name}_g{gs}_packed" in GOLD:
        assert np.array_equal(ow.pack_int4_along_k(q), GOLD[f"{name}_g{gs}_packed"])


@pytest.mark.parametrize("name", ["Wn32", "Wn16"])
@pytest.mark.parametrize("gs", [64, 128])
def test_quantizer_nonfinite_matches_reference_golden(name, gs):
    """Weights holding NaN, +-inf and fp16 overflow: a group column with a
    NaN stores scale NaN, one with an inf (no NaN) +inf, and codes 0."""
    with np.errstate(invalid="ignore"):
        q, s = ow.quantize_weights_int4_groupwise(GOLD[name], gs)
    g = GOLD[f"{name}_g{gs}_s"]
    assert np.array_equal(q, GOLD[f"{name}_g{gs}_q"])
    # NaN matches any NaN (torch's payload depends on its reduction path).
    assert s.dtype == g.dtype and np.array_equal(np.isnan(s), np.isnan(g))
    assert np.array_equal(s[~np.isnan(s)].view(np.uint8), g[~np.isnan(g)].view(np.uint8))
    assert np.array_equal(ow.pack_int4_along_k(q), GOLD[f"{name}_g{gs}_packed"])
    assert np.isnan(s.astype(np.float32)).any() and np.isinf(s.astype(np.float32)).any()


def test_fp16_and_fp32_weight_conventions_differ():
    # For fp16 W the scale is rounded before the division; the codes of the
    # two conventions must not be assumed equal.
    q16, _ = ow.quantize_weights_int4_groupwise(GOLD["W16"], 128)
    q32, _ = ow.quantize_weights_int4_groupwise(GOLD["W16"].astype(np.float32), 128)
    assert (q16 != q32).any()


def test_matmul_matches_reference_golden_and_brute_force():
    q, s = GOLD["W16_g128_q"], GOLD["W16_g128_s"]
    out32 = ow.quantized_matmul_ref(GOLD["act"], q, s, 128)
    assert np.array_equal(out32.astype(np.float16), GOLD["mm_out16"])
    act = GOLD["act"].astype(np.float64)
    w = q.astype(np.float64) * s.astype(np.float64)[np.arange(256) // 128]
    brute = np.array([[sum(act[m, k] * w[k, n] for k in range(256)) for n in range(8)]
                      for m in range(3)])
    got = ow.quantized_matmul_ref(GOLD["act"], q, s, 128, acc_dtype=np.float64)[:, :8]
    assert np.abs(got - brute).max() < 1e-12


def test_dequantize_fp16_convention():
    rng = np.random.default_rng(3)
    q = rng.integers(-7, 8, size=(256, 40)).astype(np.int8)
    s = (np.abs(randn((2, 40), 4)) * 0.01 + 1e-4).astype(np.float16)
    w16 = ow.w4a16_dequantize_fp16(ow.pack_int4_along_k(q), s, 128)
    ref = (q.astype(np.float64) * s.astype(np.float64)[np.arange(256) // 128]).astype(np.float16)
    assert np.array_equal(w16, ref)
