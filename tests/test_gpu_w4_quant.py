"""GPU parity: the W4 weight quantiser and packer against the reference's
own outputs and the oracle.

Pins, all bit-exact (codes, packed words, scales in their dtype):
  * the golden vectors tests/golden/w4a16_golden.npz, written by the
    reference's quantize_weights_int4_groupwise / pack_int4_along_k
    (reference/quant_matmul_ref.py:39-88, 140-165): fp32 and fp16 weights,
    groups of 64 and 128, and a 100-row matrix whose last group is short;
  * the oracle (oracle/w4a16.py) on larger random matrices, groups 32..256,
    with outlier rows;
  * hand-made ties (quotients exactly x.5 round half to even), all-zero
    groups (fp16: scale 0 and 0/0 codes -> 0; fp32: the 1e-8 floor), and a
    group size that is not a multiple of 8 (quantise, then pack);
  * the fused QuantizedLinear convention (integration/w4a16_patch.py:78-84:
    fp32 codes, fp16 scales) and a W4A16 GEMM on its output.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import w4a16 as ow
from tests.helpers import randn

pytestmark = pytest.mark.gpu

GOLD = np.load(Path(__file__).resolve().parent / "golden" / "w4a16_golden.npz")


def _dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _bits(t: torch.Tensor) -> np.ndarray:
    a = t.cpu().numpy()
    return a.view({1: np.uint8, 2: np.uint16, 4: np.uint32}[a.itemsize])


@pytest.mark.parametrize("name", ["W32", "W16", "Wp32", "Wp16"])
@pytest.mark.parametrize("gs", [64, 128])
def test_quantizer_matches_reference_golden(llmik, cuda, name, gs):
    W = _dev(GOLD[name], cuda)
    q, s = llmik.quantize_weights_int4_groupwise(W, gs)
    assert q.dtype == torch.int8 and s.dtype == W.dtype
    assert np.array_equal(q.cpu().numpy(), GOLD[f"{name}_g{gs}_q"])
    assert np.array_equal(_bits(s), GOLD[f"{name}_g{gs}_s"].view(_bits(s).dtype))
    key = f"{name}_g{gs}_packed"
    if key in GOLD.files:
        assert np.array_equal(llmik.pack_int4_along_k(q).cpu().numpy(), GOLD[key])


@pytest.mark.parametrize("name", ["Wn32", "Wn16"])
@pytest.mark.parametrize("gs", [64, 128])
def test_quantizer_nonfinite_matches_reference_golden(llmik, cuda, name, gs):
    """Weights holding NaN, +-inf and fp16 overflow: torch's amax propagates
    NaN (quant_matmul_ref.py:79-80), so a group column with a NaN stores
    scale NaN, one with an inf +inf, and their codes are 0. NaN matches any
    NaN (torch's payload depends on its reduction path)."""
    W = _dev(GOLD[name], cuda)
    q, s = llmik.quantize_weights_int4_groupwise(W, gs)
    assert np.array_equal(q.cpu().numpy(), GOLD[f"{name}_g{gs}_q"])
    got, ref = s.cpu().numpy(), GOLD[f"{name}_g{gs}_s"]
    assert got.dtype == ref.dtype and np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(got[~np.isnan(got)].view(np.uint8), ref[~np.isnan(ref)].view(np.uint8))
    assert np.array_equal(llmik.pack_int4_along_k(q).cpu().numpy(), GOLD[f"{name}_g{gs}_packed"])


@pytest.mark.parametrize("K,N,gs,dtype", [(4096, 512, 128, np.float32), (1024, 320, 64, np.float16),
                                          (1000, 96, 128, np.float32), (768, 130, 256, np.float16),
                                          (512, 64, 32, np.float32), (2048, 48, 32, np.float16)])
def test_quantizer_matches_oracle(llmik, cuda, K, N, gs, dtype):
    W = randn((K, N), K + N + gs, scale=0.02)
    W[::97] *= 25.0   # outlier rows
    W = W.astype(dtype)
    q, s = llmik.quantize_weights_int4_groupwise(_dev(W, cuda), gs)
    rq, rs = ow.quantize_weights_int4_groupwise(W, gs)
    assert np.array_equal(q.cpu().numpy(), rq)
    assert np.array_equal(_bits(s), rs.view(_bits(s).dtype))
    if K % 8 == 0:
        assert np.array_equal(llmik.pack_int4_along_k(q).cpu().numpy(), ow.pack_int4_along_k(rq))


def test_ties_zero_groups_and_floor(llmik, cuda):
    # Column 0: absmax 7 -> scale exactly 1, quotients x.5 -> half to even.
    col = np.array([7.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5], dtype=np.float32)
    W = np.zeros((16, 3), dtype=np.float32)
    W[:8, 0] = col
    W[8:, 0] = -col
    W[:, 1] = 0.0                   # an all-zero column: scale floor, codes 0
    W[:8, 2] = 1e-12                # below the floor (fp16: underflows to a zero group)
    W[8:, 2] = -3e-9                # the floor scale: codes round to 0
    for dtype in (np.float32, np.float16):
        Wd = W.astype(dtype)
        q, s = llmik.quantize_weights_int4_groupwise(_dev(Wd, cuda), 8)
        rq, rs = ow.quantize_weights_int4_groupwise(Wd, 8)
        assert np.array_equal(q.cpu().numpy(), rq), dtype
        assert np.array_equal(_bits(s), rs.view(_bits(s).dtype)), dtype
    q32, s32 = llmik.quantize_weights_int4_groupwise(_dev(W, cuda), 8)
    assert q32.cpu().numpy()[:8, 0].tolist() == [7, 0, 2, 2, 0, -2, -2, 4]
    assert float(s32[0, 1]) == np.float32(1e-8) and not q32[:, 1].any()
    q16, s16 = llmik.quantize_weights_int4_groupwise(_dev(W.astype(np.float16), cuda), 8)
    assert float(s16[0, 1]) == 0.0 and not q16[:, 1].any()   # 0/0 -> code 0


def test_group_not_multiple_of_8_and_fused_convention(llmik, cuda):
    W = randn((96, 40), 5, scale=0.02)
    packed, s16 = llmik.quantize_pack_weights_int4(_dev(W, cuda), 12)
    rq, rs = ow.quantize_weights_int4_groupwise(W, 12)
    assert np.array_equal(packed.cpu().numpy(), ow.pack_int4_along_k(rq))
    assert np.array_equal(_bits(s16), rs.astype(np.float16).view(np.uint16))
    # QuantizedLinear: fp16 Linear weight [N, K] -> W_kn.float() -> fp32 codes, fp16 scales.
    lin = randn((256, 1024), 6, scale=0.02).astype(np.float16)
    W_kn = np.ascontiguousarray(lin.T).astype(np.float32)
    packed, s16 = llmik.quantize_pack_weights_int4(_dev(W_kn, cuda), 128)
    rq, rs = ow.quantize_weights_int4_groupwise(W_kn, 128)
    assert np.array_equal(packed.cpu().numpy(), ow.pack_int4_along_k(rq))
    assert np.array_equal(_bits(s16), rs.astype(np.float16).view(np.uint16))


def test_quantized_weights_feed_the_gemm(llmik, cuda):
    K, N = 4096, 1024
    W = randn((K, N), 7, scale=0.02)
    packed, s16 = llmik.quantize_pack_weights_int4(_dev(W, cuda), 128)
    rq, rs = ow.quantize_weights_int4_groupwise(W, 128)
    act = randn((4, K), 8).astype(np.float16)
    a = _dev(act, cuda)
    got = llmik.w4a16_gemm(a, packed, s16, 128)
    ref = llmik.w4a16_gemm(a, _dev(ow.pack_int4_along_k(rq), cuda), _dev(rs.astype(np.float16), cuda), 128)
    assert torch.equal(got, ref)
