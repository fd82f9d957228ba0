"""GPU parity: W4A16 GEMV/GEMM and dequantise.

Gate (written here): the fp32-output instantiation of the kernels is within
2e-3 max-abs of the float64 oracle act @ (q * scale); the fp16 output equals
round-to-nearest-even of that same fp32 accumulator, bit for bit. The fp16
output is also reported against the oracle in fp16 ulps (<= 1 ulp + 2e-3),
since |out| reaches ~10 at K=14336 where an fp16 half-ulp exceeds 2e-3.
Weights follow the QuantizedLinear convention (fp32 W quantised,
integration/w4a16_patch.py:78-84); dequantise is bit-exact.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import w4a16 as ow
from tests.helpers import randn

pytestmark = pytest.mark.gpu

TOL = 2e-3
LLAMA = [(4096, 4096), (4096, 14336), (14336, 4096)]


def _dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


_CACHE = {}


def _weights(K, N, gs, seed):
    key = (K, N, gs, seed)
    if key not in _CACHE:
        W = randn((K, N), seed, scale=0.02)
        q, s = ow.quantize_weights_int4_groupwise(W, gs)
        _CACHE.clear()
        _CACHE[key] = (q, s.astype(np.float16), ow.pack_int4_along_k(q))
    return _CACHE[key]


def _check(llmik, cuda, M, K, N, gs, seed):
    q, s, packed = _weights(K, N, gs, seed)
    act = randn((M, K), seed + 1).astype(np.float16)
    a, w, sc = _dev(act, cuda), _dev(packed, cuda), _dev(s, cuda)
    out32 = llmik.w4a16_gemm_f32out(a, w, sc, gs)
    out16 = llmik.w4a16_gemm(a, w, sc, gs)
    ref = ow.quantized_matmul_ref(act, q, s, gs, acc_dtype=np.float64)
    o32 = out32.cpu().numpy()
    assert np.abs(o32 - ref).max() <= TOL
    assert np.array_equal(out16.cpu().numpy().view(np.uint16), o32.astype(np.float16).view(np.uint16))
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    assert (np.abs(out16.cpu().numpy().astype(np.float64) - ref) <= ulp + TOL).all()


@pytest.mark.parametrize("K,N", LLAMA)
@pytest.mark.parametrize("M", [1, 2, 16, 128])
def test_llama_shapes(llmik, cuda, M, K, N):
    _check(llmik, cuda, M, K, N, 128, seed=K + N)


@pytest.mark.parametrize("M,K,N,gs", [(1, 256, 64, 64), (3, 512, 100, 128), (1, 1024, 1000, 32),
                                      (5, 128, 4, 128), (17, 768, 96, 256), (1, 8192, 36, 128),
                                      (33, 256, 260, 64),
                                      # M == 1 matrix-core GEMV: fewest steps, idle waves,
                                      # several load batches per wave
                                      (1, 32, 16, 32), (1, 96, 48, 32), (1, 512, 32, 256),
                                      (1, 16384, 32, 128),
                                      # M == 1 split-K VALU GEMV: group below 32
                                      # or not a power of two, K beyond the staged row
                                      (1, 512, 128, 16), (1, 256, 64, 8), (1, 384, 32, 96),
                                      (1, 20480, 32, 128),
                                      # M >= 2 16-row matrix-core GEMM (N % 128 != 0): row tiles
                                      # 1/2/4/8, partial and several m tiles, one-step K
                                      (2, 1024, 128, 32), (17, 512, 192, 64), (33, 2048, 64, 256),
                                      (200, 256, 64, 32), (7, 32, 64, 32), (65, 4096, 64, 128),
                                      # M > 16 32x32 matrix-core GEMM (N % 128 == 0): partial and
                                      # several m tiles, one-step and odd-step K, K splits, K
                                      # ranges without steps, groups 32..256
                                      (100, 384, 128, 128), (64, 1024, 128, 128), (65, 4096, 128, 128),
                                      (129, 512, 128, 64), (48, 14336, 128, 128), (300, 128, 256, 32),
                                      (24, 32, 128, 32), (40, 96, 128, 32), (127, 2048, 384, 256),
                                      # 2 <= M <= 16 matrix-core GEMV: 32-column tiles, splits,
                                      # a K range that ends inside a batch
                                      (3, 4096, 96, 128), (16, 1056, 32, 32), (9, 7168, 64, 512),
                                      # M >= 256 LDS-staged GEMM (256 x 128 tiles, >= 86 of them
                                      # on 256 CUs): 2 splits with group 32, one split with group
                                      # 64, 2 splits of whole 256-groups, ragged M with 2 splits
                                      # of 6 and 4 stages, a 256-group cut by the split boundary,
                                      # one and two 64-K stages (the second prologue stage clamped),
                                      # groups of 512 and 1024 (8 and 16 stages) in 2 splits
                                      (257, 256, 5504, 32), (600, 512, 6144, 64), (300, 1024, 6400, 256),
                                      (1000, 640, 2816, 128), (260, 256, 5632, 256),
                                      (300, 64, 11008, 32), (513, 128, 11008, 64),
                                      (300, 2048, 6400, 512), (257, 2048, 5504, 1024)])
def test_odd_shapes(llmik, cuda, M, K, N, gs):
    _check(llmik, cuda, M, K, N, gs, seed=M * 7 + K)


@pytest.mark.parametrize("M,K,N,f32", [(128, 4096, 4096, False), (128, 4096, 4096, True),
                                      (300, 128, 256, False), (513, 256, 6144, False),
                                      (300, 512, 6400, True)])
def test_unaligned_output_pointer(llmik, cuda, M, K, N, f32):
    """The 32x32 GEMM stores 8 / 16 bytes at a time only when the output is
    16-byte aligned. An output 4 bytes off (the C ABI's minimum alignment for
    out; a caller's offset view) takes the per-value stores: same bits as the
    aligned output, nothing written outside it. (128, 4096, 4096) splits K;
    (300, 128, 256) does not. (513, 256, 6144) and (300, 512, 6400) run the
    LDS-staged GEMM (one store per value, rows past M dropped by the buffer
    bound), without and with a K split."""
    from llmik_cuda._lib import lib
    q, s, packed = _weights(K, N, 128, 5)
    a = _dev(randn((M, K), 6).astype(np.float16), cuda)
    w, sc = _dev(packed, cuda), _dev(s, cuda)
    dt = torch.float32 if f32 else torch.float16
    ref = (llmik.w4a16_gemm_f32out if f32 else llmik.w4a16_gemm)(a, w, sc, 128)
    buf = torch.full((M * N + 8,), float("nan"), dtype=dt, device=cuda)
    need = lib.llmik_w4a16_workspace_size(M, N, K, 128)
    ws = torch.zeros(max(need, 1), dtype=torch.uint8, device=cuda)
    fn = lib.llmik_w4a16_gemm_f32out if f32 else lib.llmik_w4a16_gemm
    torch.cuda.synchronize()
    off = 4 // buf.element_size()
    st = fn(a.data_ptr(), w.data_ptr(), sc.data_ptr(), buf.data_ptr() + 4,
            M, N, K, 128, ws.data_ptr() if need else None, need,
            torch.cuda.current_stream().cuda_stream)
    assert st == 0, lib.llmik_last_error()
    torch.cuda.synchronize()
    bits = torch.int32 if f32 else torch.int16
    assert torch.equal(buf[off:off + M * N].view(bits), ref.reshape(-1).view(bits))
    assert bool(torch.isnan(buf[:off]).all()) and bool(torch.isnan(buf[off + M * N:]).all())


def test_deterministic(llmik, cuda):
    q, s, packed = _weights(4096, 4096, 128, 1)
    a = _dev(randn((16, 4096), 2).astype(np.float16), cuda)
    w, sc = _dev(packed, cuda), _dev(s, cuda)
    first = llmik.w4a16_gemm(a, w, sc, 128)
    for _ in range(3):
        assert torch.equal(first, llmik.w4a16_gemm(a, w, sc, 128))


@pytest.mark.parametrize("M,K,N", [(128, 4096, 4096), (64, 4096, 4096), (128, 14336, 4096),
                                   (300, 4096, 1024), (100, 384, 128), (40, 2048, 1152),
                                   (300, 1024, 6400)])
def test_split_gemm_repeatable(llmik, cuda, M, K, N):
    """The M > 16 GEMM with K splits (the last split to arrive adds every
    split's partial in split order, its own from registers): the same bits
    over repeated calls in fp32 and fp16 out, fp32 within 2e-3 of the oracle.
    Shapes: column tiles a multiple of 8 (a tile's splits on one XCD) and not
    (its splits on several)."""
    q, s, packed = _weights(K, N, 128, seed=M + K + N)
    act = randn((M, K), M + 5).astype(np.float16)
    a, w, sc = _dev(act, cuda), _dev(packed, cuda), _dev(s, cuda)
    base = llmik.w4a16_gemm_f32out(a, w, sc, 128)
    ref = ow.quantized_matmul_ref(act, q, s, 128, acc_dtype=np.float64)
    assert np.abs(base.cpu().numpy() - ref).max() <= TOL
    for _ in range(5):
        assert torch.equal(llmik.w4a16_gemm_f32out(a, w, sc, 128), base)
        assert torch.equal(llmik.w4a16_gemm(a, w, sc, 128), base.half())


@pytest.mark.parametrize("K,N,gs", [(4096, 4096, 128), (256, 100, 64), (512, 36, 128)])
def test_dequantize_bit_exact(llmik, cuda, K, N, gs):
    q, s, packed = _weights(K, N, gs, seed=K + 3)
    out = llmik.w4a16_dequantize(_dev(packed, cuda), _dev(s, cuda), gs)
    ref = ow.w4a16_dequantize_fp16(packed, s, gs)
    assert np.array_equal(out.cpu().numpy().view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("M,K,N,gs", [(2048, 4096, 4096, 128), (512, 4096, 14336, 128),
                                      (768, 14336, 4096, 128), (1024, 2048, 4096, 32),
                                      (2000, 1024, 11008, 64), (768, 1024, 14336, 128),
                                      (2048, 4096, 14336, 128), (3072, 1024, 14336, 32)])
def test_prefill_sizes_lds_gemm(llmik, cuda, M, K, N, gs):
    """Prefill sizes on the LDS-staged GEMM (M >= 256 with at least 86
    256 x 128 tiles), on 256 CUs: (768, 14336, 4096) and (1024, 2048, 4096)
    with every tile in 2 K splits; (768, 1024, 14336) 256 tiles whole and
    the 80 left in 3 splits of 6, 6 and 4 stages; (2048, 4096, 14336) 768
    whole and 128 in 2; (3072, 1024, 14336) 1280 whole and 64 in 4 (group
    32); (2000, 1024, 11008) 688 tiles, unsplit (splitting the 176 left
    would cost more); the others unsplit. Group 32 and 64, ragged M (2000).
    Reference: act @ (q * scale) in
    float64 on the GPU (the numpy oracle's formula, restated in torch for
    these sizes; the oracle itself covers the smaller shapes above). Gate:
    fp32 output within 2e-3, fp16 output the RNE rounding of the fp32 one,
    repeat calls bit-identical."""
    q, s, packed = _weights(K, N, gs, seed=M + K + N + gs)
    act = randn((M, K), M + 11).astype(np.float16)
    a, w, sc = _dev(act, cuda), _dev(packed, cuda), _dev(s, cuda)
    out32 = llmik.w4a16_gemm_f32out(a, w, sc, gs)
    out16 = llmik.w4a16_gemm(a, w, sc, gs)
    wq = _dev(q, cuda).double() * _dev(s, cuda).double().repeat_interleave(gs, dim=0)
    ref = a.double() @ wq
    assert float((out32.double() - ref).abs().max()) <= TOL
    assert torch.equal(out16, out32.half())
    assert torch.equal(llmik.w4a16_gemm_f32out(a, w, sc, gs), out32)

