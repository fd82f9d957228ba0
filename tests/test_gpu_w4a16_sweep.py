"""GPU parity sweep: W4A16 GEMV/GEMM over randomly drawn shapes.

The shapes come from one fixed seed, so the sweep is the same on every run:
M = 1 (every fifth draw), 2-16 or 17-200, group sizes 32-256 (powers of
two, 70 % of the draws) or 8, 16, 48, 96, K up to 4096 in whole groups, N
up to 1024 (a multiple of 128, 64 or 32 in 70 % of the draws, where the
matrix-core kernels take over; any N otherwise). The draws reach the
16-row matrix-core GEMV, the 32x32 and 16 rt x 64 matrix-core GEMMs and
both generic fallbacks; the M = 1 matrix-core GEMV and the streaming GEMV
(weights above 8 MiB) are covered by test_gpu_w4a16.py and
test_gpu_w4a16_stream.py. A second seeded sweep draws prefill sizes (M
256-3072, N up to 16384): the LDS-staged GEMM unsplit, with every tile in
2 K splits and with the tiles past whole rounds split 2 or 4 ways, and the
64 x 128 and 16-row-tile GEMMs where N or K rule it out. Gate, as in test_gpu_w4a16.py: the fp32-output
instantiation within 2e-3 of the float64 oracle act @ (q * scale); the
fp16 output equals round-to-nearest-even of that same fp32 result bit for
bit; a second call returns the same bits.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import w4a16 as ow
from tests.helpers import randn

pytestmark = pytest.mark.gpu

TOL = 2e-3


def _configs(n: int = 30):
    rng = np.random.default_rng(4162026)
    out = []
    for i in range(n):
        M = 1 if i % 5 == 0 else int(rng.integers(2, 17)) if i % 2 == 0 else int(rng.integers(17, 201))
        gs = int(rng.choice([32, 64, 128, 256] if rng.random() < 0.7 else [8, 16, 48, 96]))
        K = gs * int(rng.integers(1, max(2, 4096 // gs + 1)))
        u = rng.random()
        unit = 128 if u < 0.4 else 64 if u < 0.6 else 32 if u < 0.7 else 1
        N = unit * int(rng.integers(1, 1024 // unit + 1))
        out.append((M, K, N, gs, 7 * i + 1))
    return out


CONFIGS = _configs()


def _dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("M,K,N,gs,seed", CONFIGS,
                         ids=[f"M{c[0]}-K{c[1]}-N{c[2]}-g{c[3]}" for c in CONFIGS])
def test_random_shapes_match_oracle(llmik, cuda, M, K, N, gs, seed):
    W = randn((K, N), seed, scale=0.02)
    q, s = ow.quantize_weights_int4_groupwise(W, gs)
    s = s.astype(np.float16)
    act = randn((M, K), seed + 1).astype(np.float16)
    a, w, sc = _dev(act, cuda), _dev(ow.pack_int4_along_k(q), cuda), _dev(s, cuda)
    out32 = llmik.w4a16_gemm_f32out(a, w, sc, gs)
    out16 = llmik.w4a16_gemm(a, w, sc, gs)
    assert out32.shape == (M, N) and out16.shape == (M, N) and out16.dtype == torch.float16
    ref = ow.quantized_matmul_ref(act, q, s, gs, acc_dtype=np.float64)
    o32 = out32.cpu().numpy()
    assert np.abs(o32 - ref).max() <= TOL
    assert np.array_equal(out16.cpu().numpy().view(np.uint16), o32.astype(np.float16).view(np.uint16))
    assert torch.equal(llmik.w4a16_gemm_f32out(a, w, sc, gs), out32)


def _prefill_configs(n: int = 12):
    """Prefill sizes: M 256-3072, K up to 8192 in whole groups (a multiple of
    64 reaches the LDS-staged GEMM, an odd multiple of 32 the 64 x 128-tile
    one), N up to 16384 in multiples of 128 (three draws in four) or 64 (the
    16-row-tile GEMM), group sizes 32-256."""
    rng = np.random.default_rng(20261202)
    out = []
    for i in range(n):
        M = int(rng.integers(256, 3073))
        gs = int(rng.choice([32, 64, 128, 256]))
        K = gs * int(rng.integers(max(1, 256 // gs), 8192 // gs + 1))
        unit = 128 if i % 4 else 64
        N = unit * int(rng.integers(8, 16384 // unit + 1))
        out.append((M, K, N, gs, 11 * i + 3))
    return out


PREFILL = _prefill_configs()


@pytest.mark.parametrize("M,K,N,gs,seed", PREFILL,
                         ids=[f"M{c[0]}-K{c[1]}-N{c[2]}-g{c[3]}" for c in PREFILL])
def test_random_prefill_shapes(llmik, cuda, M, K, N, gs, seed):
    """Random packed words and scales drawn on the GPU (any 32-bit word is 8
    valid int4 codes); reference act @ (code * scale) in float64 on the GPU,
    its nibble decode checked against the oracle's unpack_int4_along_k on a
    slice. Same gate as above."""
    g = torch.Generator(device=cuda).manual_seed(seed)
    w = torch.randint(-2 ** 31, 2 ** 31 - 1, (K // 8, N), generator=g, device=cuda, dtype=torch.int32)
    sc = (torch.rand((K // gs, N), generator=g, device=cuda) * 0.02 + 0.001).half()
    a = torch.randn((M, K), generator=g, device=cuda, dtype=torch.float16)
    out32 = llmik.w4a16_gemm_f32out(a, w, sc, gs)
    out16 = llmik.w4a16_gemm(a, w, sc, gs)
    shifts = torch.arange(0, 32, 4, device=cuda, dtype=torch.int32).view(1, 8, 1)
    codes = (w.unsqueeze(1) >> shifts) & 0xF
    codes = torch.where(codes >= 8, codes - 16, codes).reshape(K, N)
    assert np.array_equal(codes[:64, :128].cpu().numpy(),
                          ow.unpack_int4_along_k(w[:8, :128].cpu().numpy()).astype(np.int32))
    ref = a.double() @ (codes.double() * sc.double().repeat_interleave(gs, dim=0))
    assert float((out32.double() - ref).abs().max()) <= TOL
    assert torch.equal(out16, out32.half())
    assert torch.equal(llmik.w4a16_gemm_f32out(a, w, sc, gs), out32)

