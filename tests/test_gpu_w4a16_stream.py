"""GPU parity for the streaming W4A16 GEMV (1 <= M <= 16, N % 64 == 0).

The shapes are chosen so that the planner's choices are all exercised:
2, 4 and 8 steps per wave (single batch, two batches) and the batched loop
(16 and 24 steps per wave); 8, 13, 14 and 16 waves per workgroup (the
two-stage LDS reduction with and without a partner wave); one split and
several, with a short last split and waves past the end of the K range;
scale groups of 32..512 (a flush per group, or per batch inside a longer
group); M = 1 and 2..16; more tiles than CUs (a second round of
workgroups); and split counts forced with llmik_w4a16_set_plan_override.

The library serves these shapes with the streaming kernel when the packed
weights exceed 8 MiB; the tests force it (llmik_w4a16_set_plan_override) so that the small
shapes take it too. Every packed word is random (every code -8..7 occurs),
scales are random positive fp16, and the reference is act @ (code * scale)
accumulated in float64 on the GPU in K chunks. Gate (written here): the
fp32-output call is
within 2e-3 max-abs of that reference, and the fp16-output call equals
round-to-nearest-even of the same fp32 accumulator bit for bit.
"""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

TOL = 2e-3

# (M, K, N, group_size) and the plan each one lands on with 256 CUs
# (tiles = N / 64, splits = CUs // tiles, then waves x steps per wave).
CASES = [
    (1, 4096, 4096, 128),      # 4 splits, 16 waves x 2 steps
    (1, 8192, 4096, 128),      # 4 splits, 16 x 4
    (1, 4096, 16384, 128),     # 1 split, 16 x 8 (two batches)
    (1, 14336, 4096, 128),     # 4 splits, 14 x 8
    (16, 14336, 4096, 128),    # the same with 16 rows
    (1, 28672, 4096, 128),     # 4 splits, 14 x 16 (loop, 4 batches)
    (5, 28672, 4096, 64),      # loop, groups of 2 steps
    (2, 49152, 4096, 256),     # 4 splits, 16 x 24 (loop, 6 batches), flush inside a group
    (1, 3168, 16384, 32),      # 1 split, 99 steps: 13 x 8 with idle steps, groups of 1 step
    (3, 4096, 4096, 64),       # 2-step waves, groups of 2 steps
    (1, 4096, 4096, 512),      # 2-step waves inside a 16-step group
    (16, 8192, 2048, 128),     # 8 splits of 32 steps, 16 rows
    (7, 2048, 8192, 128),      # 2 splits, 7 rows
    (1, 32, 64, 32),           # one step: 8 waves, 7 of them idle
    (16, 96, 128, 32),         # three steps, 16 rows
    (8, 4096, 28672, 128),     # 448 tiles, more than the CUs: no split, a second round
                               # of workgroups (a decode step's fused gate|up)
    (8, 4096, 6144, 128),      # 96 tiles, 2 splits (a decode step's fused q|k|v)
]


def _ref(act: torch.Tensor, w: torch.Tensor, sc: torch.Tensor, gs: int) -> torch.Tensor:
    """float64 act @ (code * scale), K processed in chunks of 4096."""
    M, K = act.shape
    N = w.shape[1]
    out = torch.zeros((M, N), dtype=torch.float64, device=act.device)
    shifts = (torch.arange(8, device=w.device, dtype=torch.int32) * 4).view(1, 8, 1)
    chunk = 4096
    for k0 in range(0, K, chunk):
        k1 = min(K, k0 + chunk)
        words = w[k0 // 8:k1 // 8]
        codes = ((words.unsqueeze(1) << (28 - shifts)) >> 28).reshape(k1 - k0, N)
        scale = sc.double().repeat_interleave(gs, dim=0)[k0:k1]
        out += act[:, k0:k1].double() @ (codes.double() * scale)
    return out


def _set_plan(stream_mode: int, splits: int) -> None:
    from llmik_cuda._lib import lib
    lib.llmik_w4a16_set_plan_override(stream_mode, splits)


@pytest.fixture(autouse=True)
def _force_stream(llmik):
    """Route every eligible shape to the streaming kernel (the library
    otherwise keeps it for weights of more than 8 MiB); restore the planner
    afterwards."""
    _set_plan(1, -1)
    yield
    _set_plan(-1, -1)


@pytest.mark.parametrize("M,K,N,gs", CASES)
def test_stream_gemv(llmik, cuda, M, K, N, gs):
    g = torch.Generator(device=cuda).manual_seed(M * 1000003 + K * 31 + N + gs)
    w = torch.randint(-2 ** 31, 2 ** 31 - 1, (K // 8, N), generator=g, device=cuda,
                      dtype=torch.int32)
    sc = (torch.rand((K // gs, N), generator=g, device=cuda) * 0.004 + 0.001).half()
    act = torch.randn((M, K), generator=g, device=cuda, dtype=torch.float32).half()
    out32 = llmik.w4a16_gemm_f32out(act, w, sc, gs)
    out16 = llmik.w4a16_gemm(act, w, sc, gs)
    ref = _ref(act, w, sc, gs)
    err = (out32.double() - ref).abs().max().item()
    assert err <= TOL, f"max-abs {err:.3e}"
    assert torch.equal(out16.view(torch.int16), out32.half().view(torch.int16))


@pytest.mark.parametrize("splits", [1, 2, 3, 5, 8])
def test_stream_forced_splits(llmik, cuda, splits):
    """A forced K split count (llmik_w4a16_set_plan_override); every count
    gives results within the gate, and the same fp16 bits as its own fp32 call."""
    _set_plan(1, splits)
    test_stream_gemv(llmik, cuda, 8, 4096, 6144, 128)
    test_stream_gemv(llmik, cuda, 1, 4096, 28672, 128)


def test_stream_repeated_calls_bitwise(llmik, cuda):
    """Split hand-off over repeated calls: identical bits every time."""
    g = torch.Generator(device=cuda).manual_seed(7)
    K, N = 14336, 4096
    w = torch.randint(-2 ** 31, 2 ** 31 - 1, (K // 8, N), generator=g, device=cuda,
                      dtype=torch.int32)
    sc = (torch.rand((K // 128, N), generator=g, device=cuda) * 0.004 + 0.001).half()
    act = torch.randn((1, K), generator=g, device=cuda).half()
    first = llmik.w4a16_gemm(act, w, sc, 128)
    for _ in range(20):
        assert torch.equal(first, llmik.w4a16_gemm(act, w, sc, 128))
