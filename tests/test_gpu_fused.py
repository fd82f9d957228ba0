"""GPU parity: fused RMSNorm / SwiGLU / RoPE vs the fp32 oracle (output
within one fp16 rounding of the fp32 value), plus the reference tests'
shapes and broadcast rules (tests/test_fused.py:65-115 of the reference)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import fused as of
from tests.helpers import randn

pytestmark = pytest.mark.gpu


def _dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _within_one_rounding(out: torch.Tensor, ref: np.ndarray, slack: float = 1e-6):
    got = out.float().cpu().numpy()
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float32)
    assert (np.abs(got - ref) <= ulp + slack * np.abs(ref) + 1e-7).all(), np.abs(got - ref).max()


@pytest.mark.parametrize("shape", [(16, 4096), (16, 1024), (1, 4096), (512, 4096), (3, 100),
                                   (4, 8192), (2, 6144), (2, 8200)])
def test_rmsnorm(llmik, cuda, shape):
    x = randn(shape, 1).astype(np.float16)
    w = randn((shape[-1],), 2).astype(np.float16)
    out = llmik.rmsnorm(_dev(x, cuda), _dev(w, cuda), 1e-5)
    _within_one_rounding(out, of.rmsnorm(x, w, 1e-5), slack=1e-5)


def test_rmsnorm_3d_shape(llmik, cuda):
    x = randn((4, 128, 4096), 3).astype(np.float16)
    w = randn((4096,), 4).astype(np.float16)
    out = llmik.rmsnorm(_dev(x, cuda), _dev(w, cuda), 1e-5)
    assert out.shape == x.shape
    _within_one_rounding(out, of.rmsnorm(x, w, 1e-5), slack=1e-5)


@pytest.mark.parametrize("shape", [(16, 14336), (1, 14336), (512, 4096), (7, 13)])
def test_silu_mul(llmik, cuda, shape):
    g = randn(shape, 5).astype(np.float16)
    u = randn(shape, 6).astype(np.float16)
    out = llmik.silu_mul(_dev(g, cuda), _dev(u, cuda))
    _within_one_rounding(out, of.silu_mul(g, u), slack=1e-5)


@pytest.mark.parametrize("B,H,S,D", [(16, 32, 1, 128), (16, 8, 1, 128), (16, 32, 512, 128),
                                     (2, 3, 5, 10)])
def test_rope(llmik, cuda, B, H, S, D):
    x = randn((B, H, S, D), 7).astype(np.float16)
    c = randn((B, S, D), 8).astype(np.float16)
    s = randn((B, S, D), 9).astype(np.float16)
    out = llmik.rope(_dev(x, cuda), _dev(c, cuda), _dev(s, cuda))
    _within_one_rounding(out, of.rope(x, c, s), slack=1e-5)


def test_rope_broadcast_cos(llmik, cuda):
    B, H, S, D = 8, 32, 1, 128
    x = randn((B, H, S, D), 10).astype(np.float16)
    c = randn((S, D), 11).astype(np.float16)
    s = randn((S, D), 12).astype(np.float16)
    out = llmik.rope(_dev(x, cuda), _dev(c, cuda), _dev(s, cuda))
    cb = np.broadcast_to(c, (B, S, D))
    sb = np.broadcast_to(s, (B, S, D))
    _within_one_rounding(out, of.rope(x, cb, sb), slack=1e-5)
