"""Pins for oracle/fused.py (CPU): closed forms and the reference test's
PyTorch formulas (tests/test_fused.py:54-62 of the reference)."""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from oracle import fused as of
from tests.helpers import randn


def test_rmsnorm_closed_form_and_torch():
    x = np.full((2, 64), 3.0, dtype=np.float16)
    w = np.ones(64, dtype=np.float16)
    assert np.allclose(of.rmsnorm(x, w, 0.0), 1.0, atol=1e-7)
    x = randn((4, 256), 1).astype(np.float16)
    w = randn((256,), 2).astype(np.float16)
    xt = torch.from_numpy(x).float()
    ref = xt * torch.rsqrt(xt.pow(2).mean(-1, keepdim=True) + 1e-5) * torch.from_numpy(w).float()
    assert np.abs(of.rmsnorm(x, w, 1e-5) - ref.numpy()).max() < 1e-5
    hf = of.rmsnorm_hf(x, w, 1e-5).astype(np.float32)
    assert np.abs(hf - ref.numpy()).max() < 2e-2


def test_silu_mul_matches_torch():
    g = randn((3, 100), 3).astype(np.float16)
    u = randn((3, 100), 4).astype(np.float16)
    ref = F.silu(torch.from_numpy(g).float()) * torch.from_numpy(u).float()
    assert np.abs(of.silu_mul(g, u) - ref.numpy()).max() < 1e-5
    assert of.silu_mul(np.zeros(4, np.float16), np.ones(4, np.float16)).max() == 0.0


def test_rope_identity_and_torch():
    x = randn((2, 3, 5, 8), 5).astype(np.float16)
    ones = np.ones((2, 5, 8), dtype=np.float16)
    zeros = np.zeros((2, 5, 8), dtype=np.float16)
    assert np.array_equal(of.rope(x, ones, zeros), x.astype(np.float32))
    c = randn((2, 5, 8), 6).astype(np.float16)
    s = randn((2, 5, 8), 7).astype(np.float16)
    xt = torch.from_numpy(x).float()
    rot = torch.cat((-xt[..., 4:], xt[..., :4]), dim=-1)
    ref = xt * torch.from_numpy(c).float()[:, None] + rot * torch.from_numpy(s).float()[:, None]
    assert np.abs(of.rope(x, c, s) - ref.numpy()).max() < 1e-6


def test_rope_is_the_stated_plane_rotation():
    """rope rotates each (i, i + D/2) plane by the angle whose cos / sin it
    is given, in the direction the reference states for its kernel
    (kernels/fused/fused_ops.cu:65: rotate_half(x) = [-x[D/2:], x[:D/2]]):
    e_i -> cos e_i + sin e_{i+D/2} and e_{i+D/2} -> cos e_{i+D/2} - sin e_i.
    A rotation by theta then -theta is the identity, and two rotations add
    their angles: a wrong pairing, sign or half fails one of these."""
    D, h = 8, 4
    th = np.array([0.3, -1.1, 2.0, 0.7], dtype=np.float64)
    ang = np.concatenate([th, th])                    # duplicated-frequency layout

    def cs(a):
        return (np.cos(a)[None, None, :].astype(np.float32), np.sin(a)[None, None, :].astype(np.float32))

    c, s = cs(ang)
    for i in range(h):
        e = np.zeros((1, 1, 1, D), np.float32)
        e[..., i] = 1.0
        out = of.rope(e, c, s)[0, 0, 0]
        want = np.zeros(D)
        want[i], want[i + h] = np.cos(th[i]), np.sin(th[i])
        assert np.allclose(out, want, atol=1e-6)
        e = np.zeros((1, 1, 1, D), np.float32)
        e[..., i + h] = 1.0
        out = of.rope(e, c, s)[0, 0, 0]
        want = np.zeros(D)
        want[i + h], want[i] = np.cos(th[i]), -np.sin(th[i])
        assert np.allclose(out, want, atol=1e-6)
    x = randn((1, 1, 1, D), 9)
    cm, sm = cs(-ang)
    assert np.allclose(of.rope(of.rope(x, c, s), cm, sm), x, atol=1e-6)
    c2, s2 = cs(2 * ang)
    assert np.allclose(of.rope(of.rope(x, c, s), c, s), of.rope(x, c2, s2), atol=1e-5)
