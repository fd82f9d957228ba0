"""Host-side pieces of llmik_cuda.decode_layer (no GPU needed)."""
from __future__ import annotations

import math

import pytest
import torch

import tests.helpers  # noqa: F401  (puts the package on sys.path)


def test_rope_tables_are_the_half_split_rotary_angles():
    from llmik_cuda.decode_layer import rope_tables
    cos, sin = rope_tables(7, 128, 500000.0, torch.device("cpu"))
    assert cos.shape == (7, 128) and cos.dtype == torch.float16
    for pos in (0, 3, 6):
        for i in (0, 1, 17, 63):
            ang = pos / (500000.0 ** (2 * i / 128))
            for col in (i, i + 64):      # both halves carry frequency i
                assert float(cos[pos, col]) == float(torch.tensor(math.cos(ang)).half())
                assert float(sin[pos, col]) == float(torch.tensor(math.sin(ang)).half())
    assert torch.all(cos[0] == 1) and torch.all(sin[0] == 0)


def test_layer_shape_validation():
    from llmik_cuda.decode_layer import DecodeLayer
    with pytest.raises(RuntimeError, match="hidden must be n_heads"):
        DecodeLayer(hidden=500, n_heads=4, n_kv_heads=2, intermediate=1024, batch=1, max_len=8,
                    device="cpu")
    with pytest.raises(RuntimeError, match="multiple of n_kv_heads"):
        DecodeLayer(hidden=384, n_heads=3, n_kv_heads=2, intermediate=1024, batch=1, max_len=8,
                    device="cpu")


def test_stack_needs_merged_layers():
    from llmik_cuda.decode_layer import DecodeStack

    class _Layer:
        def __init__(self, fused):
            self.fused = fused

    with pytest.raises(RuntimeError, match="fused=True"):
        DecodeStack([])
    with pytest.raises(RuntimeError, match="fused=True"):
        DecodeStack([_Layer(True), _Layer(False)])
    assert len(DecodeStack([_Layer(True), _Layer(True)]).layers) == 2


def test_interleave_gate_up_tiles():
    """64-column tiles of 32 gate columns then the same 32 up columns; the
    column indices DecodeLayer records for gate and up pick them back out."""
    import llmik_cuda
    K, inter = 3, 96
    gate = torch.arange(K * inter, dtype=torch.float32).reshape(K, inter)
    up = -gate - 1
    w = llmik_cuda.interleave_gate_up(gate, up)
    assert w.shape == (K, 2 * inter)
    for t in range(inter // 32):
        assert torch.equal(w[:, 64 * t:64 * t + 32], gate[:, 32 * t:32 * t + 32])
        assert torch.equal(w[:, 64 * t + 32:64 * t + 64], up[:, 32 * t:32 * t + 32])
    cols = (torch.arange(inter) // 32) * 64 + torch.arange(inter) % 32
    assert torch.equal(w[:, cols], gate) and torch.equal(w[:, cols + 32], up)
    with pytest.raises(RuntimeError, match="I % 32"):
        llmik_cuda.interleave_gate_up(gate[:, :40], up[:, :40])


def test_interleave_head_halves_pairs_rotary_dimensions():
    """Each head's 128 columns become dimensions 0..31, 64..95, 32..63,
    96..127: in 64-column tile t, column i pairs with i + 32 as the rotary
    pair (d, d + 64), d = 32 (t % 2) + i."""
    import llmik_cuda
    K, heads = 2, 3
    w = torch.arange(K * heads * 128, dtype=torch.float32).reshape(K, heads * 128)
    wi = llmik_cuda.interleave_head_halves(w)
    for t in range(2 * heads):
        for i in range(32):
            d = 32 * (t % 2) + i
            assert torch.equal(wi[:, 64 * t + i], w[:, 128 * (t // 2) + d])
            assert torch.equal(wi[:, 64 * t + 32 + i], w[:, 128 * (t // 2) + d + 64])
    with pytest.raises(RuntimeError, match="n_heads_total"):
        llmik_cuda.interleave_head_halves(w[:, :100])
