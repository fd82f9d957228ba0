"""GPU: one decoder layer's decode step on llmik ops (llmik_cuda.decode_layer),
eager and captured in a HIP graph.

* The step is the reference's patched decode sequence
  (integration/prealloc_cache.py:82-144 with W4A16 projections,
  integration/w4a16_patch.py:67-116); it is checked against the same
  sequence restated on the CPU from the oracle's pieces (oracle/fused.py,
  oracle/attention.py, oracle/w4a16.py), rounding to fp16 where the GPU ops
  hand fp16 tensors to each other.
* Both forms of the step are checked: the merged one (q|k|v and gate|up
  projections, rope + cache write, residual add + RMSNorm in one launch
  each) and the op-by-op one.
* Graph replays reproduce the eager step bit for bit: every llmik kernel is
  deterministic (fixed-order split-K reductions), and the module's
  per-stream workspace keeps its counters zero between calls. Replays are
  interleaved with eager work of the program and checked one by one.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import fused as of
from oracle import w4a16 as ow

pytestmark = pytest.mark.gpu

CFG = dict(hidden=512, n_heads=4, n_kv_heads=2, intermediate=1024, batch=4, max_len=160)
POS = 129


def _layer(cuda, seed=0, fused=True):
    from llmik_cuda.decode_layer import DecodeLayer
    layer = DecodeLayer(device=cuda, seed=seed, fused=fused, **CFG)
    g = torch.Generator(device=cuda).manual_seed(seed + 100)
    # context already in the cache for positions < POS
    layer.kbuf[:, :, :POS] = torch.randn(layer.kbuf[:, :, :POS].shape, generator=g, device=cuda).half()
    layer.vbuf[:, :, :POS] = torch.randn(layer.vbuf[:, :, :POS].shape, generator=g, device=cuda).half()
    return layer


def _x(cuda, seed):
    g = torch.Generator(device=cuda).manual_seed(seed)
    return torch.randn((CFG["batch"], CFG["hidden"]), generator=g, device=cuda).half()


def _w_hat(layer, name) -> np.ndarray:
    key, cols = layer.columns[name]
    lin = layer.proj[key]
    codes = ow.unpack_int4_along_k(lin.weight_packed.cpu().numpy())
    w = ow.dequantize_weights_int4_groupwise(codes, lin.scale.cpu().numpy(), lin.group_size)
    return w[:, cols.numpy()]


def _h(a: np.ndarray) -> np.ndarray:
    return a.astype(np.float16)


def _oracle_step(layer, x16: np.ndarray, kbuf: np.ndarray, vbuf: np.ndarray, pos: int) -> np.ndarray:
    B, H, Hkv, D = layer.batch, layer.n_heads, layer.n_kv_heads, layer.head_dim
    W = {n: _w_hat(layer, n) for n in layer.NAMES}
    mm = lambda a, n: _h(a.astype(np.float32) @ W[n])   # noqa: E731  fp32 accumulate, fp16 out
    cos = np.broadcast_to(layer.cos[pos:pos + 1].cpu().numpy()[None], (B, 1, D))
    sin = np.broadcast_to(layer.sin[pos:pos + 1].cpu().numpy()[None], (B, 1, D))
    n1 = _h(of.rmsnorm(x16, layer.ln1.cpu().numpy(), layer.eps))
    q = _h(of.rope(mm(n1, "q").reshape(B, H, 1, D), cos, sin))
    k = _h(of.rope(mm(n1, "k").reshape(B, Hkv, 1, D), cos, sin))
    kbuf = kbuf.copy()
    vbuf = vbuf.copy()
    kbuf[:, :, pos] = k[:, :, 0]
    vbuf[:, :, pos] = mm(n1, "v").reshape(B, Hkv, D)
    attn = _h(oa.decode_attention(q.reshape(B, H, D), kbuf, vbuf, layer.scale, seqlen=pos + 1))
    h = _h(x16.astype(np.float32) + mm(attn.reshape(B, H * D), "o").astype(np.float32))
    n2 = _h(of.rmsnorm(h, layer.ln2.cpu().numpy(), layer.eps))
    m = _h(of.silu_mul(mm(n2, "gate"), mm(n2, "up")))
    return _h(h.astype(np.float32) + mm(m, "down").astype(np.float32))


@pytest.mark.parametrize("fused", [True, False])
def test_decode_step_matches_oracle_composition(llmik, cuda, fused):
    layer = _layer(cuda, fused=fused)
    assert layer.fused == fused
    x = _x(cuda, 1)
    k0, v0 = layer.kbuf.cpu().numpy(), layer.vbuf.cpu().numpy()
    got = layer.step(x, POS).cpu().numpy().astype(np.float32)
    ref = _oracle_step(layer, x.cpu().numpy(), k0, v0, POS).astype(np.float32)
    x32 = x.cpu().numpy().astype(np.float32)
    delta = np.abs(ref - x32).max()
    assert delta > 0.05, delta          # the layer changes its input
    err = np.abs(got - ref).max()
    assert err <= 1e-2, (err, delta)
    # the step wrote this token's K at slot POS and left the context alone
    assert torch.equal(layer.kbuf[:, :, :POS].cpu(), torch.from_numpy(k0[:, :, :POS]))
    assert not torch.equal(layer.kbuf[:, :, POS].cpu(), torch.from_numpy(k0[:, :, POS]))


@pytest.mark.parametrize("fused", [True, False])
def test_graph_replays_reproduce_eager_step(llmik, cuda, fused):
    layer = _layer(cuda, seed=3, fused=fused)
    x = _x(cuda, 4)
    eager = layer.step(x, POS).clone()
    graph, out = layer.capture(x, POS)
    for r in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {r}"
        # the program's own eager work between replays: a later position's
        # step (its cache slot is outside this graph's attention range)
        layer.step(_x(cuda, 10 + r), POS + 1 + r)
        torch.cuda.synchronize()
    # the graph reads x in place: new input, same position
    x.copy_(_x(cuda, 5))
    graph.replay()
    torch.cuda.synchronize()
    replayed = out.clone()
    assert torch.equal(replayed, layer.step(x, POS))


def test_position_bounds(llmik, cuda):
    layer = _layer(cuda)
    with pytest.raises(RuntimeError, match="outside the cache"):
        layer.step(_x(cuda, 1), CFG["max_len"])


def test_stack_equals_chained_layer_steps(llmik, cuda):
    """DecodeStack hands (h, mlp) from layer to layer and adds them in the
    next layer's first RMSNorm launch: the same bits as chaining step()."""
    from llmik_cuda.decode_layer import DecodeStack
    layers = [_layer(cuda, seed=s) for s in (5, 6, 7)]
    x = _x(cuda, 8)
    chained = x
    for layer in layers:
        chained = layer.step(chained, POS)
    stack = DecodeStack(layers)
    assert torch.equal(stack.step(x, POS), chained)
    graph, out = stack.capture(x, POS)
    for r in range(2):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, chained), f"replay {r}"
    with pytest.raises(RuntimeError, match="fused=True"):
        DecodeStack([_layer(cuda, seed=9, fused=False)])


@pytest.mark.parametrize("batch,merge", [(20, True), (4, False)])
def test_merged_step_without_the_projection_merges(llmik, cuda, batch, merge):
    """The merged step where its two projection merges do not apply (a batch
    above 16 rows) or are switched off: the concatenated q|k|v and gate|up
    projections with rope_qkv_append and silu_mul_halves, against the same
    oracle composition."""
    from llmik_cuda.decode_layer import DecodeLayer
    cfg = dict(CFG, batch=batch)
    layer = DecodeLayer(device=cuda, seed=3, merge_swiglu=merge, merge_rope=merge, **cfg)
    assert layer.fused and not layer.swiglu and not layer.qkv_rope
    g = torch.Generator(device=cuda).manual_seed(103)
    layer.kbuf[:, :, :POS] = torch.randn(layer.kbuf[:, :, :POS].shape, generator=g, device=cuda).half()
    layer.vbuf[:, :, :POS] = torch.randn(layer.vbuf[:, :, :POS].shape, generator=g, device=cuda).half()
    x = torch.randn((batch, CFG["hidden"]), generator=g, device=cuda).half()
    k0, v0 = layer.kbuf.cpu().numpy(), layer.vbuf.cpu().numpy()
    got = layer.step(x, POS).cpu().numpy().astype(np.float32)
    ref = _oracle_step(layer, x.cpu().numpy(), k0, v0, POS).astype(np.float32)
    assert np.abs(got - ref).max() <= 1e-2
