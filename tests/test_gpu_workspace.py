"""GPU: the shared per-stream workspace. Calls of different ops and plans
interleave on one stream; stale split partials left past the counter region
must never be read as completion counters (regression: a W4A16 call with
256 column tiles once read an earlier attention call's partials as
counters)."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import w4a16 as ow
from tests.helpers import randn

pytestmark = pytest.mark.gpu

COUNTER_BYTES = 16384


def _dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _poison_workspaces(llmik):
    torch.cuda.synchronize()
    for ws in llmik._WORKSPACES.values():
        ws[COUNTER_BYTES:].fill_(0xA5)
        assert int(ws[:COUNTER_BYTES].count_nonzero()) == 0   # counters were left zeroed


def _attn_case(llmik, cuda, B, S, seed):
    q = randn((B, 32, 128), seed).astype(np.float16)
    k = randn((B, 8, S, 128), seed + 1).astype(np.float16)
    v = randn((B, 8, S, 128), seed + 2).astype(np.float16)
    out = llmik.decode_attention(_dev(q, cuda), _dev(k, cuda), _dev(v, cuda), 1 / math.sqrt(128))
    ref = oa.decode_attention(q, k, v, 1 / math.sqrt(128))
    assert float(np.abs(out.float().cpu().numpy() - ref).max()) <= 2e-3


def _gemm_case(llmik, cuda, M, K, N, seed):
    W = randn((K, N), seed, scale=0.02)
    q, s = ow.quantize_weights_int4_groupwise(W, 128)
    s = s.astype(np.float16)
    act = randn((M, K), seed + 1).astype(np.float16)
    out = llmik.w4a16_gemm_f32out(_dev(act, cuda), _dev(ow.pack_int4_along_k(q), cuda),
                                  _dev(s, cuda), 128)
    ref = ow.quantized_matmul_ref(act, q, s, 128, acc_dtype=np.float64)
    assert float(np.abs(out.cpu().numpy() - ref).max()) <= 2e-3


def test_interleaved_ops_with_poisoned_partials(llmik, cuda):
    _attn_case(llmik, cuda, 2, 16384, 1)      # many splits, large partials
    _poison_workspaces(llmik)
    _gemm_case(llmik, cuda, 128, 4096, 4096, 2)   # 256 column x row tiles, split K
    _poison_workspaces(llmik)
    _gemm_case(llmik, cuda, 1, 4096, 4096, 3)
    _poison_workspaces(llmik)
    _attn_case(llmik, cuda, 8, 4096, 4)
    _poison_workspaces(llmik)
    _gemm_case(llmik, cuda, 16, 14336, 4096, 5)
    _poison_workspaces(llmik)
    _attn_case(llmik, cuda, 1, 100, 6)


@pytest.mark.parametrize("B,S", [(1, 16384), (2, 4096), (8, 4096)])
def test_split_handoff_is_deterministic(llmik, cuda, B, S):
    """Many splits per (batch, kv head): 40 repeated calls must agree bit for
    bit with the first (a stale or torn partial would show up as a change)."""
    gen = torch.Generator(device=cuda).manual_seed(B * S)
    q = torch.randn((B, 32, 128), generator=gen, device=cuda, dtype=torch.float16)
    k = torch.randn((B, 8, S, 128), generator=gen, device=cuda, dtype=torch.float16)
    v = torch.randn((B, 8, S, 128), generator=gen, device=cuda, dtype=torch.float16)
    first = llmik.decode_attention(q, k, v, 0.0883883)
    outs = [llmik.decode_attention(q, k, v, 0.0883883) for _ in range(40)]
    torch.cuda.synchronize()
    assert all(torch.equal(first, o) for o in outs)
    act = torch.randn((1, 4096), generator=gen, device=cuda, dtype=torch.float16)
    w = torch.randint(-2 ** 31, 2 ** 31 - 1, (512, 4096), generator=gen, device=cuda,
                      dtype=torch.int32)
    sc = (torch.rand((32, 4096), generator=gen, device=cuda) * 0.01).half()
    g0 = llmik.w4a16_gemm_f32out(act, w, sc, 128)
    assert all(torch.equal(g0, llmik.w4a16_gemm_f32out(act, w, sc, 128)) for _ in range(40))


def test_graph_keeps_its_workspace_after_the_stream_grows(llmik, cuda):
    """A graph captured with a small workspace on a stream, then a larger call
    on the same stream that replaces that stream's workspace: the graph's
    replays still use the buffer they were captured with, which must stay
    allocated, and their outputs must equal the eager call bit for bit while
    the caching allocator hands the freed-looking memory to other tensors."""
    gen = torch.Generator(device=cuda).manual_seed(11)
    q = torch.randn((1, 32, 128), generator=gen, device=cuda, dtype=torch.float16)
    k = torch.randn((1, 8, 2048, 128), generator=gen, device=cuda, dtype=torch.float16)
    v = torch.randn((1, 8, 2048, 128), generator=gen, device=cuda, dtype=torch.float16)
    kb = torch.randn((4, 8, 32768, 128), generator=gen, device=cuda, dtype=torch.float16)
    qb = torch.randn((4, 32, 128), generator=gen, device=cuda, dtype=torch.float16)
    torch.cuda.synchronize()   # the inputs are written on the default stream
    stream = torch.cuda.Stream(device=cuda)
    with torch.cuda.stream(stream):
        eager = llmik.decode_attention(q, k, v, 0.0883883)   # sizes this stream's workspace
    stream.synchronize()
    key = (cuda.index or 0, stream.cuda_stream)
    small = llmik._WORKSPACES[key].data_ptr()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        out = llmik.decode_attention(q, k, v, 0.0883883)
    # A call with more slot groups grows the same stream's workspace.
    with torch.cuda.stream(stream):
        big = llmik.decode_attention(qb, kb, kb, 0.0883883)
    stream.synchronize()
    assert llmik._WORKSPACES[key].data_ptr() != small, "the test must force a workspace growth"
    # Fresh allocations that could land on a freed workspace, filled with garbage.
    junk = [torch.full((1 << 20,), 7, dtype=torch.uint8, device=cuda) for _ in range(8)]
    torch.cuda.synchronize()
    for _ in range(3):
        with torch.cuda.stream(stream):
            graph.replay()
        stream.synchronize()
        assert torch.equal(out, eager)
        assert all(int((j != 7).count_nonzero()) == 0 for j in junk)
    with torch.cuda.stream(stream):
        assert torch.equal(llmik.decode_attention(qb, kb, kb, 0.0883883), big)
    torch.cuda.synchronize()


def test_graphs_captured_without_an_eager_call(llmik, cuda):
    """Two graphs captured on a stream that never ran the ops eagerly. Each
    capture creates its own workspace, zeroed inside that graph only, and
    none is cached for the stream: replaying the second graph before the
    first, then an eager call on the same stream, all match eager calls on
    another stream bit for bit (a cached capture-time buffer would reach the
    second graph and the eager call with counters never zeroed)."""
    gen = torch.Generator(device=cuda).manual_seed(21)
    q = torch.randn((2, 32, 128), generator=gen, device=cuda, dtype=torch.float16)
    k = torch.randn((2, 8, 4096, 128), generator=gen, device=cuda, dtype=torch.float16)
    v = torch.randn((2, 8, 4096, 128), generator=gen, device=cuda, dtype=torch.float16)
    q2 = torch.randn((1, 32, 128), generator=gen, device=cuda, dtype=torch.float16)
    k2 = torch.randn((1, 8, 3000, 128), generator=gen, device=cuda, dtype=torch.float16)
    v2 = torch.randn((1, 8, 3000, 128), generator=gen, device=cuda, dtype=torch.float16)
    act = torch.randn((1, 4096), generator=gen, device=cuda, dtype=torch.float16)
    w = torch.randint(-2 ** 31, 2 ** 31 - 1, (512, 4096), generator=gen, device=cuda, dtype=torch.int32)
    sc = (torch.rand((32, 4096), generator=gen, device=cuda) * 0.01).half()
    ref1 = llmik.decode_attention(q, k, v, 0.0883883)
    ref2 = llmik.decode_attention(q2, k2, v2, 0.0883883)
    refw = llmik.w4a16_gemm_f32out(act, w, sc, 128)
    torch.cuda.synchronize()
    # torch draws streams from a pool: take one whose handle no op has used.
    streams = [torch.cuda.Stream(device=cuda) for _ in range(40)]
    stream = next(s for s in streams if (cuda.index or 0, s.cuda_stream) not in llmik._WORKSPACES)
    key = (cuda.index or 0, stream.cuda_stream)
    g1, g2 = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    with torch.cuda.graph(g1, stream=stream):
        o1 = llmik.decode_attention(q, k, v, 0.0883883)
    with torch.cuda.graph(g2, stream=stream):
        o2 = llmik.decode_attention(q2, k2, v2, 0.0883883)
        ow_ = llmik.w4a16_gemm_f32out(act, w, sc, 128)
    assert key not in llmik._WORKSPACES, "a capture-time workspace must not be cached"
    for _ in range(3):
        with torch.cuda.stream(stream):
            g2.replay()
        stream.synchronize()
        assert torch.equal(o2, ref2) and torch.equal(ow_, refw)
        with torch.cuda.stream(stream):
            g1.replay()
        stream.synchronize()
        assert torch.equal(o1, ref1)
    with torch.cuda.stream(stream):
        e1 = llmik.decode_attention(q, k, v, 0.0883883)
        e2 = llmik.decode_attention(q2, k2, v2, 0.0883883)
    stream.synchronize()
    assert torch.equal(e1, ref1) and torch.equal(e2, ref2)
    assert key in llmik._WORKSPACES
