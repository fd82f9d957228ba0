"""GPU: llmik_decode_attention_f16_noalloc (the allocation-free entry point,
its split-K workspace in a static device array) called through the C ABI
gives the same bits as llmik_decode_attention_f16 with a caller workspace,
on consecutive calls of different sizes (the array keeps the previous
call's partials), including a call that needs no workspace, and when its
first call on the device is made under HIP graph capture."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as oa

pytestmark = pytest.mark.gpu


def _inputs(cuda, B, S, buf, seed):
    gen = torch.Generator(device=cuda).manual_seed(seed)
    q = torch.randn((B, 32, 128), generator=gen, device=cuda, dtype=torch.float16)
    k = torch.randn((B, 8, buf, 128), generator=gen, device=cuda, dtype=torch.float16)
    v = torch.randn((B, 8, buf, 128), generator=gen, device=cuda, dtype=torch.float16)
    torch.cuda.synchronize()
    return q, k, v


def _both(lib, q, k, v, S):
    B, buf = q.shape[0], k.shape[2]
    scale = 1.0 / math.sqrt(128)
    stream = torch.cuda.current_stream().cuda_stream
    need = lib.llmik_attention_workspace_size(B, 32, 8, S, 128)
    ws = torch.zeros(max(need, 1), dtype=torch.uint8, device=q.device)
    out_ws = torch.empty_like(q)
    out_na = torch.empty_like(q)
    assert lib.llmik_decode_attention_f16(q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                          out_ws.data_ptr(), B, 32, 8, S, 128, buf, scale,
                                          ws.data_ptr() if need else None, need, stream) == 0
    st = lib.llmik_decode_attention_f16_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                               out_na.data_ptr(), B, 32, 8, S, 128, buf, scale,
                                               stream)
    assert st == 0, lib.llmik_last_error()
    torch.cuda.synchronize()
    return out_ws, out_na, need


def test_noalloc_first_call_under_graph_capture(llmik, cuda):
    """The entry point's first call on the device resolves the scratch
    array's device address (hipGetSymbolAddress). This test runs first in
    its file and no other test calls the entry point, so that first call
    happens inside torch.cuda.graph capture, alone or after the rest of the
    suite. Every replay, with eager no-alloc calls of another size on the
    same scratch between them, equals llmik_decode_attention_f16 with a
    caller workspace bit for bit."""
    from llmik_cuda._lib import lib
    B, S = 8, 4096
    q, k, v = _inputs(cuda, B, S, S, 11)
    scale = 1.0 / math.sqrt(128)
    out = torch.empty_like(q)
    stream = torch.cuda.Stream(device=cuda)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        st = lib.llmik_decode_attention_f16_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                                   out.data_ptr(), B, 32, 8, S, 128, S, scale,
                                                   torch.cuda.current_stream().cuda_stream)
    assert st == 0, lib.llmik_last_error()
    need = lib.llmik_attention_workspace_size(B, 32, 8, S, 128)
    assert need > 0
    ws = torch.zeros(need, dtype=torch.uint8, device=cuda)
    ref = torch.empty_like(q)
    assert lib.llmik_decode_attention_f16(q.data_ptr(), k.data_ptr(), v.data_ptr(), ref.data_ptr(), B, 32,
                                          8, S, 128, S, scale, ws.data_ptr(), need,
                                          torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    small = _inputs(cuda, 2, 1000, 1024, 12)
    for _ in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            graph.replay()
        stream.synchronize()
        assert torch.equal(out, ref)
        out_ws, out_na, _ = _both(lib, *small, 1000)   # eager, same scratch, between replays
        assert torch.equal(out_na, out_ws)


def test_noalloc_matches_the_workspace_entry_point(llmik, cuda):
    from llmik_cuda._lib import lib
    cases = [(8, 4096, 4096, 1),     # 4 splits per slot group
             (2, 1000, 1024, 2),     # smaller, live length inside a longer buffer
             (1, 16384, 16384, 3),   # 32 splits
             (64, 4096, 4096, 4),    # enough workgroups: no split, no workspace
             (2, 1000, 1024, 5)]     # small again after the large ones
    for B, S, buf, seed in cases:
        q, k, v = _inputs(cuda, B, S, buf, seed)
        out_ws, out_na, need = _both(lib, q, k, v, S)
        assert need <= (2 << 20)
        assert torch.equal(out_na, out_ws), (B, S)
        ref = oa.decode_attention(q[:1].cpu().numpy(), k[:1].cpu().numpy(), v[:1].cpu().numpy(),
                                  1.0 / math.sqrt(128), seqlen=S, acc_dtype=np.float64)
        assert float(np.abs(out_na[:1].double().cpu().numpy() - ref).max()) <= 2e-3


def test_noalloc_rejects_bad_arguments(llmik, cuda):
    from llmik_cuda._lib import lib
    q = torch.zeros((1, 32, 64), dtype=torch.float16, device=cuda)
    st = lib.llmik_decode_attention_f16_noalloc(q.data_ptr(), q.data_ptr(), q.data_ptr(),
                                               q.data_ptr(), 1, 32, 8, 1, 64, 1, 0.1, None)
    assert st == -1 and b"head_dim" in lib.llmik_last_error()
