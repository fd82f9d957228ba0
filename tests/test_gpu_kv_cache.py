"""GPU parity: the in-place writers and the cat-free caches.

* The *_into writers produce the codes and scales of the out-of-place
  writers bit for bit at any offset, from contiguous inputs and from token
  slices of a larger buffer, and leave every other cache position untouched
  (poisoned before the call).
* Int4KIVICache after a sequence of appends (single tokens, chunks that
  cross group boundaries, whole groups) holds exactly what the reference's
  Int4KIVICache holds for the same tokens (integration/kv_int4_cache.py:
  full groups quantised per group, the trailing residual as one partial
  group, V per token), computed here with the oracle's quantisers on the
  same fp16 tokens; Int8KVCache holds the per-token codes.
* Attention through either cache over its live length matches the oracle
  on the dequantised live KV within 2e-3 max-abs.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import kv_quant as kq
from tests.helpers import kv_with_outliers, randn

pytestmark = pytest.mark.gpu

TOL = 2e-3


def _dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _np(t):
    return t.cpu().numpy()


@pytest.mark.parametrize("n,offset,cache_len,slice_from", [
    (1, 0, 64, None), (1, 37, 64, None), (17, 5, 64, None), (64, 0, 64, None),
    (12, 20, 96, (3, 40)),   # a token slice [3, 15) of a 40-token buffer
])
def test_per_token_into_matches_out_of_place(llmik, cuda, n, offset, cache_len, slice_from):
    B, H = 2, 8
    if slice_from is None:
        x = _dev(kv_with_outliers((B, H, n, 128), n + offset).astype(np.float16), cuda)
    else:
        a, L = slice_from
        buf = _dev(kv_with_outliers((B, H, L, 128), n + offset).astype(np.float16), cuda)
        x = buf[:, :, a:a + n]
    for int4 in (False, True):
        width = 64 if int4 else 128
        qc = torch.full((B, H, cache_len, width), 0x5A, dtype=torch.int8, device=cuda)
        sc = torch.full((B, H, cache_len), 1234.0, dtype=torch.float16, device=cuda)
        if int4:
            llmik.quantize_v_per_token_int4_into(x, qc, sc, offset)
            rq, rs = llmik.quantize_v_per_token_int4(x.contiguous())
        else:
            llmik.quantize_per_token_into(x, qc, sc, offset)
            rq, rs = llmik.quantize_per_token(x.contiguous())
        assert torch.equal(qc[:, :, offset:offset + n], rq)
        assert torch.equal(sc[:, :, offset:offset + n].view(torch.int16), rs.view(torch.int16))
        rest = torch.ones(cache_len, dtype=torch.bool, device=cuda)
        rest[offset:offset + n] = False
        assert (qc[:, :, rest] == 0x5A).all() and (sc[:, :, rest] == 1234.0).all()


@pytest.mark.parametrize("n,offset,cache_len,g", [
    (32, 0, 64, 32), (5, 32, 64, 32), (70, 64, 160, 32), (128, 128, 256, 128), (1, 0, 8, 8),
    (200, 256, 512, 128),
])
def test_k_groupwise_into_matches_out_of_place(llmik, cuda, n, offset, cache_len, g):
    B, H = 2, 8
    buf = _dev(kv_with_outliers((B, H, n + 3, 128), n * 7 + g).astype(np.float16), cuda)
    x = buf[:, :, 3:3 + n]
    ng = (cache_len + g - 1) // g
    qc = torch.full((B, H, cache_len, 64), 0x5A, dtype=torch.int8, device=cuda)
    sc = torch.full((B, H, ng, 128), 1234.0, dtype=torch.float16, device=cuda)
    llmik.quantize_k_per_channel_groupwise_int4_into(x, qc, sc, offset, g)
    rq, rs = llmik.quantize_k_per_channel_groupwise_int4(x.contiguous(), g)
    g0, ngx = offset // g, rs.size(2)
    assert torch.equal(qc[:, :, offset:offset + n], rq)
    assert torch.equal(sc[:, :, g0:g0 + ngx].view(torch.int16), rs.view(torch.int16))
    tok = torch.ones(cache_len, dtype=torch.bool, device=cuda)
    tok[offset:offset + n] = False
    grp = torch.ones(ng, dtype=torch.bool, device=cuda)
    grp[g0:g0 + ngx] = False
    assert (qc[:, :, tok] == 0x5A).all() and (sc[:, :, grp] == 1234.0).all()


def _reference_kivi_view(k_all, v_all, g):
    """What the reference Int4KIVICache stores for these tokens (oracle
    quantisers): full groups of K quantised per group, the residual as one
    partial group, V per token. Returns unpacked codes and fp16 scales."""
    S = k_all.shape[2]
    full = S // g * g
    kqs, kss = [], []
    if full:
        q, s = kq.quantize_per_channel_groupwise(k_all[:, :, :full].astype(np.float32), 4, g)
        kqs.append(q)
        kss.append(s.astype(np.float16))
    if S > full:
        q, s = kq.quantize_per_channel_groupwise(k_all[:, :, full:].astype(np.float32), 4, g)
        kqs.append(q)
        kss.append(s.astype(np.float16))
    vq, vs = kq.quantize_per_token(v_all.astype(np.float32), 4)
    return (np.concatenate(kqs, axis=2), np.concatenate(kss, axis=2), vq, vs.astype(np.float16))


@pytest.mark.parametrize("g,appends", [
    (32, [1] * 40),                         # decode: single tokens across a group boundary
    (32, [100, 1, 1, 30, 1, 64, 3]),        # prefill with a partial group, then mixed appends
    (128, [128, 5, 123, 1, 300]),           # KIVI at group 128
    (16, [7, 9, 16, 1, 48]),
    (64, [1] * 70),                         # single tokens through a whole group of 64
    (100, [50] + [1] * 60),                 # a group size that is no power of two
])
def test_int4_cache_matches_reference_semantics(llmik, cuda, g, appends):
    from llmik_cuda.kv_cache import Int4KIVICache
    B, H, Hq = 2, 8, 32
    total = sum(appends)
    k_all = kv_with_outliers((B, H, total, 128), g + total).astype(np.float16)
    v_all = randn((B, H, total, 128), g + total + 1).astype(np.float16)
    cache = Int4KIVICache(B, H, max_len=total + 17, group_size=g, device=cuda)
    pos = 0
    scale = 1.0 / math.sqrt(128)
    for step, n in enumerate(appends):
        cache.append(_dev(k_all[:, :, pos:pos + n], cuda), _dev(v_all[:, :, pos:pos + n], cuda))
        pos += n
        assert cache.length == pos
        rq, rs, rvq, rvs = _reference_kivi_view(k_all[:, :, :pos], v_all[:, :, :pos], g)
        k_q, k_s, v_q, v_s, L = cache.get_quantized_for_attention()
        ng = (pos + g - 1) // g
        assert np.array_equal(_np(k_q[:, :, :L]), kq.pack_kv_int4(rq))
        assert np.array_equal(_np(k_s[:, :, :ng]).view(np.uint16), rs.view(np.uint16))
        assert np.array_equal(_np(v_q[:, :, :L]), kq.pack_kv_int4(rvq))
        assert np.array_equal(_np(v_s[:, :, :L]).view(np.uint16), rvs.view(np.uint16))
        if step in (0, len(appends) // 2, len(appends) - 1):
            q = randn((B, Hq, 128), step + pos).astype(np.float16)
            out = cache.attention(_dev(q, cuda), scale)
            k_dq = kq.dequantize_per_channel_groupwise(rq, rs, g)
            v_dq = kq.dequantize_per_token(rvq, rvs)
            ref = oa.decode_attention(q, k_dq, v_dq, scale)
            assert float(np.abs(out.float().cpu().numpy() - ref).max()) <= TOL


def test_int8_cache_appends_and_attention(llmik, cuda):
    from llmik_cuda.kv_cache import Int8KVCache
    B, H, Hq = 3, 8, 32
    appends = [50, 1, 1, 13, 1, 64]
    total = sum(appends)
    k_all = kv_with_outliers((B, H, total, 128), 11).astype(np.float16)
    v_all = randn((B, H, total, 128), 12).astype(np.float16)
    cache = Int8KVCache(B, H, max_len=200, device=cuda)
    pos = 0
    scale = 1.0 / math.sqrt(128)
    for n in appends:
        cache.append(_dev(k_all[:, :, pos:pos + n], cuda), _dev(v_all[:, :, pos:pos + n], cuda))
        pos += n
    rkq, rks = kq.quantize_per_token(k_all.astype(np.float32), 8)
    rvq, rvs = kq.quantize_per_token(v_all.astype(np.float32), 8)
    k_q, k_s, v_q, v_s, L = cache.get_quantized_for_attention()
    assert L == total
    assert np.array_equal(_np(k_q[:, :, :L]), rkq) and np.array_equal(_np(v_q[:, :, :L]), rvq)
    assert np.array_equal(_np(k_s[:, :, :L]).view(np.uint16), rks.astype(np.float16).view(np.uint16))
    assert np.array_equal(_np(v_s[:, :, :L]).view(np.uint16), rvs.astype(np.float16).view(np.uint16))
    q = randn((B, Hq, 128), 13).astype(np.float16)
    out = cache.attention(_dev(q, cuda), scale)
    k_dq = kq.dequantize_per_token(rkq, rks.astype(np.float16))
    v_dq = kq.dequantize_per_token(rvq, rvs.astype(np.float16))
    ref = oa.decode_attention(q, k_dq, v_dq, scale)
    assert float(np.abs(out.float().cpu().numpy() - ref).max()) <= TOL


def test_cache_capacity_is_enforced(llmik, cuda):
    from llmik_cuda.kv_cache import Int4KIVICache
    cache = Int4KIVICache(1, 8, max_len=8, group_size=4, device=cuda)
    x = torch.zeros((1, 8, 9, 128), dtype=torch.float16, device=cuda)
    with pytest.raises(RuntimeError, match="capacity"):
        cache.append(x, x)
