"""GPU parity sweep: decode attention over randomly drawn shapes, all three
KV formats, against the oracle on the same (dequantised) cache, max-abs
<= 2e-3.

The shapes come from one fixed seed, so the sweep is the same on every run:
batch 1-4, 1-8 KV heads, 1, 2, 3, 4 or 8 query heads per KV head, buffers
of 1-2000 tokens with the live length anywhere in them (or the whole
buffer), INT4 groups of 16, 32, 48, 64 and 128 tokens (16 and 48 run the
VALU kernel). These reach split counts from 1 to 8, 4- and 8-wave
workgroups, one, two and four query heads per workgroup, partial last
tiles and partial last INT4 groups. The fp16 shapes run a second time with
every call forced onto the 16-token-tile kernel.
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


def _configs(n: int = 12):
    rng = np.random.default_rng(20261202)
    out = []
    for fmt in ("fp16", "int8", "int4"):
        for i in range(n):
            B = int(rng.integers(1, 5))
            Hkv = int(rng.choice([1, 2, 4, 8]))
            gqa = int(rng.choice([1, 2, 3, 4, 8]))
            L = int(rng.integers(1, 2001))
            live = int(rng.integers(1, L + 1)) if rng.random() < 0.5 else -1
            gs = int(rng.choice([16, 32, 48, 64, 128])) if fmt == "int4" else 0
            out.append((fmt, B, Hkv * gqa, Hkv, L, live, gs, 1000 * i + L))
    return out


CONFIGS = _configs()


def _dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("fmt,B,H,Hkv,L,live,gs,seed", CONFIGS,
                         ids=[f"{c[0]}-B{c[1]}-H{c[2]}-Hkv{c[3]}-L{c[4]}-live{c[5]}-g{c[6]}" for c in CONFIGS])
def test_random_shapes_match_oracle(llmik, cuda, fmt, B, H, Hkv, L, live, gs, seed):
    q = randn((B, H, 128), seed).astype(np.float16)
    k = (randn((B, Hkv, L, 128), seed + 1) if fmt == "fp16"
         else kv_with_outliers((B, Hkv, L, 128), seed + 1)).astype(np.float16)
    v = randn((B, Hkv, L, 128), seed + 2).astype(np.float16)
    scale = 1.0 / math.sqrt(128)
    qd = _dev(q, cuda)
    if fmt == "fp16":
        out = llmik.decode_attention(qd, _dev(k, cuda), _dev(v, cuda), scale, live)
        k_ref, v_ref = k, v
    elif fmt == "int8":
        kq_, ks = llmik.quantize_per_token(_dev(k, cuda))
        vq_, vs = llmik.quantize_per_token(_dev(v, cuda))
        out = llmik.decode_attention_int8(qd, kq_, ks, vq_, vs, scale, seqlen=live)
        k_ref = kq.dequantize_per_token(kq_.cpu().numpy(), ks.cpu().numpy())
        v_ref = kq.dequantize_per_token(vq_.cpu().numpy(), vs.cpu().numpy())
    else:
        kq_, ks = llmik.quantize_k_per_channel_groupwise_int4(_dev(k, cuda), gs)
        vq_, vs = llmik.quantize_v_per_token_int4(_dev(v, cuda))
        out = llmik.decode_attention_int4(qd, kq_, ks, vq_, vs, gs, scale, seqlen=live)
        k_ref = kq.dequantize_per_channel_groupwise(kq.unpack_kv_int4(kq_.cpu().numpy()),
                                                    ks.cpu().numpy(), gs)
        v_ref = kq.dequantize_per_token(kq.unpack_kv_int4(vq_.cpu().numpy()), vs.cpu().numpy())
    ref = oa.decode_attention(q, k_ref, v_ref, scale, seqlen=None if live < 0 else live)
    assert out.shape == (B, H, 128) and out.dtype == torch.float16
    assert float(np.abs(out.float().cpu().numpy() - ref).max()) <= TOL


FP16_CONFIGS = [c for c in CONFIGS if c[0] == "fp16"]


@pytest.mark.parametrize("fmt,B,H,Hkv,L,live,gs,seed", FP16_CONFIGS,
                         ids=[f"half-B{c[1]}-H{c[2]}-Hkv{c[3]}-L{c[4]}-live{c[5]}" for c in FP16_CONFIGS])
def test_random_shapes_fp16_half_tiles(llmik, cuda, fmt, B, H, Hkv, L, live, gs, seed):
    """The same fp16 shapes with every call forced onto the 16-token-tile
    kernel (llmik_attention_set_plan_override(1)), which the planner picks
    only for larger batches."""
    from llmik_cuda._lib import lib
    q = randn((B, H, 128), seed).astype(np.float16)
    k = randn((B, Hkv, L, 128), seed + 1).astype(np.float16)
    v = randn((B, Hkv, L, 128), seed + 2).astype(np.float16)
    scale = 1.0 / math.sqrt(128)
    lib.llmik_attention_set_plan_override(1)
    try:
        out = llmik.decode_attention(_dev(q, cuda), _dev(k, cuda), _dev(v, cuda), scale, live)
        torch.cuda.synchronize()
    finally:
        lib.llmik_attention_set_plan_override(-1)
    ref = oa.decode_attention(q, k, v, scale, seqlen=None if live < 0 else live)
    assert float(np.abs(out.float().cpu().numpy() - ref).max()) <= TOL
