"""GPU: the decode-step merges (rope_qkv_append, add_rmsnorm,
silu_mul_halves, w4a16_gemm_swiglu, w4a16_gemm_qkv_rope) give the same bits
as the ops they replace, which the fused op and W4A16 tests pin against the fp32 oracle;
add_rmsnorm and w4a16_gemm_swiglu are also checked against the oracle
directly."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import fused as of
from oracle import w4a16 as ow
from tests.helpers import randn

pytestmark = pytest.mark.gpu


def _dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("B,H,Hkv,D,max_len,pos", [
    (8, 32, 8, 128, 64, 17),     # Llama-3-8B heads
    (4, 4, 2, 128, 160, 159),    # last slot
    (3, 6, 3, 64, 5, 0),         # first slot, head_dim 64
    (1, 2, 1, 10, 3, 1),         # head_dim not a multiple of 8
])
def test_rope_qkv_append_equals_rope_and_slot_copies(llmik, cuda, B, H, Hkv, D, max_len, pos):
    qkv = _dev(randn((B, (H + 2 * Hkv) * D), 1).astype(np.float16), cuda)
    cos = _dev(randn((D,), 2).astype(np.float16), cuda)
    sin = _dev(randn((D,), 3).astype(np.float16), cuda)
    kc = _dev(randn((B, Hkv, max_len, D), 4).astype(np.float16), cuda)
    vc = _dev(randn((B, Hkv, max_len, D), 5).astype(np.float16), cuda)
    k_ref, v_ref = kc.clone(), vc.clone()
    parts = qkv.view(B, H + 2 * Hkv, D)
    cs = cos.view(1, 1, D).expand(B, 1, D)
    sn = sin.view(1, 1, D).expand(B, 1, D)
    q_ref = llmik.rope(parts[:, :H].contiguous().view(B, H, 1, D), cs, sn).view(B, H, D)
    k_ref[:, :, pos] = llmik.rope(parts[:, H:H + Hkv].contiguous().view(B, Hkv, 1, D), cs, sn)[:, :, 0]
    v_ref[:, :, pos] = parts[:, H + Hkv:]
    q = llmik.rope_qkv_append(qkv, cos, sin, kc, vc, pos)
    assert q.shape == (B, H, D)
    assert torch.equal(q, q_ref)
    assert torch.equal(kc, k_ref)      # slot pos rewritten, every other slot untouched
    assert torch.equal(vc, v_ref)


@pytest.mark.parametrize("rows,hidden", [(8, 4096), (1, 8192), (3, 520), (5, 2056), (2, 6144)])
def test_add_rmsnorm_equals_add_then_rmsnorm(llmik, cuda, rows, hidden):
    x16 = randn((rows, hidden), 6).astype(np.float16)
    r16 = randn((rows, hidden), 7).astype(np.float16)
    w16 = randn((hidden,), 8).astype(np.float16)
    x, r, w = _dev(x16, cuda), _dev(r16, cuda), _dev(w16, cuda)
    h, n = llmik.add_rmsnorm(x, r, w, 1e-5)
    h_ref = x + r
    assert torch.equal(h, h_ref)
    assert torch.equal(n, llmik.rmsnorm(h_ref, w, 1e-5))
    # and against the oracle: h is the one fp16 rounding of the fp32 sum
    h_np = (x16.astype(np.float32) + r16.astype(np.float32)).astype(np.float16)
    assert np.array_equal(h.cpu().numpy(), h_np)
    ref = of.rmsnorm(h_np, w16, 1e-5)
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float32)
    assert (np.abs(n.float().cpu().numpy() - ref) <= ulp + 1e-5 * np.abs(ref) + 1e-7).all()


@pytest.mark.parametrize("rows,cols", [(8, 14336), (1, 1024), (3, 8), (16, 520)])
def test_silu_mul_halves_equals_silu_mul(llmik, cuda, rows, cols):
    gu = _dev(randn((rows, 2 * cols), 9).astype(np.float16), cuda)
    out = llmik.silu_mul_halves(gu)
    assert out.shape == (rows, cols)
    assert torch.equal(out, llmik.silu_mul(gu[:, :cols].contiguous(), gu[:, cols:].contiguous()))


def test_merges_reject_bad_shapes(llmik, cuda):
    kc = torch.zeros((2, 2, 4, 128), dtype=torch.float16, device=cuda)
    cs = torch.zeros(128, dtype=torch.float16, device=cuda)
    qkv = torch.zeros((2, 6 * 128), dtype=torch.float16, device=cuda)
    with pytest.raises(RuntimeError, match="pos outside the cache"):
        llmik.rope_qkv_append(qkv, cs, cs, kc, kc.clone(), 4)
    with pytest.raises(RuntimeError, match="fewer than"):
        llmik.rope_qkv_append(qkv[:, :4 * 128], cs, cs, kc, kc.clone(), 0)
    x = torch.zeros((2, 8200), dtype=torch.float16, device=cuda)
    with pytest.raises(RuntimeError, match="at most 8192"):
        llmik.add_rmsnorm(x, x, x[0], 1e-5)
    with pytest.raises(RuntimeError, match="multiple of 8"):
        llmik.silu_mul_halves(torch.zeros((2, 24), dtype=torch.float16, device=cuda))


@pytest.mark.parametrize("M,K,inter", [(8, 4096, 14336), (1, 4096, 14336), (16, 512, 1024), (3, 256, 96),
                                       (8, 14336, 2048), (5, 1024, 4096)])
def test_w4a16_gemm_swiglu_equals_gemm_then_silu_mul_halves(llmik, cuda, M, K, inter):
    """gate|up + SwiGLU in one launch over the interleaved weight gives the
    bits of the gate|up product over the concatenated weight (on the same
    streaming GEMV plan) followed by silu_mul_halves. Against the oracle
    (silu_mul of the float64 gate and up products g, u): the fp16 gate and up
    products are each within one fp16 ulp + 2e-3 of g and u (the W4A16
    gate), so the output is within |u| silu'(g) (ulp(g) + 2e-3) + |silu(g)|
    (ulp(u) + 2e-3) + one fp16 ulp of the result. Shapes: the Llama gate|up
    at M = 8 and 1, K splits, 96 columns (three tile pairs), the
    down-projection K."""
    from llmik_cuda._lib import lib
    gen = torch.Generator(device=cuda).manual_seed(M * 31 + K + inter)
    gate = torch.randn((K, inter), generator=gen, device=cuda) * 0.02
    up = torch.randn((K, inter), generator=gen, device=cuda) * 0.02
    wc, sc_c = llmik.quantize_pack_weights_int4(torch.cat([gate, up], dim=1).contiguous(), 128)
    wi, sc_i = llmik.quantize_pack_weights_int4(llmik.interleave_gate_up(gate, up).contiguous(), 128)
    act = torch.randn((M, K), generator=gen, device=cuda).half()
    out = llmik.w4a16_gemm_swiglu(act, wi, sc_i, 128)
    assert out.shape == (M, inter) and out.dtype == torch.float16
    lib.llmik_w4a16_set_plan_override(1, -1)   # the concatenated product on the streaming GEMV too
    try:
        ref = llmik.silu_mul_halves(llmik.w4a16_gemm(act, wc, sc_c, 128))
    finally:
        lib.llmik_w4a16_set_plan_override(-1, -1)
    assert torch.equal(out, ref)
    assert torch.equal(llmik.w4a16_gemm_swiglu(act, wi, sc_i, 128), out)   # repeatable
    codes = ow.unpack_int4_along_k(wc.cpu().numpy())
    w = ow.dequantize_weights_int4_groupwise(codes, sc_c.cpu().numpy(), 128).astype(np.float64)
    a = act.cpu().numpy().astype(np.float64)
    g, u = a @ w[:, :inter], a @ w[:, inter:]
    sg = 1.0 / (1.0 + np.exp(-g))
    want = g * sg * u
    ulp = lambda x: np.spacing(np.abs(x).astype(np.float16)).astype(np.float64)  # noqa: E731
    dsilu = np.abs(sg * (1.0 + g * (1.0 - sg)))
    tol = np.abs(u) * dsilu * (ulp(g) + 2e-3) + np.abs(g * sg) * (ulp(u) + 2e-3) + ulp(want)
    assert (np.abs(out.cpu().numpy().astype(np.float64) - want) <= tol).all()


def test_w4a16_gemm_swiglu_rejects_unsupported_shapes(llmik, cuda):
    act = torch.zeros((17, 256), dtype=torch.float16, device=cuda)
    w = torch.zeros((32, 128), dtype=torch.int32, device=cuda)
    s = torch.ones((2, 128), dtype=torch.float16, device=cuda)
    with pytest.raises(RuntimeError, match="M <= 16"):
        llmik.w4a16_gemm_swiglu(act, w, s, 128)
    with pytest.raises(RuntimeError, match="N % 64"):
        llmik.w4a16_gemm_swiglu(act[:4], w[:, :96].contiguous(), s[:, :96].contiguous(), 128)


@pytest.mark.parametrize("B,K,H,Hkv,max_len,pos", [(8, 4096, 32, 8, 64, 17), (1, 4096, 32, 8, 8, 7),
                                                   (16, 512, 4, 2, 40, 0), (3, 2048, 6, 3, 9, 4),
                                                   (5, 256, 2, 1, 3, 2)])
def test_w4a16_gemm_qkv_rope_equals_gemm_then_rope_qkv_append(llmik, cuda, B, K, H, Hkv, max_len, pos):
    """q|k|v projection + rope + cache append in one launch over the
    head-interleaved weight gives the bits of the q|k|v product over the
    concatenated weight (on the same streaming GEMV plan) followed by
    rope_qkv_append: the same q, the same slot `pos` of both caches, every
    other slot untouched (shapes: the Llama-3-8B q|k|v at B = 8 and 1, K
    splits, GQA 2 and 3, MHA-like 2:1, first and last slots)."""
    from llmik_cuda._lib import lib
    gen = torch.Generator(device=cuda).manual_seed(B * 7 + K + H + pos)
    n = (H + 2 * Hkv) * 128
    w = torch.randn((K, n), generator=gen, device=cuda) * 0.02
    wc, sc_c = llmik.quantize_pack_weights_int4(w.contiguous(), 128)
    wi, sc_i = llmik.quantize_pack_weights_int4(llmik.interleave_head_halves(w).contiguous(), 128)
    act = torch.randn((B, K), generator=gen, device=cuda).half()
    cos = torch.randn(128, generator=gen, device=cuda).half()
    sin = torch.randn(128, generator=gen, device=cuda).half()
    kc = torch.randn((B, Hkv, max_len, 128), generator=gen, device=cuda).half()
    vc = torch.randn((B, Hkv, max_len, 128), generator=gen, device=cuda).half()
    k_ref, v_ref = kc.clone(), vc.clone()
    q = llmik.w4a16_gemm_qkv_rope(act, wi, sc_i, cos, sin, kc, vc, pos, H, 128)
    assert q.shape == (B, H, 128) and q.dtype == torch.float16
    lib.llmik_w4a16_set_plan_override(1, -1)   # the concatenated product on the streaming GEMV too
    try:
        qkv = llmik.w4a16_gemm(act, wc, sc_c, 128)
    finally:
        lib.llmik_w4a16_set_plan_override(-1, -1)
    q_ref = llmik.rope_qkv_append(qkv, cos, sin, k_ref, v_ref, pos)
    assert torch.equal(q, q_ref)
    assert torch.equal(kc, k_ref) and torch.equal(vc, v_ref)


def test_w4a16_gemm_qkv_rope_rejects_bad_arguments(llmik, cuda):
    act = torch.zeros((17, 256), dtype=torch.float16, device=cuda)
    w = torch.zeros((32, 4 * 128), dtype=torch.int32, device=cuda)
    s = torch.ones((2, 4 * 128), dtype=torch.float16, device=cuda)
    cs = torch.zeros(128, dtype=torch.float16, device=cuda)
    kc = torch.zeros((17, 1, 4, 128), dtype=torch.float16, device=cuda)
    with pytest.raises(RuntimeError, match="M <= 16"):
        llmik.w4a16_gemm_qkv_rope(act, w, s, cs, cs, kc, kc.clone(), 1, 2, 128)
    with pytest.raises(RuntimeError, match="pos outside the cache"):
        llmik.w4a16_gemm_qkv_rope(act[:2], w, s, cs, cs, kc[:2].contiguous(), kc[:2].clone(), 4, 2, 128)
    with pytest.raises(RuntimeError, match="n_heads \\+ 2 n_kv_heads"):
        llmik.w4a16_gemm_qkv_rope(act[:2], w, s, cs, cs, kc[:2].contiguous(), kc[:2].clone(), 0, 4, 128)
