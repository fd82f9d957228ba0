"""GPU parity: split-K decode attention (fp16, INT8, INT4 KIVI) vs the
oracle, max-abs <= 2e-3 against the fp32 oracle on the same inputs.

INT8 / INT4 cases quantise with this build's writers (whose codes and scales
are checked bit-exact in test_gpu_kv_writers.py) and compare against the
oracle run on the fp32-dequantised cache, so the gate isolates the fused
dequant + attention arithmetic.
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


def _inputs(B, H, Hkv, L, seed, outliers=False):
    q = randn((B, H, 128), seed).astype(np.float16)
    k = (kv_with_outliers((B, Hkv, L, 128), seed + 1) if outliers
         else randn((B, Hkv, L, 128), seed + 1)).astype(np.float16)
    v = randn((B, Hkv, L, 128), seed + 2).astype(np.float16)
    return q, k, v


def _max_abs(out: torch.Tensor, ref: np.ndarray) -> float:
    return float(np.abs(out.float().cpu().numpy() - ref).max())


@pytest.mark.parametrize("B,H,Hkv,L", [
    (1, 32, 8, 512),      # CPU-plumbing config shape
    (8, 32, 8, 4096),     # headline config
    (1, 32, 8, 1), (2, 32, 8, 17), (1, 32, 8, 100), (8, 32, 8, 1024), (1, 32, 8, 16384),
    (3, 8, 8, 300),       # MHA
    (2, 16, 8, 777),      # GQA 2
    (2, 12, 4, 257),      # GQA 3
    (1, 64, 8, 2048),     # GQA 8 (two head chunks per kv head)
])
def test_fp16_matches_oracle(llmik, cuda, B, H, Hkv, L):
    q, k, v = _inputs(B, H, Hkv, L, seed=B * 1000 + L)
    scale = 1.0 / math.sqrt(128)
    out = llmik.decode_attention(_dev(q, cuda), _dev(k, cuda), _dev(v, cuda), scale)
    torch.cuda.synchronize()
    assert out.shape == (B, H, 128) and out.dtype == torch.float16
    ref = oa.decode_attention(q, k, v, scale)
    assert _max_abs(out, ref) <= TOL


def test_fp16_v3_alias_and_named_args(llmik, cuda):
    q, k, v = _inputs(2, 32, 8, 333, seed=7)
    qd, kd, vd = _dev(q, cuda), _dev(k, cuda), _dev(v, cuda)
    a = llmik.decode_attention(q=qd, k=kd, v=vd, softmax_scale=0.125)
    b = llmik.decode_attention_v3(qd, kd, vd, 0.125)
    assert torch.equal(a, b)
    assert _max_abs(a, oa.decode_attention(q, k, v, 0.125)) <= TOL


@pytest.mark.parametrize("buf,live", [(1024, 777), (4096, 2049), (256, 1), (512, 512)])
def test_fp16_live_length_in_preallocated_cache(llmik, cuda, buf, live):
    q, k, v = _inputs(2, 32, 8, buf, seed=buf + live)
    # poison the dead tail: it must not be read
    k[:, :, live:] = np.float16(60000.0)
    v[:, :, live:] = np.float16(np.nan)
    out = llmik.decode_attention(_dev(q, cuda), _dev(k, cuda), _dev(v, cuda), 0.0883883, live)
    ref = oa.decode_attention(q, k, v, 0.0883883, seqlen=live)
    assert _max_abs(out, ref) <= TOL


def test_fp16_empty_cache_gives_zeros(llmik, cuda):
    q = _dev(randn((2, 32, 128), 1).astype(np.float16), cuda)
    k = torch.zeros((2, 8, 0, 128), dtype=torch.float16, device=cuda)
    out = llmik.decode_attention(q, k, k.clone(), 0.1)
    assert torch.count_nonzero(out) == 0


def test_fp16_deterministic_across_calls(llmik, cuda):
    q, k, v = _inputs(8, 32, 8, 4096, seed=99)
    qd, kd, vd = _dev(q, cuda), _dev(k, cuda), _dev(v, cuda)
    a = llmik.decode_attention(qd, kd, vd, 0.0883883)
    for _ in range(3):
        assert torch.equal(a, llmik.decode_attention(qd, kd, vd, 0.0883883))


@pytest.mark.parametrize("B,L", [(1, 128), (4, 1000), (8, 4096), (1, 16384)])
def test_int8_pipeline_matches_oracle(llmik, cuda, B, L):
    q, k, v = _inputs(B, 32, 8, L, seed=3 * L + B, outliers=True)
    kq_, ks = llmik.quantize_per_token(_dev(k, cuda))
    vq_, vs = llmik.quantize_per_token(_dev(v, cuda))
    out = llmik.decode_attention_int8(_dev(q, cuda), kq_, ks, vq_, vs, 1 / math.sqrt(128))
    k_dq = kq.dequantize_per_token(kq_.cpu().numpy(), ks.cpu().numpy())
    v_dq = kq.dequantize_per_token(vq_.cpu().numpy(), vs.cpu().numpy())
    ref = oa.decode_attention(q, k_dq, v_dq, 1 / math.sqrt(128))
    assert _max_abs(out, ref) <= TOL


def test_int8_live_length(llmik, cuda):
    q, k, v = _inputs(2, 32, 8, 1024, seed=5, outliers=True)
    kq_, ks = llmik.quantize_per_token(_dev(k, cuda))
    vq_, vs = llmik.quantize_per_token(_dev(v, cuda))
    out = llmik.decode_attention_int8(_dev(q, cuda), kq_, ks, vq_, vs, 0.0883883, seqlen=700)
    k_dq = kq.dequantize_per_token(kq_.cpu().numpy(), ks.cpu().numpy())
    v_dq = kq.dequantize_per_token(vq_.cpu().numpy(), vs.cpu().numpy())
    assert _max_abs(out, oa.decode_attention(q, k_dq, v_dq, 0.0883883, seqlen=700)) <= TOL


@pytest.mark.parametrize("B,L,live", [(8, 4096, 4096), (4, 4097, 4097), (8, 3500, 3001), (32, 1500, 1500),
                                      (2, 16384, 16383)])
def test_int8_rotated_walk(llmik, cuda, B, L, live):
    """Under a split plan, INT8 KV head h walks its tiles starting h / Hkv
    of the way into the sequence and wraps. Cases: the A8 config; a
    one-token last tile that the rotation places mid-walk (4097); a live
    length inside a longer buffer whose tail codes and scales are poisoned
    (3001 of 3500); 4-wave workgroups and no split, the plain walk (B=32,
    S=1500); 16 splits (B=2) and a live length one short of the buffer
    (16383 of 16384).
    Oracle parity (float64) on sampled rows, bit-equal repeats, and a batch
    permutation that permutes the outputs bit for bit."""
    gen = torch.Generator(device=cuda).manual_seed(B * 13 + L)
    kd = torch.randn((B, 8, L, 128), generator=gen, device=cuda, dtype=torch.float16)
    kd[..., [7, 77]] *= 12
    vd = torch.randn((B, 8, L, 128), generator=gen, device=cuda, dtype=torch.float16)
    kq_, ks = llmik.quantize_per_token(kd)
    vq_, vs = llmik.quantize_per_token(vd)
    del kd, vd
    if live < L:
        kq_[:, :, live:] = 127
        vq_[:, :, live:] = -127
        ks[:, :, live:] = float("nan")
        vs[:, :, live:] = float("inf")
    q = randn((B, 32, 128), B * 17 + L).astype(np.float16)
    qd = _dev(q, cuda)
    scale = 1 / math.sqrt(128)
    out = llmik.decode_attention_int8(qd, kq_, ks, vq_, vs, scale, seqlen=live)
    rows = sorted({0, B // 2, B - 1})
    _sampled_rows_parity(
        out, q,
        lambda b: kq.dequantize_per_token(kq_[b:b + 1, :, :live].cpu().numpy(), ks[b:b + 1, :, :live].cpu().numpy()),
        lambda b: kq.dequantize_per_token(vq_[b:b + 1, :, :live].cpu().numpy(), vs[b:b + 1, :, :live].cpu().numpy()),
        rows, scale)
    assert torch.equal(llmik.decode_attention_int8(qd, kq_, ks, vq_, vs, scale, seqlen=live), out)
    perm = torch.randperm(B, generator=torch.Generator().manual_seed(2)).to(cuda)
    out_p = llmik.decode_attention_int8(qd[perm].contiguous(), kq_[perm].contiguous(), ks[perm].contiguous(),
                                        vq_[perm].contiguous(), vs[perm].contiguous(), scale, seqlen=live)
    assert torch.equal(out_p, out[perm])


@pytest.mark.parametrize("B,L,gs", [(1, 128, 32), (4, 1000, 32), (8, 4096, 128), (2, 100, 128),
                                    (8, 2048, 32), (1, 300, 64),
                                    # groups that are not multiples of 32: the VALU kernel
                                    (2, 300, 16), (3, 500, 48), (1, 200, 100)])
def test_int4_pipeline_matches_oracle(llmik, cuda, B, L, gs):
    q, k, v = _inputs(B, 32, 8, L, seed=7 * L + gs, outliers=True)
    kq_, ks = llmik.quantize_k_per_channel_groupwise_int4(_dev(k, cuda), gs)
    vq_, vs = llmik.quantize_v_per_token_int4(_dev(v, cuda))
    out = llmik.decode_attention_int4(_dev(q, cuda), kq_, ks, vq_, vs, gs, 1 / math.sqrt(128))
    k_dq = kq.dequantize_per_channel_groupwise(kq.unpack_kv_int4(kq_.cpu().numpy()),
                                               ks.cpu().numpy(), gs)
    v_dq = kq.dequantize_per_token(kq.unpack_kv_int4(vq_.cpu().numpy()), vs.cpu().numpy())
    ref = oa.decode_attention(q, k_dq, v_dq, 1 / math.sqrt(128))
    assert _max_abs(out, ref) <= TOL


@pytest.mark.parametrize("fmt", ["int8", "int4g128", "int4g16"])
@pytest.mark.parametrize("B,H,Hkv,L", [(2, 8, 8, 1500),     # MHA: one head per workgroup
                                        (2, 16, 8, 1500),    # GQA 2: two heads per workgroup
                                        (1, 24, 8, 2000)])   # GQA 3: one head, three head chunks
def test_quantised_head_ratios_with_splits(llmik, cuda, fmt, B, H, Hkv, L):
    """INT8 and INT4 at one, two and three query heads per KV head, with the
    sequence split over several workgroups per head chunk (the split
    hand-off's output ownership at one and two heads per workgroup). Group
    16 runs the VALU kernel; 1500 tokens end inside a 128-token group."""
    q, k, v = _inputs(B, H, Hkv, L, seed=H * 100 + L, outliers=True)
    scale = 1 / math.sqrt(128)
    if fmt == "int8":
        kq_, ks = llmik.quantize_per_token(_dev(k, cuda))
        vq_, vs = llmik.quantize_per_token(_dev(v, cuda))
        out = llmik.decode_attention_int8(_dev(q, cuda), kq_, ks, vq_, vs, scale)
        k_dq = kq.dequantize_per_token(kq_.cpu().numpy(), ks.cpu().numpy())
        v_dq = kq.dequantize_per_token(vq_.cpu().numpy(), vs.cpu().numpy())
    else:
        gs = int(fmt[5:])
        kq_, ks = llmik.quantize_k_per_channel_groupwise_int4(_dev(k, cuda), gs)
        vq_, vs = llmik.quantize_v_per_token_int4(_dev(v, cuda))
        out = llmik.decode_attention_int4(_dev(q, cuda), kq_, ks, vq_, vs, gs, scale)
        k_dq = kq.dequantize_per_channel_groupwise(kq.unpack_kv_int4(kq_.cpu().numpy()),
                                                   ks.cpu().numpy(), gs)
        v_dq = kq.dequantize_per_token(kq.unpack_kv_int4(vq_.cpu().numpy()), vs.cpu().numpy())
    assert out.shape == (B, H, 128)
    assert _max_abs(out, oa.decode_attention(q, k_dq, v_dq, scale)) <= TOL


def test_int4_large_batch_config_properties(llmik, cuda):
    """B=64, S=8192 (the second INT4 config): parity on a sample of batches
    (the oracle is run per batch row) and a batch-permutation property."""
    B, L, gs = 64, 8192, 128
    gen = torch.Generator(device=cuda).manual_seed(64)
    kd = torch.randn((B, 8, L, 128), generator=gen, device=cuda, dtype=torch.float16)
    kd[..., [3, 37, 71, 105]] *= 10
    vd = torch.randn((B, 8, L, 128), generator=gen, device=cuda, dtype=torch.float16)
    kq_, ks = llmik.quantize_k_per_channel_groupwise_int4(kd, gs)
    vq_, vs = llmik.quantize_v_per_token_int4(vd)
    del kd, vd
    q = randn((B, 32, 128), 65).astype(np.float16)
    qd = _dev(q, cuda)
    out = llmik.decode_attention_int4(qd, kq_, ks, vq_, vs, gs, 1 / math.sqrt(128))
    for b in (0, 17, 63):
        k_dq = kq.dequantize_per_channel_groupwise(
            kq.unpack_kv_int4(kq_[b:b + 1].cpu().numpy()), ks[b:b + 1].cpu().numpy(), gs)
        v_dq = kq.dequantize_per_token(kq.unpack_kv_int4(vq_[b:b + 1].cpu().numpy()),
                                       vs[b:b + 1].cpu().numpy())
        ref = oa.decode_attention(q[b:b + 1], k_dq, v_dq, 1 / math.sqrt(128))
        assert _max_abs(out[b:b + 1], ref) <= TOL
    perm = torch.randperm(B, generator=torch.Generator().manual_seed(0)).to(cuda)
    out_p = llmik.decode_attention_int4(qd[perm].contiguous(), kq_[perm].contiguous(),
                                        ks[perm].contiguous(), vq_[perm].contiguous(),
                                        vs[perm].contiguous(), gs, 1 / math.sqrt(128))
    assert torch.equal(out_p, out[perm])


def _sampled_rows_parity(out, q, k_rows, v_rows, rows, scale):
    """Oracle parity on the sampled batch rows (the oracle runs per row, in
    float64); k_rows / v_rows give the dequantised [1, Hkv, S, D] of a row."""
    for b in rows:
        ref = oa.decode_attention(q[b:b + 1], k_rows(b), v_rows(b), scale, acc_dtype=np.float64)
        assert _max_abs(out[b:b + 1], ref) <= TOL, f"batch row {b}"


@pytest.mark.parametrize("B,L", [(8, 1024), (8, 16384), (8, 32768), (1, 4096), (64, 4096)])
def test_fp16_swept_baseline_configs(llmik, cuda, B, L):
    """The fp16 sweep configs of the headline shape, each at its exact size:
    B=8 at S=1024 (4-wave workgroups, two per CU), 16384 and 32768 (the
    longest chunks), B=1 at S=4096 (16 eight-wave splits) and B=64 at
    S=4096 (512 four-wave workgroups, no split). Oracle parity on sampled
    batch rows and a batch permutation that must permute the outputs bit for
    bit."""
    gen = torch.Generator(device=cuda).manual_seed(B + L)
    kd = torch.randn((B, 8, L, 128), generator=gen, device=cuda, dtype=torch.float16)
    vd = torch.randn((B, 8, L, 128), generator=gen, device=cuda, dtype=torch.float16)
    q = randn((B, 32, 128), B * 7 + L).astype(np.float16)
    qd = _dev(q, cuda)
    scale = 1 / math.sqrt(128)
    out = llmik.decode_attention(qd, kd, vd, scale)
    _sampled_rows_parity(out, q, lambda b: kd[b:b + 1].cpu().numpy(),
                         lambda b: vd[b:b + 1].cpu().numpy(), sorted({0, max(0, B // 2 - 1), B - 1}), scale)
    perm = torch.randperm(B, generator=torch.Generator().manual_seed(1)).to(cuda)
    out_p = llmik.decode_attention(qd[perm].contiguous(), kd[perm].contiguous(),
                                   vd[perm].contiguous(), scale)
    assert torch.equal(out_p, out[perm])


@pytest.mark.parametrize("B,L", [(8, 16385), (32, 600), (64, 4100)])
def test_fp16_ragged_interleaved_tiles(llmik, cuda, B, L):
    """Ragged lengths under the interleaved tile order (split s, wave w reads
    tiles s + n_splits * (w + NW * i)): B=8, S=16385 (4 splits; the one-token
    last tile falls to split 0, wave 0, its 17th tile), B=32, S=600 (4-wave
    workgroups, no split, a 24-token last tile) and B=64, S=4100 (a 4-token
    last tile). Oracle parity on sampled batch rows."""
    gen = torch.Generator(device=cuda).manual_seed(B * 3 + L)
    kd = torch.randn((B, 8, L, 128), generator=gen, device=cuda, dtype=torch.float16)
    vd = torch.randn((B, 8, L, 128), generator=gen, device=cuda, dtype=torch.float16)
    q = randn((B, 32, 128), B * 11 + L).astype(np.float16)
    scale = 1 / math.sqrt(128)
    out = llmik.decode_attention(_dev(q, cuda), kd, vd, scale)
    _sampled_rows_parity(out, q, lambda b: kd[b:b + 1].cpu().numpy(),
                         lambda b: vd[b:b + 1].cpu().numpy(), (0, B // 2, B - 1), scale)


def _peaked_inputs(B, L, seed):
    """q heads of a kv group share one direction; three tokens of each (b, kv
    head) have keys along it (scores ~12 against ~N(0,1) for the rest), so
    ~95 % of the softmax mass sits on 2-3 near-equal tokens. V has three
    channels x8 (|v| up to ~30)."""
    rng = np.random.default_rng(seed)
    Hkv, G, D = 8, 4, 128
    base = rng.standard_normal((B, Hkv, 1, D))
    q = (base + 0.05 * rng.standard_normal((B, Hkv, G, D))).reshape(B, Hkv * G, D)
    k = rng.standard_normal((B, Hkv, L, D))
    unit = base[:, :, 0] / np.linalg.norm(base[:, :, 0], axis=-1, keepdims=True)
    peaks = (L // 7, L // 2 + 3, L - 2)
    for i, t in enumerate(peaks):
        k[:, :, t] = unit * math.sqrt(D) * (1.05 + 0.002 * i)
    v = rng.standard_normal((B, Hkv, L, D))
    v[..., [5, 50, 90]] *= 8.0
    return q.astype(np.float16), k.astype(np.float16), v.astype(np.float16)


def _half_ulp_f16(x: np.ndarray) -> np.ndarray:
    """Half the fp16 spacing at |x| (the output's own rounding)."""
    a = np.abs(x).astype(np.float16)
    return (np.spacing(a).astype(np.float64)) / 2.0


@pytest.mark.parametrize("fmt", ["fp16", "int8", "int4"])
@pytest.mark.parametrize("B,L", [(2, 4096), (8, 1024)])
def test_peaked_softmax_large_v_precision(llmik, cuda, fmt, B, L):
    """Large-magnitude V under a peaked softmax, all three KV formats: the
    error before the output's fp16 rounding must stay within 2e-3 of the
    float64 attention over the (dequantised) cache, as the reference's fp32
    P does (reference/attention_ref.py:71-80). Rounding P itself to fp16
    would cost ~2^-12 * |v| (~7e-3 here)."""
    q, k, v = _peaked_inputs(B, L, seed=B * 31 + L)
    scale = 1 / math.sqrt(128)
    qd, kd, vd = _dev(q, cuda), _dev(k, cuda), _dev(v, cuda)
    if fmt == "fp16":
        out = llmik.decode_attention(qd, kd, vd, scale)
        k_dq, v_dq = k, v
    elif fmt == "int8":
        kq_, ks = llmik.quantize_per_token(kd)
        vq_, vs = llmik.quantize_per_token(vd)
        out = llmik.decode_attention_int8(qd, kq_, ks, vq_, vs, scale)
        k_dq = kq.dequantize_per_token(kq_.cpu().numpy(), ks.cpu().numpy())
        v_dq = kq.dequantize_per_token(vq_.cpu().numpy(), vs.cpu().numpy())
    else:
        gs = 32
        kq_, ks = llmik.quantize_k_per_channel_groupwise_int4(kd, gs)
        vq_, vs = llmik.quantize_v_per_token_int4(vd)
        out = llmik.decode_attention_int4(qd, kq_, ks, vq_, vs, gs, scale)
        k_dq = kq.dequantize_per_channel_groupwise(kq.unpack_kv_int4(kq_.cpu().numpy()),
                                                   ks.cpu().numpy(), gs)
        v_dq = kq.dequantize_per_token(kq.unpack_kv_int4(vq_.cpu().numpy()), vs.cpu().numpy())
    ref = oa.decode_attention(q, k_dq, v_dq, scale, acc_dtype=np.float64)
    assert np.abs(ref).max() > 8.0, "the case must produce large outputs"
    err = np.abs(out.double().cpu().numpy() - ref) - _half_ulp_f16(ref)
    assert float(err.max()) <= TOL


def test_int4_long_unsplit_large_v(llmik, cuda):
    """INT4 at B=64, S=8192 runs without splits (2048 tokens per wave), so each
    wave's PV accumulator sums 64 tiles. V has three channels x8: the error
    before output rounding stays within 2e-3 of float64 attention (a biased V
    operand whose bias dwarfs the codes would lose ~2e-3 here)."""
    B, L, gs = 64, 8192, 128
    gen = torch.Generator(device=cuda).manual_seed(640)
    kd = torch.randn((B, 8, L, 128), generator=gen, device=cuda, dtype=torch.float16)
    kd[..., [3, 37, 71, 105]] *= 10
    vd = torch.randn((B, 8, L, 128), generator=gen, device=cuda, dtype=torch.float16)
    vd[..., [5, 50, 90]] *= 8
    kq_, ks = llmik.quantize_k_per_channel_groupwise_int4(kd, gs)
    vq_, vs = llmik.quantize_v_per_token_int4(vd)
    del kd, vd
    q = randn((B, 32, 128), 641).astype(np.float16)
    out = llmik.decode_attention_int4(_dev(q, cuda), kq_, ks, vq_, vs, gs, 1 / math.sqrt(128))
    for b in (0, 63):
        k_dq = kq.dequantize_per_channel_groupwise(
            kq.unpack_kv_int4(kq_[b:b + 1].cpu().numpy()), ks[b:b + 1].cpu().numpy(), gs)
        v_dq = kq.dequantize_per_token(kq.unpack_kv_int4(vq_[b:b + 1].cpu().numpy()),
                                       vs[b:b + 1].cpu().numpy())
        ref = oa.decode_attention(q[b:b + 1], k_dq, v_dq, 1 / math.sqrt(128), acc_dtype=np.float64)
        err = np.abs(out[b:b + 1].double().cpu().numpy() - ref) - _half_ulp_f16(ref)
        assert float(err.max()) <= TOL, f"batch row {b}"
