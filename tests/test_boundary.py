"""The C ABI boundary and the llmik_cuda host layer, on the CPU.

* libllmik_hip.so loads and exports every entry point include/llmik.h
  declares, with the ABI version the host layer expects; the measurement
  floors of include/llmik_diag.h live in libllmik_diag.so alone;
* the C layer rejects bad arguments with LLMIK_ERR_* codes and messages
  before touching the GPU (null / misaligned pointers, head_dim != 128,
  seqlen > kv_buf_len, K / group_size rules);
* the Python layer raises RuntimeError with the reference binding's
  TORCH_CHECK messages (bindings/extension.cpp), for every validation path
  the reference has, without launching anything;
* the op surface has the reference's names, argument order and defaults.
No test here calls a compute entry point with valid arguments.
"""
from __future__ import annotations

import ctypes
import inspect
import re

import pytest
import torch

from tests.helpers import ROOT

HEADER = ROOT / "include" / "llmik.h"
DIAG_HEADER = ROOT / "include" / "llmik_diag.h"


def declared_symbols(header=HEADER):
    text = header.read_text()
    return sorted(set(re.findall(r"LLMIK_API\s+[\w\s\*]+?\b(llmik_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def mod():
    import llmik_cuda
    return llmik_cuda


@pytest.fixture(scope="module")
def lib(mod):
    from llmik_cuda._lib import lib
    return lib


def test_header_declares_expected_entry_points():
    syms = declared_symbols()
    for name in ["llmik_decode_attention_f16", "llmik_decode_attention_int8",
                 "llmik_decode_attention_int4", "llmik_quantize_per_token_int8",
                 "llmik_quantize_k_per_channel_groupwise_int4", "llmik_quantize_v_per_token_int4",
                 "llmik_w4a16_gemm", "llmik_w4a16_dequantize", "llmik_rmsnorm", "llmik_silu_mul",
                 "llmik_rope", "llmik_attention_workspace_size", "llmik_w4a16_workspace_size"]:
        assert name in syms


def test_library_exports_every_declared_symbol(lib):
    for name in declared_symbols():
        assert hasattr(lib, name), name
    assert lib.llmik_abi_version() == 1


def test_library_was_built_for_gfx950_only():
    from llmik_cuda._lib import DIAG_LIB_PATH, LIB_PATH
    for path in (LIB_PATH, DIAG_LIB_PATH):
        data = path.read_bytes()
        assert b"gfx950" in data
        for other in (b"gfx942", b"gfx90a", b"gfx1100"):
            assert other not in data


def test_measurement_floors_live_in_their_own_library(lib):
    from llmik_cuda._lib import diag_lib
    diag = diag_lib()
    names = declared_symbols(DIAG_HEADER)
    assert {"llmik_diag_empty", "llmik_diag_read", "llmik_diag_read_write", "llmik_diag_last_error"} <= set(names)
    for name in names:
        assert hasattr(diag, name), name
        assert not hasattr(lib, name), f"{name} is exported by the product library"
    # argument checks come before any HIP call
    assert diag.llmik_diag_read(None, 100, None, 1, 4, None) != 0
    assert "multiple of 16" in diag.llmik_diag_last_error().decode()
    assert diag.llmik_diag_read_write(16, 64, 16, 5, 1, 4, None) != 0
    assert "write_bytes_per_16" in diag.llmik_diag_last_error().decode()
    assert diag.llmik_diag_empty(0, None) != 0
    assert "n_workgroups" in diag.llmik_diag_last_error().decode()


def _err(lib):
    return lib.llmik_last_error().decode()


def test_c_layer_argument_errors(lib):
    S = None
    st = lib.llmik_decode_attention_f16(16, 16, 16, 16, 1, 32, 8, 10, 64, 10, 1.0, None, 0, S)
    assert st == -1 and "head_dim=128" in _err(lib)
    st = lib.llmik_decode_attention_f16(16, 16, 16, 16, 1, 32, 8, 11, 128, 10, 1.0, None, 0, S)
    assert st == -1 and "seqlen exceeds" in _err(lib)
    st = lib.llmik_decode_attention_f16(16, 16, 16, 16, 1, 30, 8, 10, 128, 10, 1.0, None, 0, S)
    assert st == -1 and "multiple of n_kv_heads" in _err(lib)
    st = lib.llmik_decode_attention_f16(17, 16, 16, 16, 1, 32, 8, 10, 128, 10, 1.0, None, 0, S)
    assert st == -4
    st = lib.llmik_decode_attention_int4(16, 16, 16, 16, 16, 16, 1, 32, 8, 100, 128, 100, 32, 3,
                                         1.0, None, 0, S)
    assert st == -1 and "fewer groups" in _err(lib)
    st = lib.llmik_quantize_per_token_int8(16, 16, 16, 1, 8, 4, 64, S)
    assert st == -1 and "head_dim=128" in _err(lib)
    st = lib.llmik_quantize_k_per_channel_groupwise_int4(16, 16, 16, 1, 8, 4, 128, 0, S)
    assert st == -1 and "group_size must be positive" in _err(lib)
    st = lib.llmik_w4a16_gemm(16, 16, 16, 16, 1, 64, 100, 100, None, 0, S)
    assert st == -1 and "K_packs * 8" in _err(lib)
    st = lib.llmik_w4a16_gemm(16, 16, 16, 16, 1, 64, 128, 12, None, 0, S)
    assert st == -1 and "multiple of 8" in _err(lib)
    st = lib.llmik_w4a16_gemm(16, 16, 16, 16, 1, 64, 128, 48, None, 0, S)
    assert st == -1 and "n_groups * group_size" in _err(lib)
    st = lib.llmik_rope(16, 16, 16, 16, 1, 1, 1, 7, S)
    assert st == -1 and "even" in _err(lib)
    st = lib.llmik_quantize_weights_int4_groupwise(16, 0, 96, 40, 12, None, 16, 16, None, S)
    assert st == -1 and "multiples of 8" in _err(lib)
    st = lib.llmik_quantize_weights_int4_groupwise(16, 0, 64, 40, 0, 16, None, 16, None, S)
    assert st == -1 and "group_size must be positive" in _err(lib)
    st = lib.llmik_quantize_weights_int4_groupwise(18, 0, 64, 40, 32, 16, None, 16, None, S)
    assert st == -4
    st = lib.llmik_pack_int4_along_k(16, 12, 40, 16, S)
    assert st == -1 and "multiple of 8" in _err(lib)
    kivi = (16, 1, 16, 1, 16, 16, 16, 16, 16, 1, 8)    # k .. v_scale, batch, n_kv_heads
    st = lib.llmik_kivi_append_token_int4(*kivi, 128, 64, 32, 64, S)
    assert st == -1 and "full" in _err(lib)
    st = lib.llmik_kivi_append_token_int4(*kivi, 128, 512, 256, 64, S)
    assert st == -1 and "1..128" in _err(lib)
    st = lib.llmik_kivi_append_token_int4(*kivi, 64, 64, 32, 0, S)
    assert st == -1 and "head_dim=128" in _err(lib)
    st = lib.llmik_rope_qkv_append_f16(16, 16, 16, 16, 16, 16, 2, 4, 2, 128, 8, 8, S)
    assert st == -1 and "pos outside" in _err(lib)
    st = lib.llmik_rope_qkv_append_f16(16, 16, 16, 16, 16, 16, 2, 4, 2, 9, 8, 0, S)
    assert st == -1 and "even" in _err(lib)
    st = lib.llmik_add_rmsnorm(16, 16, 16, 16, 16, 2, 8200, 1e-5, S)
    assert st == -1 and "at most 8192" in _err(lib)
    st = lib.llmik_add_rmsnorm(16, 16, 16, 16, 18, 2, 4096, 1e-5, S)
    assert st == -4
    st = lib.llmik_silu_mul_halves(16, 16, 2, 12, S)
    assert st == -1 and "multiple of 8" in _err(lib)


def test_workspace_sizes_without_gpu(lib):
    assert lib.llmik_attention_workspace_size(8, 32, 8, 4096, 128) > 0
    assert lib.llmik_attention_workspace_size(8, 32, 8, 4096, 64) == 0
    # Split-K plans need the counter region plus one fp32 partial per split
    # and output; a plan without splits needs none.
    for M, N, K, gs in [(1, 4096, 4096, 128), (1, 4096, 4096, 16), (16, 4096, 4096, 128),
                        (1, 14336, 4096, 128)]:
        ws = lib.llmik_w4a16_workspace_size(M, N, K, gs)
        assert ws == 0 or (ws >= 16384 + M * N * 4 * 2 and ws % 256 == 0)
    assert lib.llmik_w4a16_workspace_size(1, 4096, 4096, 16) > 0


@pytest.mark.parametrize("M,N,K,gs,rest,splits", [
    (768, 14336, 1024, 128, 80, 3),    # 336 tiles: 256 unsplit, 80 in 3 K splits
    (2048, 14336, 4096, 128, 128, 2),  # 896 tiles: 768 unsplit, 128 in 2
    (3072, 14336, 1024, 32, 64, 4),    # 1344 tiles: 1280 unsplit, 64 in 4 (group 32)
    (768, 4096, 14336, 128, 96, 2),    # 96 tiles, each in 2 splits
    (1024, 14336, 4096, 128, 0, 1),    # 448 tiles: splitting the 192 left costs more
    (2048, 4096, 4096, 128, 0, 1),     # 256 tiles, one round
])
def test_lds_gemm_plans_without_gpu(lib, M, N, K, gs, rest, splits):
    """The 256 x 128-tile W4A16 GEMM's plan on 256 CUs (the CU count the
    library assumes without a device): tiles in whole rounds of the CUs run
    unsplit, the rest split K when the round-cost model says so; the
    workspace holds the counters and one 256 x 128 fp32 partial per split
    tile and split."""
    ws = lib.llmik_w4a16_workspace_size(M, N, K, gs)
    part = rest * splits * 256 * 128 * 4
    assert ws == (16384 + (part + 255) // 256 * 256 if splits > 1 else 0)


def test_op_surface_matches_reference(mod):
    expect = {
        "decode_attention": ["q", "k", "v", "softmax_scale", "seqlen"],
        "decode_attention_v3": ["q", "k", "v", "softmax_scale"],
        "quantize_per_token": ["x"],
        "decode_attention_int8": ["q", "k_q", "k_scale", "v_q", "v_scale", "softmax_scale"],
        "quantize_k_per_channel_groupwise_int4": ["x", "group_size"],
        "quantize_v_per_token_int4": ["x"],
        "decode_attention_int4": ["q", "k_q", "k_scale", "v_q", "v_scale", "group_size",
                                  "softmax_scale"],
        "w4a16_gemm": ["act", "weight_packed", "scale", "group_size"],
        "w4a16_dequantize": ["weight_packed", "scale", "group_size"],
        "rmsnorm": ["x", "weight", "eps"],
        "silu_mul": ["gate", "up"],
        "rope": ["x", "cos", "sin"],
    }
    for name, params in expect.items():
        sig = inspect.signature(getattr(mod, name))
        got = list(sig.parameters)
        assert got[:len(params)] == params, name
        for extra in got[len(params):]:
            assert sig.parameters[extra].default is not inspect.Parameter.empty, (name, extra)
    assert inspect.signature(mod.decode_attention).parameters["seqlen"].default == -1


H16 = torch.float16


def _t(*shape, dtype=H16):
    return torch.zeros(*shape, dtype=dtype)


@pytest.fixture
def as_device(mod, monkeypatch):
    """Treat CPU tensors as device tensors so the later checks are reachable;
    every case below must raise before any launch."""
    monkeypatch.setattr(mod, "_is_device", lambda t: True)
    return mod


def test_python_checks_device_first(mod):
    with pytest.raises(RuntimeError, match="q, k, v must be CUDA tensors"):
        mod.decode_attention(_t(1, 32, 128), _t(1, 8, 4, 128), _t(1, 8, 4, 128), 0.1)
    with pytest.raises(RuntimeError, match="x must be CUDA"):
        mod.quantize_per_token(_t(1, 8, 4, 128))
    with pytest.raises(RuntimeError, match="all inputs must be CUDA tensors"):
        mod.w4a16_gemm(_t(1, 64), _t(8, 16, dtype=torch.int32), _t(1, 16), 64)


@pytest.mark.parametrize("case", [
    ("decode_attention", lambda m: m.decode_attention(_t(1, 32, 128, dtype=torch.float32),
                                                      _t(1, 8, 4, 128), _t(1, 8, 4, 128), 0.1),
     "fp16 only for now"),
    ("decode_attention", lambda m: m.decode_attention(_t(1, 32, 128), _t(1, 8, 4, 128).transpose(2, 3),
                                                      _t(1, 8, 4, 128), 0.1),
     "inputs must be contiguous"),
    ("decode_attention", lambda m: m.decode_attention(_t(1, 32, 128), _t(1, 8, 4, 128),
                                                      _t(1, 8, 4, 128), 0.1, 5),
     "seqlen exceeds allocated cache length"),
    ("quantize_per_token", lambda m: m.quantize_per_token(_t(1, 8, 4, 128, dtype=torch.float32)),
     "x must be fp16"),
    ("quantize_per_token", lambda m: m.quantize_per_token(_t(8, 4, 128)),
     r"x must be \[batch, n_kv_heads, seqlen, head_dim\]"),
    ("quantize_per_token", lambda m: m.quantize_per_token(_t(1, 8, 4, 64)),
     "only head_dim=128 supported"),
    ("quantize_k", lambda m: m.quantize_k_per_channel_groupwise_int4(_t(1, 8, 4, 128), 0),
     "group_size must be positive"),
    ("quantize_v", lambda m: m.quantize_v_per_token_int4(_t(1, 8, 4, 128)[:, :, :, ::2]),
     "x must be contiguous"),
    ("int8", lambda m: m.decode_attention_int8(_t(1, 32, 128), _t(1, 8, 4, 128), _t(1, 8, 4),
                                               _t(1, 8, 4, 128), _t(1, 8, 4), 0.1),
     "k_q and v_q must be int8"),
    ("int8", lambda m: m.decode_attention_int8(_t(1, 32, 128), _t(1, 8, 4, 128, dtype=torch.int8),
                                               _t(1, 8, 4, dtype=torch.float32),
                                               _t(1, 8, 4, 128, dtype=torch.int8), _t(1, 8, 4), 0.1),
     "k_scale and v_scale must be fp16"),
    ("int4", lambda m: m.decode_attention_int4(_t(1, 32, 128), _t(1, 8, 4, 64),
                                               _t(1, 8, 1, 128), _t(1, 8, 4, 64), _t(1, 8, 4), 32, 0.1),
     r"k_q and v_q must be int8 \(packed int4\)"),
    ("gemm", lambda m: m.w4a16_gemm(_t(1, 64, dtype=torch.float32), _t(8, 16, dtype=torch.int32),
                                    _t(1, 16), 64), "act must be fp16"),
    ("gemm", lambda m: m.w4a16_gemm(_t(1, 64), _t(8, 16), _t(1, 16), 64),
     r"weight_packed must be int32 \(uint32 bit pattern\)"),
    ("gemm", lambda m: m.w4a16_gemm(_t(1, 72), _t(8, 16, dtype=torch.int32), _t(1, 16), 64),
     "act.K must equal weight_packed.K_packs"),
    ("gemm", lambda m: m.w4a16_gemm(_t(1, 64), _t(8, 16, dtype=torch.int32), _t(1, 8), 64),
     "scale and weight_packed N mismatch"),
    ("gemm", lambda m: m.w4a16_gemm(_t(1, 64), _t(8, 16, dtype=torch.int32), _t(1, 16), 12),
     "group_size must be a positive multiple of 8"),
    ("gemm", lambda m: m.w4a16_gemm(_t(1, 64), _t(8, 16, dtype=torch.int32), _t(2, 16), 64),
     "K must equal n_groups \\* group_size"),
    ("gemm", lambda m: m.w4a16_gemm(_t(64), _t(8, 16, dtype=torch.int32), _t(1, 16), 64),
     "all inputs must be 2D"),
    ("dequant", lambda m: m.w4a16_dequantize(_t(8, 16, dtype=torch.int32), _t(1, 16), 48),
     "K must be a multiple of group_size"),
    ("rmsnorm", lambda m: m.rmsnorm(_t(2, 64), _t(32), 1e-5), "weight length must match"),
    ("silu", lambda m: m.silu_mul(_t(2, 64), _t(2, 32)), "gate and up must have the same shape"),
    ("rope", lambda m: m.rope(_t(2, 4, 1, 7), _t(2, 1, 7), _t(2, 1, 7)), "head_dim must be even"),
    ("rope", lambda m: m.rope(_t(2, 4, 3, 8), _t(2, 8), _t(2, 8)), "cos/sin must be"),
])
def test_python_validation_messages(as_device, case):
    _, call, msg = case
    with pytest.raises(RuntimeError, match=msg):
        call(as_device)


def test_weight_quantiser_validation(mod, as_device):
    """The GPU weight quantiser / packer mirror the reference functions'
    arguments; the packer's K % 8 check is the reference's assertion
    (reference/quant_matmul_ref.py:157)."""
    with pytest.raises(RuntimeError, match="W must be fp16 or fp32"):
        mod.quantize_weights_int4_groupwise(_t(64, 8, dtype=torch.int32), 32)
    with pytest.raises(RuntimeError, match="group_size must be positive"):
        mod.quantize_weights_int4_groupwise(_t(64, 8), 0)
    with pytest.raises(RuntimeError, match=r"W must be 2D \[K, N\]"):
        mod.quantize_weights_int4_groupwise(_t(64), 32)
    with pytest.raises(AssertionError, match="K=12 must be a multiple of 8"):
        mod.pack_int4_along_k(_t(12, 4, dtype=torch.int8))
    with pytest.raises(AssertionError, match="K=12 must be a multiple of 8"):
        mod.quantize_pack_weights_int4(_t(12, 4), 4)
    sig = inspect.signature(mod.quantize_weights_int4_groupwise)
    assert list(sig.parameters) == ["W", "group_size"] and sig.parameters["group_size"].default == 128
    assert list(inspect.signature(mod.pack_int4_along_k).parameters) == ["q_int8"]


# ------------------------------------------------------- in-place KV writers

def test_c_layer_in_place_writer_errors(lib):
    S = None
    # x_len 4 < n_tok 5
    st = lib.llmik_quantize_per_token_int8_into(16, 4, 16, 16, 1, 8, 5, 128, 64, 0, S)
    assert st == -1 and "n_tok exceeds" in _err(lib)
    # offset 60 + 5 > cache_len 64
    st = lib.llmik_quantize_v_per_token_int4_into(16, 8, 16, 16, 1, 8, 5, 128, 64, 60, S)
    assert st == -1 and "exceeds the cache length" in _err(lib)
    st = lib.llmik_quantize_per_token_int8_into(16, 8, 16, 16, 1, 8, 5, 64, 64, 0, S)
    assert st == -1 and "head_dim=128" in _err(lib)
    # K groupwise: offset not on a group boundary
    st = lib.llmik_quantize_k_per_channel_groupwise_int4_into(16, 8, 16, 16, 1, 8, 5, 128, 64, 16,
                                                              32, S)
    assert st == -1 and "multiple of group_size" in _err(lib)
    st = lib.llmik_quantize_k_per_channel_groupwise_int4_into(16, 8, 16, 16, 1, 8, 5, 128, 64, 0,
                                                              0, S)
    assert st == -1 and "group_size must be positive" in _err(lib)
    st = lib.llmik_quantize_per_token_int8_into(16, 8, 20, 16, 1, 8, 5, 128, 64, 0, S)
    assert st == -4   # q not 8-byte aligned


@pytest.mark.parametrize("case", [
    (lambda m: m.quantize_per_token_into(_t(1, 8, 4, 128), _t(1, 8, 16, 128), _t(1, 8, 16), 0),
     "q_cache must be int8 and scale_cache fp16"),
    (lambda m: m.quantize_per_token_into(_t(1, 8, 4, 128), _t(1, 8, 16, 128, dtype=torch.int8),
                                         _t(1, 8, 16), 13), "offset \\+ n exceeds the cache length"),
    (lambda m: m.quantize_per_token_into(_t(1, 8, 4, 128), _t(1, 8, 16, 64, dtype=torch.int8),
                                         _t(1, 8, 16), 0), r"q_cache must be \[batch"),
    (lambda m: m.quantize_per_token_into(_t(1, 8, 4, 128), _t(1, 8, 16, 128, dtype=torch.int8),
                                         _t(1, 8, 15), 0), "scale_cache must be"),
    (lambda m: m.quantize_v_per_token_int4_into(_t(1, 8, 8, 128)[:, :, ::2],
                                                _t(1, 8, 16, 64, dtype=torch.int8), _t(1, 8, 16), 0),
     "contiguous within each"),
    (lambda m: m.quantize_k_per_channel_groupwise_int4_into(
        _t(1, 8, 4, 128), _t(1, 8, 64, 64, dtype=torch.int8), _t(1, 8, 2, 128), 16, 32),
     "offset must be a multiple of group_size"),
    (lambda m: m.quantize_k_per_channel_groupwise_int4_into(
        _t(1, 8, 4, 128), _t(1, 8, 64, 64, dtype=torch.int8), _t(1, 8, 3, 128), 0, 32),
     r"scale_cache must be \[batch, n_kv_heads, ceil"),
])
def test_python_in_place_writer_validation(as_device, case):
    call, msg = case
    with pytest.raises(RuntimeError, match=msg):
        call(as_device)


def test_token_row_stride_of_slices(mod):
    buf = torch.zeros(2, 3, 40, 128, dtype=torch.float16)
    assert mod._token_rows(buf) == 40
    assert mod._token_rows(buf[:, :, 5:17]) == 40
    assert mod._token_rows(buf[:1, :1, :7]) == 7
    assert mod._token_rows(buf[:, :1, 3:9]) == 120   # rows of one head: batch stride
    with pytest.raises(RuntimeError):
        mod._token_rows(buf[:, ::2])   # unequally spaced rows (3 heads, stride 2)


# ------------------------------------------- decode-step merges and KIVI append

@pytest.mark.parametrize("case", [
    (lambda m: m.rope_qkv_append(_t(2, 6 * 128), _t(128), _t(128), _t(2, 2, 4, 128), _t(2, 2, 4, 128), 4),
     "pos outside the cache"),
    (lambda m: m.rope_qkv_append(_t(2, 4 * 128), _t(128), _t(128), _t(2, 2, 4, 128), _t(2, 2, 4, 128), 0),
     "fewer than 2 n_kv_heads"),
    (lambda m: m.rope_qkv_append(_t(2, 6 * 128), _t(64), _t(64), _t(2, 2, 4, 128), _t(2, 2, 4, 128), 0),
     "one \\[head_dim\\] row"),
    (lambda m: m.rope_qkv_append(_t(2, 6 * 128), _t(128), _t(128), _t(2, 2, 4, 128),
                                 _t(2, 2, 4, 128, dtype=torch.float32), 0), "fp16 only"),
    (lambda m: m.add_rmsnorm(_t(2, 64), _t(2, 32), _t(64), 1e-5), "same shape"),
    (lambda m: m.add_rmsnorm(_t(2, 64), _t(2, 64), _t(32), 1e-5), "weight length"),
    (lambda m: m.silu_mul_halves(_t(2, 24)), "multiple of 8"),
    (lambda m: m.kivi_append_token_int4(_t(1, 8, 1, 128), _t(1, 8, 1, 128), _t(1, 8, 16, 128),
                                        _t(1, 8, 64, 64, dtype=torch.int8), _t(1, 8, 2, 128),
                                        _t(1, 8, 64, 64, dtype=torch.int8), _t(1, 8, 64), 5, 32),
     "k_open must be"),
    (lambda m: m.kivi_append_token_int4(_t(1, 8, 1, 128), _t(1, 8, 1, 128), _t(1, 8, 32, 128),
                                        _t(1, 8, 64, 64, dtype=torch.int8), _t(1, 8, 2, 128, dtype=torch.float32),
                                        _t(1, 8, 64, 64, dtype=torch.int8), _t(1, 8, 64), 5, 32),
     "must be fp16"),
])
def test_python_merge_and_append_validation(as_device, case):
    fn, msg = case
    with pytest.raises(RuntimeError, match=msg):
        fn(as_device)


def test_merges_check_device_first(mod):
    with pytest.raises(RuntimeError, match="inputs must be CUDA"):
        mod.add_rmsnorm(_t(2, 64), _t(2, 64), _t(64), 1e-5)
    with pytest.raises(RuntimeError, match="all inputs must be CUDA tensors"):
        mod.kivi_append_token_int4(_t(1, 8, 1, 128), _t(1, 8, 1, 128), _t(1, 8, 32, 128),
                                   _t(1, 8, 64, 64, dtype=torch.int8), _t(1, 8, 2, 128),
                                   _t(1, 8, 64, 64, dtype=torch.int8), _t(1, 8, 64), 5, 32)
