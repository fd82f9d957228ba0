"""Loader and ctypes signatures for libllmik_hip.so (include/llmik.h).

The library is loaded after torch so that it binds to the HIP runtime torch
already mapped (both carry the soname libamdhip64.so.7). A missing library
is an ImportError: there is no fallback path.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime first)

# Always the in-package library: _C links this same file (through an $ORIGIN
# rpath), so the dynamic loader maps one copy and ctypes calls (plan
# overrides, the last-error text, the no-alloc scratch) reach the state the
# ops use.
LIB_PATH = Path(__file__).resolve().parent / "libllmik_hip.so"

if not LIB_PATH.exists():
    raise ImportError(
        f"llmik_cuda: {LIB_PATH} is missing. Build it with "
        "`python llm-inference-kernels_amd/build_lib.py` (or __graft_entry__.build()).")

lib = ctypes.CDLL(str(LIB_PATH))

_p = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float
_sz = ctypes.c_size_t
_l = ctypes.c_long

_SIGNATURES = {
    "llmik_last_error": (ctypes.c_char_p, []),
    "llmik_abi_version": (_i, []),
    "llmik_attention_workspace_size": (_sz, [_i, _i, _i, _i, _i]),
    "llmik_decode_attention_f16": (_i, [_p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _f, _p, _sz, _p]),
    "llmik_decode_attention_f16_noalloc": (_i, [_p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _f, _p]),
    "llmik_decode_attention_int8": (
        _i, [_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _f, _p, _sz, _p]),
    "llmik_decode_attention_int4": (
        _i, [_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i, _i, _f, _p, _sz, _p]),
    "llmik_quantize_per_token_int8": (_i, [_p, _p, _p, _i, _i, _i, _i, _p]),
    "llmik_quantize_k_per_channel_groupwise_int4": (_i, [_p, _p, _p, _i, _i, _i, _i, _i, _p]),
    "llmik_quantize_v_per_token_int4": (_i, [_p, _p, _p, _i, _i, _i, _i, _p]),
    "llmik_quantize_per_token_int8_into": (_i, [_p, _i, _p, _p, _i, _i, _i, _i, _i, _i, _p]),
    "llmik_quantize_v_per_token_int4_into": (_i, [_p, _i, _p, _p, _i, _i, _i, _i, _i, _i, _p]),
    "llmik_quantize_k_per_channel_groupwise_int4_into": (
        _i, [_p, _i, _p, _p, _i, _i, _i, _i, _i, _i, _i, _p]),
    "llmik_kivi_append_token_int4": (
        _i, [_p, _i, _p, _i, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _p]),
    "llmik_w4a16_workspace_size": (_sz, [_i, _i, _i, _i]),
    "llmik_w4a16_gemm": (_i, [_p, _p, _p, _p, _i, _i, _i, _i, _p, _sz, _p]),
    "llmik_w4a16_gemm_f32out": (_i, [_p, _p, _p, _p, _i, _i, _i, _i, _p, _sz, _p]),
    "llmik_w4a16_dequantize": (_i, [_p, _p, _p, _i, _i, _i, _p]),
    "llmik_w4a16_set_plan_override": (None, [_i, _i]),
    "llmik_attention_set_plan_override": (None, [_i]),
    "llmik_w4a16_swiglu_workspace_size": (_sz, [_i, _i, _i, _i]),
    "llmik_w4a16_gemm_swiglu": (_i, [_p, _p, _p, _p, _i, _i, _i, _i, _p, _sz, _p]),
    "llmik_w4a16_qkv_rope_workspace_size": (_sz, [_i, _i, _i, _i, _i]),
    "llmik_w4a16_gemm_qkv_rope_f16": (
        _i, [_p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i, _p, _sz, _p]),
    "llmik_quantize_weights_int4_groupwise": (_i, [_p, _i, _i, _i, _i, _p, _p, _p, _p, _p]),
    "llmik_pack_int4_along_k": (_i, [_p, _i, _i, _p, _p]),
    "llmik_rmsnorm": (_i, [_p, _p, _p, _i, _i, _f, _p]),
    "llmik_silu_mul": (_i, [_p, _p, _p, _l, _p]),
    "llmik_rope": (_i, [_p, _p, _p, _p, _i, _i, _i, _i, _p]),
    "llmik_rope_qkv_append_f16": (_i, [_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _p]),
    "llmik_add_rmsnorm": (_i, [_p, _p, _p, _p, _p, _i, _i, _f, _p]),
    "llmik_silu_mul_halves": (_i, [_p, _p, _l, _i, _p]),
}

for _name, (_res, _args) in _SIGNATURES.items():
    _fn = getattr(lib, _name)
    _fn.restype = _res
    _fn.argtypes = _args

ABI_VERSION = 1
if lib.llmik_abi_version() != ABI_VERSION:
    raise ImportError(f"llmik_cuda: {LIB_PATH} has ABI {lib.llmik_abi_version()}, "
                      f"expected {ABI_VERSION}; rebuild it")


def check(status: int) -> None:
    """Raise RuntimeError for a non-zero llmik_status."""
    if status != 0:
        msg = lib.llmik_last_error().decode(errors="replace")
        raise RuntimeError(f"llmik: {msg} (status {status})")


# The measurement floors (include/llmik_diag.h) live in a library of their
# own; only bench.py --floors and their tests load it.
DIAG_LIB_PATH = LIB_PATH.parent / "libllmik_diag.so"
_DIAG_SIGNATURES = {
    "llmik_diag_last_error": (ctypes.c_char_p, []),
    "llmik_diag_empty": (_i, [_i, _p]),
    "llmik_diag_read": (_i, [_p, _sz, _p, _i, _i, _p]),
    "llmik_diag_read_write": (_i, [_p, _sz, _p, _i, _i, _i, _p]),
}
_diag = None


def diag_lib():
    """libllmik_diag.so with its signatures set (loaded on first use)."""
    global _diag
    if _diag is None:
        if not DIAG_LIB_PATH.exists():
            raise ImportError(f"llmik_cuda: {DIAG_LIB_PATH} is missing; build it with "
                              "`python llm-inference-kernels_amd/build_lib.py`")
        d = ctypes.CDLL(str(DIAG_LIB_PATH))
        for name, (res, args) in _DIAG_SIGNATURES.items():
            fn = getattr(d, name)
            fn.restype = res
            fn.argtypes = args
        _diag = d
    return _diag


def diag_check(status: int) -> None:
    """check() for the entry points of libllmik_diag.so."""
    if status != 0:
        msg = diag_lib().llmik_diag_last_error().decode(errors="replace")
        raise RuntimeError(f"llmik_diag: {msg} (status {status})")
