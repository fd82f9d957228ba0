"""CPU: the transformers 5 integration (llmik_cuda.hf) — registration, the
attention function's call signature, its fallback to transformers' SDPA
path off the GPU (so a CPU model gives the stock logits), the cat-free
PreallocCache against DynamicCache, and the buffer-view detection the
decode path relies on. The kernels themselves run in
tests/test_gpu_hf_integration.py."""
from __future__ import annotations

import inspect

import numpy as np
import pytest
import torch

transformers = pytest.importorskip("transformers")

from oracle import kv_quant as kq  # noqa: E402


@pytest.fixture(scope="module")
def hf():
    from llmik_cuda import hf as mod
    mod.register()
    return mod


def _tiny_llama(attn: str, seed: int = 0):
    from transformers import LlamaConfig, LlamaForCausalLM
    cfg = LlamaConfig(hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=2, num_key_value_heads=1, head_dim=128, vocab_size=128,
                      max_position_embeddings=256)
    torch.manual_seed(seed)
    m = LlamaForCausalLM(cfg).eval()
    m.set_attn_implementation(attn)
    return m


def test_register_adds_attention_and_mask(hf):
    from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    assert hf.register() == "llmik"
    assert ALL_ATTENTION_FUNCTIONS["llmik"] is hf.llmik_attention_forward
    assert "llmik" in ALL_MASK_ATTENTION_FUNCTIONS


def test_attention_function_signature_matches_sdpa(hf):
    from transformers.integrations.sdpa_attention import sdpa_attention_forward
    ours = list(inspect.signature(hf.llmik_attention_forward).parameters)
    ref = list(inspect.signature(sdpa_attention_forward).parameters)
    assert ours[:5] == ref[:5] == ["module", "query", "key", "value", "attention_mask"]
    assert "scaling" in ours and "dropout" in ours and ours[-1] == "kwargs"


def _run(model, cache, prompt, steps):
    logits = []
    with torch.no_grad():
        out = model(input_ids=prompt, past_key_values=cache, use_cache=True)
        logits.append(out.logits[:, -1])
        for t in steps:
            out = model(input_ids=t, past_key_values=cache, use_cache=True)
            logits.append(out.logits[:, -1])
    return torch.stack(logits)


def test_cpu_model_falls_back_to_sdpa_exactly(hf):
    from transformers import DynamicCache
    g = torch.Generator().manual_seed(1)
    prompt = torch.randint(0, 128, (2, 9), generator=g)
    steps = [torch.randint(0, 128, (2, 1), generator=g) for _ in range(3)]
    a = _run(_tiny_llama("sdpa"), DynamicCache(), prompt, steps)
    b = _run(_tiny_llama("llmik"), DynamicCache(), prompt, steps)
    assert torch.equal(a, b)


def test_prealloc_cache_matches_dynamic_cache(hf):
    from transformers import DynamicCache
    g = torch.Generator().manual_seed(2)
    prompt = torch.randint(0, 128, (2, 11), generator=g)
    steps = [torch.randint(0, 128, (2, 1), generator=g) for _ in range(4)]
    model = _tiny_llama("sdpa")
    a = _run(model, DynamicCache(), prompt, steps)
    cache = hf.PreallocCache(max_len=32)
    b = _run(model, cache, prompt, steps)
    assert torch.allclose(a, b, atol=1e-5, rtol=1e-5)
    assert cache.get_seq_length() == 15
    assert cache.layers[0].keys.shape == (2, 1, 32, 128)


def test_prealloc_cache_rejects_overflow(hf):
    layer = hf.PreallocLayer(max_len=4)
    x = torch.zeros((1, 1, 3, 128))
    layer.update(x, x)
    with pytest.raises(RuntimeError, match="exceed max_len"):
        layer.update(x, x)


def test_full_buffer_view_detection(hf):
    buf = torch.arange(2 * 3 * 10 * 128, dtype=torch.float32).reshape(2, 3, 10, 128)
    view = buf[:, :, :7]
    full = hf._full_buffer(view)
    assert full is not None and full.shape == buf.shape and full.data_ptr() == buf.data_ptr()
    assert torch.equal(full, buf)
    assert hf._full_buffer(buf[:, :, 2:9]) is None          # does not start at token 0
    assert hf._full_buffer(buf[1:, :, :5]) is not None       # later batch rows: a whole sub-buffer
    assert hf._full_buffer(buf.transpose(1, 2)) is None     # not [B, H, L, D] token rows
    assert hf._full_buffer(buf[:, :, :, :64]) is None       # channel slice


def test_unpack_int4_matches_oracle(hf):
    rng = np.random.default_rng(3)
    codes = rng.integers(-8, 8, size=(2, 3, 5, 128)).astype(np.int8)
    packed = kq.pack_kv_int4(codes)
    assert np.array_equal(hf._unpack_int4(torch.from_numpy(packed)).numpy(), codes)
