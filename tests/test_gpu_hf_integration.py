"""GPU: the transformers 5 integration (llmik_cuda.hf) inside a small
randomly initialised Llama (hidden 512, 4 heads and 2 KV heads of
head_dim 128, 2 layers; no download) in fp16. Each test feeds the same
prompt and decode tokens (teacher-forced) to the stock model and to the
patched one and compares the logits of the prefill and of every decode
step. The llmik kernels must actually run (call counters on the decode
paths); transformers' own SDPA serves prefill, as in the reference's hooks
(integration/attention_patch.py:178-273, prealloc_cache.py:82-110)."""
from __future__ import annotations

import copy

import pytest
import torch

pytest.importorskip("transformers")

pytestmark = pytest.mark.gpu

LOGIT_TOL = 2e-2


@pytest.fixture(scope="module")
def hf(llmik):
    from llmik_cuda import hf as mod
    mod.register()
    return mod


def _model(cuda, attn="sdpa", seed=0):
    from transformers import LlamaConfig, LlamaForCausalLM
    cfg = LlamaConfig(hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=128, vocab_size=512,
                      max_position_embeddings=1024)
    torch.manual_seed(seed)
    m = LlamaForCausalLM(cfg).to(device=cuda, dtype=torch.float16).eval()
    m.set_attn_implementation(attn)
    return m


def _tokens(cuda, B=2, prompt_len=45, steps=7, seed=1):
    g = torch.Generator().manual_seed(seed)
    prompt = torch.randint(0, 512, (B, prompt_len), generator=g).to(cuda)
    return prompt, [torch.randint(0, 512, (B, 1), generator=g).to(cuda) for _ in range(steps)]


def _run(model, cache, prompt, steps):
    with torch.no_grad():
        out = [model(input_ids=prompt, past_key_values=cache, use_cache=True).logits[:, -1].float()]
        for t in steps:
            out.append(model(input_ids=t, past_key_values=cache, use_cache=True).logits[:, -1].float())
    torch.cuda.synchronize()
    return torch.stack(out)


def _counting(monkeypatch, module, name):
    calls = {"n": 0}
    fn = getattr(module, name)

    def wrapped(*a, **k):
        calls["n"] += 1
        return fn(*a, **k)
    monkeypatch.setattr(module, name, wrapped)
    return calls


def test_decode_attention_with_dynamic_cache(hf, cuda, monkeypatch):
    from transformers import DynamicCache
    prompt, steps = _tokens(cuda)
    ref = _run(_model(cuda, "sdpa"), DynamicCache(), prompt, steps)
    calls = _counting(monkeypatch, hf, "_decode_fp16")
    got = _run(_model(cuda, "llmik"), DynamicCache(), prompt, steps)
    assert calls["n"] == 2 * len(steps)        # every layer of every decode step
    assert float((got - ref).abs().max()) <= LOGIT_TOL


def test_decode_attention_over_prealloc_cache(hf, cuda, monkeypatch):
    from transformers import DynamicCache
    prompt, steps = _tokens(cuda, seed=2)
    ref = _run(_model(cuda, "sdpa"), DynamicCache(), prompt, steps)
    decode = _counting(monkeypatch, hf, "decode_attention")
    cache = hf.PreallocCache(max_len=128)
    got = _run(_model(cuda, "llmik"), cache, prompt, steps)
    assert decode["n"] == 2 * len(steps)
    assert cache.get_seq_length() == prompt.shape[1] + len(steps)
    assert float((got - ref).abs().max()) <= LOGIT_TOL


def _kivi_emulation(hf, gs):
    """Attention over the KIVI quantisation of K/V done the reference's way
    (kv_int4_cache.py): prefill on its fp16 view (dequantised full groups +
    fp16 open group), decode on the whole cache quantised (K groups, the
    last one partial; V per token), dequantised in fp32."""
    import llmik_cuda as llmik
    from transformers.integrations.sdpa_attention import sdpa_attention_forward

    def dq(k, v):
        kq, ks = llmik.quantize_k_per_channel_groupwise_int4(k.contiguous(), gs)
        vq, vs = llmik.quantize_v_per_token_int4(v.contiguous())
        grp = torch.arange(k.shape[2], device=k.device) // gs
        kd = hf._unpack_int4(kq).float() * ks.index_select(2, grp).float()
        vd = hf._unpack_int4(vq).float() * vs.float().unsqueeze(-1)
        return kd, vd

    def attn(module, query, key, value, attention_mask, dropout=0.0, scaling=None, **kwargs):
        S = key.shape[2]
        full = S // gs * gs
        if query.shape[2] > 1:
            kd, vd = dq(key[:, :, :full], value[:, :, :full])
            key = torch.cat([kd.half(), key[:, :, full:]], dim=2)
            value = torch.cat([vd.half(), value[:, :, full:]], dim=2)
            return sdpa_attention_forward(module, query, key, value, attention_mask, dropout=dropout,
                                          scaling=scaling, **kwargs)
        kd, vd = dq(key, value)
        G = query.shape[1] // key.shape[1]
        kd, vd = kd.repeat_interleave(G, dim=1), vd.repeat_interleave(G, dim=1)
        s = torch.matmul(query.float(), kd.transpose(-1, -2)) * scaling
        o = torch.matmul(torch.softmax(s, dim=-1), vd).half()
        return o.transpose(1, 2).contiguous(), None
    return attn


@pytest.mark.parametrize("gs,prompt_len,n_steps", [(32, 45, 21), (128, 228, 37)])
def test_kivi_cache_decode_runs_the_int4_kernel(hf, cuda, monkeypatch, gs, prompt_len, n_steps):
    """Prefill leaves an open group; the decode steps fill it and open the next."""
    from transformers import AttentionInterface, DynamicCache
    from transformers.masking_utils import AttentionMaskInterface, sdpa_mask
    AttentionInterface.register("kivi_emul", _kivi_emulation(hf, gs))
    AttentionMaskInterface.register("kivi_emul", sdpa_mask)
    prompt, steps = _tokens(cuda, prompt_len=prompt_len, steps=n_steps, seed=3)
    ref = _run(_model(cuda, "kivi_emul"), DynamicCache(), prompt, steps)
    calls = _counting(monkeypatch, hf.KIVILayer, "attention")
    cache = hf.KIVICache(max_len=512, group_size=gs)
    got = _run(_model(cuda, "llmik"), cache, prompt, steps)
    assert calls["n"] == 2 * len(steps)
    assert cache.get_seq_length() == prompt.shape[1] + len(steps)
    assert float((got - ref).abs().max()) <= LOGIT_TOL


def test_w4a16_patch(hf, cuda):
    """QuantizedLinear against the same model with each projection's weight
    replaced by its dequantised W4 (fp16) -- the quantisation is common to
    both, so the difference is the GEMM path's."""
    import llmik_cuda as llmik
    from transformers import DynamicCache
    prompt, steps = _tokens(cuda, seed=4)
    base = _model(cuda, "llmik")
    ref_model = copy.deepcopy(base)
    assert hf.patch_model_w4a16(base, group_size=128) == 2 * 7
    for layer_q, layer_r in zip(base.model.layers, ref_model.model.layers):
        for parent in ("self_attn", "mlp"):
            for name, mod in getattr(layer_q, parent).named_children():
                if isinstance(mod, hf.QuantizedLinear):
                    W = llmik.w4a16_dequantize(mod.weight_packed, mod.scale, 128)   # [K, N]
                    getattr(getattr(layer_r, parent), name).weight.data.copy_(W.t())
    got = _run(base, DynamicCache(), prompt, steps)
    ref = _run(ref_model, DynamicCache(), prompt, steps)
    assert float((got - ref).abs().max()) <= LOGIT_TOL
    # the prefill-size path (dequantise + matmul) from the crossover on
    assert hf.dequant_path_threshold(512) == 1536 and hf.dequant_path_threshold(14336) == 1024
    x = torch.randn((1600, 512), device=cuda, dtype=torch.float16)
    q = base.model.layers[0].self_attn.q_proj
    W = llmik.w4a16_dequantize(q.weight_packed, q.scale, 128)
    assert torch.equal(q(x), x @ W)


def test_fused_ops_patch(hf, cuda):
    from transformers import DynamicCache
    prompt, steps = _tokens(cuda, seed=5)
    model = _model(cuda, "llmik")
    ref = _run(model, DynamicCache(), prompt, steps)
    with hf.fused_ops():
        got = _run(model, DynamicCache(), prompt, steps)
    after = _run(model, DynamicCache(), prompt, steps)
    assert torch.equal(after, ref)               # the originals are restored
    assert float((got - ref).abs().max()) <= LOGIT_TOL


def test_softcap_sinks_and_windows_take_the_sdpa_path(hf, cuda, monkeypatch):
    """A decode-shaped call carrying logit soft-capping, attention sinks or a
    sliding window is not what the decode kernels compute: it must return
    SDPA's result and never reach decode_attention."""
    from transformers.integrations.sdpa_attention import sdpa_attention_forward
    calls = _counting(monkeypatch, hf, "decode_attention")
    g = torch.Generator(device=cuda).manual_seed(5)
    q = torch.randn((2, 4, 1, 128), generator=g, device=cuda, dtype=torch.float16)
    k = torch.randn((2, 2, 40, 128), generator=g, device=cuda, dtype=torch.float16)
    v = torch.randn((2, 2, 40, 128), generator=g, device=cuda, dtype=torch.float16)
    module = torch.nn.Module()
    module.num_key_value_groups = 2
    module.is_causal = True
    plain, _ = hf.llmik_attention_forward(module, q, k, v, None, scaling=0.088)
    assert calls["n"] == 1
    for extra in ({"softcap": 5.0}, {"sliding_window": 16}):
        got, _ = hf.llmik_attention_forward(module, q, k, v, None, scaling=0.088, **extra)
        ref, _ = sdpa_attention_forward(module, q, k, v, None, scaling=0.088, **extra)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), extra
    assert calls["n"] == 1
    assert plain.shape == (2, 1, 4, 128)
