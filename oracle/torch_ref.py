"""The reference's PyTorch paths, restated with torch ops on the CPU (test
infrastructure; see oracle/__init__.py).

These are the host-CPU baselines that run beside the GPU kernels: the same
torch operations, in the same order, as the reference's Python oracles, so
that a CPU figure times what the reference's CPU path does. Their results
are pinned against this package's numpy restatement
(tests/test_oracle_torch_ref.py), which is itself pinned by golden vectors,
closed forms and brute force.

  eager_decode_attention   reference/attention_ref.py:15-40 (_expand_gqa by
                           repeat_interleave), :43-80 (eager_attention: fp32
                           scores * scale, softmax, probs @ v, .to(q.dtype)),
                           :108-123 (decode_attention: q_len == 1)
  quantize_per_token       reference/kv_cache_ref.py:46-62 on x.float()
                           (the reference tests' convention,
                           tests/test_kv_cache.py:234,333,360)
  quantize_per_channel_groupwise
                           reference/kv_cache_ref.py:73-112 on x.float()
  quantized_matmul_ref     reference/quant_matmul_ref.py:91-135 (fp32
                           dequantised W materialised per call, fp32 matmul,
                           .to(act.dtype))
"""
from __future__ import annotations

import math
import os
from typing import Optional, Tuple

import torch


def host_threads() -> int:
    """Cores this process may run on (os.sched_getaffinity), capped by
    OMP_NUM_THREADS when the environment sets one (a GPU box's CPU share)."""
    n = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def eager_decode_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                           scale: Optional[float] = None) -> torch.Tensor:
    """q [B, H, D]; k, v [B, Hkv, S, D] -> [B, H, D] in q.dtype."""
    q4 = q.unsqueeze(2)                                   # [B, H, 1, D]
    n_heads, head_dim = q4.shape[1], q4.shape[3]
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    if k.shape[1] != n_heads:
        rep = n_heads // k.shape[1]
        k = k.repeat_interleave(rep, dim=1)
        v = v.repeat_interleave(rep, dim=1)
    scores = torch.matmul(q4.float(), k.float().transpose(-1, -2)) * scale
    probs = torch.softmax(scores, dim=-1)
    return torch.matmul(probs, v.float()).to(q.dtype).squeeze(2)


def _qmax(bits: int) -> int:
    return (1 << (bits - 1)) - 1


def quantize_per_token(x: torch.Tensor, bits: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """x [B, Hkv, S, D] fp32 -> (q int8, scale [B, Hkv, S] fp32)."""
    qm = _qmax(bits)
    scale = (x.abs().amax(dim=-1, keepdim=True) / qm).clamp(min=1e-8)
    q = (x / scale).round().clamp(-qm, qm).to(torch.int8)
    return q, scale.squeeze(-1)


def quantize_per_channel_groupwise(x: torch.Tensor, bits: int, group_size: int
                                   ) -> Tuple[torch.Tensor, torch.Tensor]:
    """x [B, Hkv, S, D] fp32 -> (q int8 [B, Hkv, S, D], scale [B, Hkv, ceil(S/g), D])."""
    qm = _qmax(bits)
    B, H, S, D = x.shape
    ng = (S + group_size - 1) // group_size
    pad = ng * group_size - S
    xp = torch.nn.functional.pad(x, (0, 0, 0, pad)) if pad else x
    xg = xp.reshape(B, H, ng, group_size, D)
    scale = (xg.abs().amax(dim=3, keepdim=True) / qm).clamp(min=1e-8)
    q = (xg / scale).round().clamp(-qm, qm).to(torch.int8)
    return q.reshape(B, H, ng * group_size, D)[:, :, :S], scale.squeeze(3)


def quantized_matmul_ref(act: torch.Tensor, q_weights: torch.Tensor, scale: torch.Tensor,
                         group_size: int) -> torch.Tensor:
    """act [M, K] fp16, q_weights [K, N] int8 codes, scale [K/g, N] fp16 -> [M, N] fp16."""
    K = q_weights.shape[0]
    group_idx = torch.arange(K) // group_size
    w_hat = q_weights.float() * scale.index_select(0, group_idx).float()
    return (act.float() @ w_hat).to(act.dtype)
