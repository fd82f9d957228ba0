"""GPU parity for the fp16 attention's two tile sizes.

fp16 calls on the MFMA path run either 32-token tiles
(decode_attention_mfma_kernel) or 16-token tiles with the next tile in
flight (decode_attention_f16h_kernel); the planner picks the 16-token form
for at least 32 (batch, kv head, head chunk) slabs, a workgroup count that is
a multiple of the CU count, and at least two 32-token tiles per wave unless
the workgroups have 4 waves. Here each case runs under both
(llmik_attention_set_plan_override) and under the rule:
* both are within 2e-3 max-abs of the float64 oracle;
* the rule's call equals the forced call of the form the rule names, bit for
  bit (the knob and the rule reach the same kernel);
* the 16-token form is deterministic across calls and permutes with a batch
  permutation bit for bit.
Shapes: ragged lengths (a last tile of 1, 5 and 15 tokens), a live length
inside a larger buffer with a poisoned tail, 1, 2 and 4 query heads per
workgroup, 4- and 8-wave workgroups, one split and several.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as oa
from tests.helpers import randn

pytestmark = pytest.mark.gpu

TOL = 2e-3


def _set(mode: int) -> None:
    from llmik_cuda._lib import lib
    lib.llmik_attention_set_plan_override(mode)


@pytest.fixture(autouse=True)
def _restore_rule(llmik):
    yield
    _set(-1)


# (B, H, Hkv, S, buf, rule_half): rule_half is the form plan_attention's rule
# picks on a 256-CU MI355X.
CASES = [
    (8, 32, 8, 4096, 4096, True),     # headline: 4 splits x 8 waves, 4 tiles per wave
    (4, 32, 8, 4096, 4096, True),     # 8 splits, 2 tiles per wave
    (8, 32, 8, 4097, 4097, True),     # a 1-token last tile
    (16, 32, 8, 2053, 2053, True),    # a 5-token last tile, 2 splits
    (4, 32, 8, 8191, 8192, True),     # live length 8191 of 8192: a 15-token last tile
    (8, 16, 8, 3000, 3500, True),     # two heads per workgroup, poisoned tail past 3000
    (32, 8, 8, 1500, 1500, True),     # MHA, 256 slabs, no split: 4 waves, 12 tiles per wave
    (2, 32, 8, 4096, 4096, False),    # 16 slabs
    (8, 32, 8, 1024, 1024, True),     # 4-wave workgroups (512), 1 tile per wave
    (4, 64, 8, 2000, 2000, True),     # GQA 8: two head chunks per kv head
    (8, 24, 8, 2000, 2000, False),    # GQA 3: one head per workgroup, three chunks per kv head (384 workgroups)
]


def _run(llmik, cuda, q, k, v, scale, live):
    return llmik.decode_attention(torch.from_numpy(q).to(cuda), torch.from_numpy(k).to(cuda),
                                  torch.from_numpy(v).to(cuda), scale, live)


@pytest.mark.parametrize("B,H,Hkv,S,buf,rule_half", CASES)
def test_fp16_tile_forms_match_oracle(llmik, cuda, B, H, Hkv, S, buf, rule_half):
    seed = B * 131 + S
    q = randn((B, H, 128), seed).astype(np.float16)
    k = randn((B, Hkv, buf, 128), seed + 1).astype(np.float16)
    v = randn((B, Hkv, buf, 128), seed + 2).astype(np.float16)
    if buf > S:
        k[:, :, S:] = np.float16(60000.0)
        v[:, :, S:] = np.float16(np.nan)
    scale = 1 / math.sqrt(128)
    rows = sorted({0, B // 2, B - 1})
    ref = np.concatenate([oa.decode_attention(q[b:b + 1], k[b:b + 1], v[b:b + 1], scale, seqlen=S,
                                              acc_dtype=np.float64) for b in rows])
    outs = {}
    for mode in (0, 1, -1):
        _set(mode)
        outs[mode] = _run(llmik, cuda, q, k, v, scale, S)
    torch.cuda.synchronize()
    for mode in (0, 1):
        err = float(np.abs(outs[mode][rows].double().cpu().numpy() - ref).max())
        assert err <= TOL, f"form {'16' if mode else '32'}-token: {err}"
    if torch.cuda.get_device_properties(cuda).multi_processor_count == 256:   # the plans named above
        assert torch.equal(outs[-1], outs[1 if rule_half else 0])


@pytest.mark.parametrize("B,S", [(8, 4096), (4, 8191)])
def test_fp16_half_tiles_deterministic_and_batch_invariant(llmik, cuda, B, S):
    _set(1)
    gen = torch.Generator(device=cuda).manual_seed(B + S)
    kd = torch.randn((B, 8, S, 128), generator=gen, device=cuda, dtype=torch.float16)
    vd = torch.randn((B, 8, S, 128), generator=gen, device=cuda, dtype=torch.float16)
    qd = torch.randn((B, 32, 128), generator=gen, device=cuda, dtype=torch.float16)
    scale = 1 / math.sqrt(128)
    first = llmik.decode_attention(qd, kd, vd, scale)
    for _ in range(3):
        assert torch.equal(llmik.decode_attention(qd, kd, vd, scale), first)
    perm = torch.randperm(B, generator=torch.Generator().manual_seed(3)).to(cuda)
    out_p = llmik.decode_attention(qd[perm].contiguous(), kd[perm].contiguous(), vd[perm].contiguous(), scale)
    assert torch.equal(out_p, first[perm])
