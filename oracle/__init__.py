"""CPU oracle for the decode-step hot path — TEST INFRASTRUCTURE ONLY.

A from-scratch numpy restatement of the reference's PyTorch correctness
oracles (reference/attention_ref.py, reference/kv_cache_ref.py,
reference/quant_matmul_ref.py of bundle-adjuster/llm-inference-kernels) and
of the packing formats its CUDA kernels define. Each function cites the
reference file:line it follows.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker or the timed CPU baseline:
the product path (llmik_cuda) never calls into it.

Pinning (what fixes each function independently of its own formulas):
  attention   float64 brute force on tiny shapes, closed forms (one token,
              constant keys, dominant score), GQA == repeat_interleave,
              token-permutation invariance           -> tests/test_oracle_attention.py
  kv_quant    golden vectors written by the reference's own Python oracle
              (tests/golden/make_golden.py), hand-computed ties, round-trip
              bound, plant-a-mistake checks          -> tests/test_oracle_quant.py
  w4a16       the reference's literal pack/unpack KAT
              (tests/test_quant.py:201-244), golden vectors, float64 matmul
                                                     -> tests/test_oracle_w4a16.py
  fused       closed forms (unit weight / zero input) and the reference
              test's PyTorch formulas                -> tests/test_oracle_fused.py
  torch_ref   the same reference paths as torch CPU ops (the host baseline
              bench.py times), pinned to the numpy functions above
                                                     -> tests/test_oracle_torch_ref.py
"""
from . import attention, fused, kv_quant, w4a16  # noqa: F401
# torch_ref (torch CPU restatements for the host baseline) is imported on demand.
