"""Shared test helpers: paths and seeded synthetic inputs."""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "llm-inference-kernels_amd"
for _p in (str(ROOT), str(PKG)):
    if _p not in sys.path:
        sys.path.insert(0, _p)

GOLDEN = ROOT / "tests" / "golden"

# K outlier channels used by the INT8/INT4 configs (x10).
OUTLIER_CHANNELS = (3, 37, 71, 105)


def randn(shape, seed: int, scale: float = 1.0, dtype=np.float32) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(shape) * scale).astype(dtype)


def kv_with_outliers(shape, seed: int) -> np.ndarray:
    x = randn(shape, seed)
    x[..., list(OUTLIER_CHANNELS)] *= 10.0
    return x
