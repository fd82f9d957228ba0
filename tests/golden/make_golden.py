"""Write the golden vectors under tests/golden/ from the reference's own
Python oracles (run once, in the build container, on the CPU).

Only the quantisers are taken from the reference this way: their bit-level
behaviour under torch's dtype rules (fp16-input scales rounded before the
division, clamp(min=1e-8) in fp16, NaN codes of all-zero fp16 rows, and
rows holding NaN or +-inf, whose amax propagates NaN) is not fixed by any
closed form. Attention is pinned by float64 brute force and
closed forms instead and is not imported.

Functions used (bundle-adjuster/llm-inference-kernels):
  reference/kv_cache_ref.py      quantize_per_token, quantize_per_channel_groupwise
  reference/quant_matmul_ref.py  quantize_weights_int4_groupwise, pack_int4_along_k,
                                 quantized_matmul_ref

Usage: python tests/golden/make_golden.py [--reference /root/reference]
Outputs: tests/golden/kv_quant_golden.npz, tests/golden/w4a16_golden.npz
(inputs and expected outputs only; the fp16 inputs are the stored fp32
inputs rounded with numpy's astype(float16), which is round-to-nearest-even).
"""
from __future__ import annotations

import argparse
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
OUTLIER_CHANNELS = (3, 37, 71, 105)


def hard_row(rng: np.random.Generator, qmax: int, n: int = 128) -> np.ndarray:
    """A row whose quotients x/scale sit within a few ulps of half-integers,
    chosen so that rint(x * fl(1/scale)) != rint(fl(x / scale)): it separates
    true division from reciprocal multiplication."""
    f32 = np.float32
    while True:
        amax = f32(rng.uniform(0.5, 8.0))
        s = f32(amax / f32(qmax))
        r = f32(f32(1.0) / s)
        if f32(r * s) != f32(1.0):
            break
    row = np.zeros(n, dtype=f32)
    row[0] = amax
    filled = 1
    for _ in range(20000):
        if filled == n:
            break
        k = int(rng.integers(-qmax + 1, qmax - 1))
        x = f32((k + 0.5) * s)
        for step in range(-6, 7):
            xs = x
            for _ in range(abs(step)):
                xs = f32(np.nextafter(xs, f32(np.inf if step > 0 else -np.inf)))
            if abs(xs) >= amax:
                continue
            if np.rint(f32(xs / s)) != np.rint(f32(xs * r)):
                row[filled] = xs
                filled += 1
                break
    return row


def kv_input(rng: np.random.Generator, shape) -> np.ndarray:
    x = rng.standard_normal(shape).astype(np.float32)
    x[..., list(OUTLIER_CHANNELS)] *= 10.0
    # special rows: all zero, tiny magnitudes (fp16 subnormal scales), exact ties
    x[0, 0, 0, :] = 0.0
    x[0, 0, 1, :] *= 1.0e-6
    tie = np.zeros(x.shape[-1], dtype=np.float32)
    tie[:8] = [127.0, 0.5, 1.5, 2.5, -0.5, -2.5, 63.5, -126.5]
    x[0, 1, 2, :] = tie
    tie4 = np.zeros(x.shape[-1], dtype=np.float32)
    tie4[:8] = [7.0, 0.5, 1.5, 2.5, 3.5, -3.5, -6.5, 5.5]
    x[0, 1, 3, :] = tie4
    x[-1, 0, 4, :] = hard_row(rng, 127)
    x[-1, 1, 5, :] = hard_row(rng, 7)
    return x


def nonfinite_kv(rng: np.random.Generator):
    """Per-token and group-wise inputs holding NaN, +-inf and fp16 overflow
    (1e5 rounds to inf in fp16), at fixed places."""
    nan, inf = np.float32(np.nan), np.float32(np.inf)
    pt = rng.standard_normal((1, 2, 8, 128)).astype(np.float32)
    pt[..., list(OUTLIER_CHANNELS)] *= 10.0
    pt[0, 0, 0, 5] = nan
    pt[0, 0, 1, 7] = inf
    pt[0, 0, 2, 9] = -inf
    pt[0, 0, 3, :] = nan
    pt[0, 0, 4, 3], pt[0, 0, 4, 4] = inf, nan
    pt[0, 0, 5, 1], pt[0, 0, 5, 2] = inf, -inf
    pt[0, 0, 7, :] = 0.0
    pt[0, 1, 0, 127] = nan
    pt[0, 1, 3, 64] = 1.0e5
    pt[0, 1, 7, 0] = -inf
    gw = rng.standard_normal((1, 2, 100, 128)).astype(np.float32)
    gw[..., list(OUTLIER_CHANNELS)] *= 10.0
    gw[0, 0, 5, 3] = nan           # group 0 (g32, g128), channel 3
    gw[0, 0, 40, 10] = inf         # group 1 at g32
    gw[0, 0, 99, 20] = -inf        # the short last group
    gw[0, 0, 64:96, 30] = nan      # a whole g32 group of one channel
    gw[0, 1, 64, 64] = 1.0e5       # inf once rounded to fp16
    gw[0, 1, 10, 100], gw[0, 1, 11, 100] = inf, -inf
    return pt, gw


def nonfinite_w(rng: np.random.Generator) -> np.ndarray:
    W = (rng.standard_normal((256, 96)) * 0.02).astype(np.float32)
    W[3, 4] = np.nan
    W[130, 7] = np.inf
    W[200, 8] = -np.inf
    W[0:64, 10] = np.nan           # a whole g64 group of one column
    W[70, 11], W[71, 11] = np.inf, np.nan
    W[150, 12] = 1.0e5             # inf once rounded to fp16
    return W


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    args = ap.parse_args()
    sys.path.insert(0, args.reference)
    import torch
    from reference.kv_cache_ref import quantize_per_channel_groupwise, quantize_per_token
    from reference.quant_matmul_ref import (pack_int4_along_k, quantize_weights_int4_groupwise,
                                            quantized_matmul_ref)

    rng = np.random.default_rng(20260521)
    kv = {}
    x32 = kv_input(rng, (2, 2, 24, 128))
    kv["pt_x32"] = x32
    inputs = {"pt_x32": x32, "pt_x16": x32.astype(np.float16)}
    for name in ("pt_x32", "pt_x16"):
        xt = torch.from_numpy(inputs[name])
        for bits in (8, 4):
            q, s = quantize_per_token(xt, bits)
            kv[f"{name}_b{bits}_q"] = q.numpy()
            kv[f"{name}_b{bits}_s"] = s.numpy()

    g32 = kv_input(rng, (1, 2, 100, 128))
    kv["gw_x32"] = g32
    inputs = {"gw_x32": g32, "gw_x16": g32.astype(np.float16)}
    for name in ("gw_x32", "gw_x16"):
        xt = torch.from_numpy(inputs[name])
        for bits in (4, 8):
            for gs in (32, 128):
                q, s = quantize_per_channel_groupwise(xt, bits, gs)
                kv[f"{name}_b{bits}_g{gs}_q"] = q.numpy()
                kv[f"{name}_b{bits}_g{gs}_s"] = s.numpy()

    # Non-finite rows (own generator, so the arrays above do not move). The
    # KV kernels take fp16 and follow the x.float() convention; both dtype
    # conventions are stored.
    nrng = np.random.default_rng(20261202)
    pt_nf, gw_nf = nonfinite_kv(nrng)
    kv["nf_pt_x32"], kv["nf_gw_x32"] = pt_nf, gw_nf
    for pre, x32 in (("nf_pt", pt_nf), ("nf_gw", gw_nf)):
        x16 = x32.astype(np.float16)
        conv = {f"{pre}_x32": torch.from_numpy(x32), f"{pre}_x16": torch.from_numpy(x16),
                f"{pre}_x16f": torch.from_numpy(x16).float()}
        for name, xt in conv.items():
            for bits in (8, 4):
                if pre == "nf_pt":
                    q, s = quantize_per_token(xt, bits)
                    kv[f"{name}_b{bits}_q"], kv[f"{name}_b{bits}_s"] = q.numpy(), s.numpy()
                else:
                    for gs in (32, 128):
                        q, s = quantize_per_channel_groupwise(xt, bits, gs)
                        kv[f"{name}_b{bits}_g{gs}_q"] = q.numpy()
                        kv[f"{name}_b{bits}_g{gs}_s"] = s.numpy()
    np.savez_compressed(HERE / "kv_quant_golden.npz", **kv)

    w = {}
    W32 = (rng.standard_normal((256, 96)) * 0.02).astype(np.float32)
    W32[::7, ::9] *= 5.0
    W32[:, 5] = 0.0                       # an all-zero column
    w["W32"] = W32
    w["W16"] = W32.astype(np.float16)
    Wp = (rng.standard_normal((100, 40)) * 0.5).astype(np.float32)
    w["Wp32"] = Wp
    w["Wp16"] = Wp.astype(np.float16)
    for name in ("W32", "W16", "Wp32", "Wp16"):
        Wt = torch.from_numpy(w[name])
        for gs in (64, 128):
            q, s = quantize_weights_int4_groupwise(Wt, group_size=gs)
            w[f"{name}_g{gs}_q"] = q.numpy()
            w[f"{name}_g{gs}_s"] = s.numpy()
            if q.shape[0] % 8 == 0:
                w[f"{name}_g{gs}_packed"] = pack_int4_along_k(q).numpy()
    act = rng.standard_normal((3, 256)).astype(np.float16)
    w["act"] = act
    out = quantized_matmul_ref(torch.from_numpy(act), torch.from_numpy(w["W16_g128_q"]),
                               torch.from_numpy(w["W16_g128_s"]), 128)
    w["mm_out16"] = out.numpy()
    Wn = nonfinite_w(np.random.default_rng(20261203))
    w["Wn32"] = Wn
    w["Wn16"] = Wn.astype(np.float16)
    for name in ("Wn32", "Wn16"):
        for gs in (64, 128):
            q, s = quantize_weights_int4_groupwise(torch.from_numpy(w[name]), group_size=gs)
            w[f"{name}_g{gs}_q"] = q.numpy()
            w[f"{name}_g{gs}_s"] = s.numpy()
            w[f"{name}_g{gs}_packed"] = pack_int4_along_k(q).numpy()
    np.savez_compressed(HERE / "w4a16_golden.npz", **w)
    print("wrote", HERE / "kv_quant_golden.npz", HERE / "w4a16_golden.npz")


if __name__ == "__main__":
    main()
