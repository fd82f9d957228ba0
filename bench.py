"""Benchmark of the decode-step hot path on one MI355X.

Headline (the JSON `value`): fp16 split-K GQA decode attention at the
Llama-3-8B decode shape B=8, H=32, Hkv=8, D=128, S=4096 — one step is one
decode_attention call over one batch of synthetic inputs. The other
BASELINE.json configs (INT8 / INT4 KIVI attention, the KV writers, W4A16 at
M in {1, 16, 128} on the three Llama shapes, the S / B sweep) are measured
the same way and reported under "details", beside the wider rows: W4A16 at
prefill sizes (M in {256, 2048}, next to dequantise + hipBLASLt), a whole
decode step through four Llama-3-8B layers (eager and graph-replayed), the
in-place quantised KV appends and the GPU weight quantiser.

Method
  * Inputs are generated on the GPU from a seeded generator and are resident
    in HBM before timing. Each config rotates over enough distinct input
    sets (>= 768 MiB in total, three times the 256 MB Infinity Cache) that
    every step reads from HBM; a detail row's graph holds at least one call
    per set, so every set is read once per replay.
  * The K timed steps are captured in one HIP graph on a dedicated stream and
    replayed once; HIP events recorded on that stream bracket the replay,
    with torch.cuda.synchronize() on both sides. Per-launch time = elapsed/K.
  * Untimed warm-up before it: one eager call per input set, then replays of
    the same graph, at least W calls (--warmup, default 16000) and at least
    0.4 s of GPU time, then one settling replay: after the host-side set-up
    the kernels run a few per cent slower until the GPU has been under
    sustained load for 17-140 ms ("warmup_calls" in the output counts the
    untimed calls).
  * Each attention and W4A16 row also carries "dist": the median, p10 and
    p90 per-call time over 100 replays (after 25 warm-up replays) of a graph
    of max(20, sets) calls over the input sets, each replay bracketed by its
    own events. Full rows go to stderr as they are measured; the JSON line
    carries a compact {row: {us, frac, ...}} per config ("details") so that
    it stays a few KB long.
  * Before timing, every config is checked against a float64 torch
    computation on the GPU (max-abs 2e-3); a failing config aborts the run.
  * roofline.achieved = algorithmic bytes per launch / per-launch time, the
    bytes counting each tensor once (attn_bytes, w4a16_bytes: K and V once per
    KV head, plus q, out and scales); peak = 8 TB/s (MI355X HBM3E).
  * cpu_baseline: the reference's eager fp32 attention restated with torch
    CPU ops (oracle/torch_ref.py: repeat_interleave GQA, fp32 matmul,
    softmax, matmul, .to(fp16)) on the host cores given by
    os.sched_getaffinity (capped by OMP_NUM_THREADS), median of >= 10 calls
    after 3 warm-up calls, at the headline shape.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-details] [--no-cpu]
       python bench.py --floors          (empty-kernel and plain-read floors)
       python bench.py --pmc-workload X  (the program the counter passes profile)
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "llm-inference-kernels_amd"))
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
TRAFFIC_FILE = ROOT / "profiles" / "decode_attention_fp16_a16_traffic.md"
MFMA_FP16_PEAK_TFLOPS = 2500.0
ROTATE_BYTES = 768 << 20
GATE_TOL = 2e-3


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ----------------------------------------------------------- byte accounting

def attn_bytes(fmt: str, B: int, H: int, Hkv: int, S: int, D: int = 128, gs: int = 128) -> int:
    qo = 2 * B * H * D * 2
    if fmt == "fp16":
        return 2 * B * Hkv * S * D * 2 + qo
    if fmt == "int8":
        return 2 * (B * Hkv * S * D + 2 * B * Hkv * S) + qo
    if fmt == "int4":
        return B * Hkv * S * D + 2 * B * Hkv * ((S + gs - 1) // gs) * D + 2 * B * Hkv * S + qo
    raise ValueError(fmt)


def w4a16_bytes(M: int, K: int, N: int, gs: int = 128) -> int:
    return K * N // 2 + 2 * (K // gs) * N + 2 * M * K + 2 * M * N


# ----------------------------------------------------------------- timing

WARM_MS = 400.0   # untimed replays before a timed one: at least this much GPU time


def time_steps(steps_fns, warmup: int, reps: int, all_sets: bool = True, info: dict | None = None):
    """Capture `reps` steps (cycling through steps_fns) in a HIP graph, warm
    up, and time one replay with events on the capture stream.

    Untimed warm-up: one eager call per input set (an op's per-stream
    workspace is allocated and zeroed on its first call, which must not land
    inside the graph), then replays of the same graph, ceil(warmup / reps)
    of them and at least WARM_MS of GPU time. After the host-side set-up
    between configs the kernels run a few per cent slower until the GPU has
    been under sustained load for a while, then step down and stay there
    (kernel traces: fp16 B=64 S=8192 322-324 -> 308-309 us per call 48 ms
    into the run, S=32768 166-168 -> 158-160 us after 140 ms, INT8 A8
    15.7 -> 14.9 us after 17 ms; at A16, after 200 ms idle, one or two warm
    replays left 25.5-26.1 us, five or more 25.3-25.4). WARM_MS covers the
    slowest switch seen; one more untimed replay after the burst settles the
    runtime (below). With `all_sets`, the graph holds at least one step
    per input set, so a replay reads every set. Returns per-step
    microseconds; `info`, if given, receives the untimed call count as
    "warmup_calls"."""
    import torch
    if all_sets:
        reps = max(reps, len(steps_fns))
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for fn in steps_fns:
            fn()
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(reps):
            steps_fns[i % len(steps_fns)]()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):   # replay() launches on the current stream
        start.record(stream)
        graph.replay()                # first untimed replay: its length sizes the warm-up
        end.record(stream)
        torch.cuda.synchronize()
        n_warm = max(-(-warmup // reps), math.ceil(WARM_MS / max(start.elapsed_time(end), 1e-3)))
        n_warm = min(n_warm, 4000)
        for _ in range(n_warm - 1):
            graph.replay()
        torch.cuda.synchronize()
        # The first replay after a burst of hundreds pays a one-off runtime
        # cost (measured: after 400-800 queued replays of a 50-call graph
        # the next replay took 15.8-18.1 us per call instead of 10.3, the
        # ones after it 10.3 again); one more untimed replay absorbs it.
        graph.replay()
        torch.cuda.synchronize()
        start.record(stream)
        graph.replay()
        end.record(stream)
    torch.cuda.synchronize()
    if info is not None:
        info["warmup_calls"] = len(steps_fns) + (n_warm + 1) * reps
    us = start.elapsed_time(end) * 1000.0 / reps
    del graph
    return us


def sample_steps(steps_fns, n_samples: int = 100, warmup_replays: int = 25, min_calls: int = 20):
    """Per-call time distribution: capture max(min_calls, sets) calls cycling
    through the input sets in a HIP graph (every set read at least once per
    replay, so each replay reads HBM; >= 20 calls so that the gap between
    two replays is spread over enough calls), replay it `warmup_replays`
    times, then `n_samples` times with an event recorded between replays on
    the capture stream. Each sample is one replay's elapsed time over its
    calls. Returns {median_us, p10_us, p90_us, samples, calls_per_sample}."""
    import torch
    calls = max(min_calls, len(steps_fns))
    stream = torch.cuda.Stream()
    # One eager call per set first: an op's per-stream workspace is allocated
    # (and zeroed) on its first call, which must not land inside the graph.
    with torch.cuda.stream(stream):
        for fn in steps_fns:
            fn()
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(calls):
            steps_fns[i % len(steps_fns)]()
    events = [torch.cuda.Event(enable_timing=True) for _ in range(n_samples + 1)]
    with torch.cuda.stream(stream):
        for _ in range(warmup_replays):
            graph.replay()
        events[0].record(stream)
        for i in range(n_samples):
            graph.replay()
            events[i + 1].record(stream)
    torch.cuda.synchronize()
    per_call = sorted(events[i].elapsed_time(events[i + 1]) * 1000.0 / calls
                      for i in range(n_samples))
    del graph

    def q(f):
        return round(per_call[min(n_samples - 1, int(f * n_samples))], 3)
    return {"median_us": q(0.5), "p10_us": q(0.1), "p90_us": q(0.9), "samples": n_samples,
            "calls_per_sample": calls}


def n_sets_for(bytes_per_set: int) -> int:
    """Input sets whose total is >= ROTATE_BYTES (at most 512)."""
    return max(2, min(512, math.ceil(ROTATE_BYTES / max(1, bytes_per_set))))


# ------------------------------------------------------------ correctness gates

def torch_attention_ref(q, k, v, scale):
    """float64 GQA attention on the GPU (grouped, no KV expansion)."""
    import torch
    B, H, D = q.shape
    Hkv = k.shape[1]
    G = H // Hkv
    qf = q.double().reshape(B, Hkv, G, D)
    s = torch.matmul(qf, k.double().transpose(-1, -2).contiguous()) * scale
    p = torch.softmax(s, dim=-1)
    return torch.matmul(p, v.double()).reshape(B, H, D)


def gate(name: str, got, ref) -> float:
    err = float((got.double() - ref.double()).abs().max())
    if not err <= GATE_TOL:
        raise SystemExit(f"correctness gate failed for {name}: max-abs {err:.3e} > {GATE_TOL}")
    return err


def excess_over_output_rounding(got, ref) -> float:
    """max(|got - ref| - half an fp16 ulp of ref): the error that is not the
    fp16 output's own rounding."""
    import torch
    a = ref.abs().to(torch.float16)
    nxt = torch.nextafter(a, torch.full_like(a, float("inf"))).double()
    half_ulp = (nxt - a.double()) / 2
    return float(((got.double() - ref.double()).abs() - half_ulp).max())


# ------------------------------------------------------------------ configs

def bench_attention(llmik, fmt: str, B: int, S: int, steps: int, warmup: int, gs: int = 128,
                    H: int = 32, Hkv: int = 8, seed: int = 0, exact_steps: bool = False):
    import torch
    dev = torch.device("cuda:0")
    D = 128
    scale = 1.0 / math.sqrt(D)
    nbytes = attn_bytes(fmt, B, H, Hkv, S, D, gs)
    n_sets = n_sets_for(nbytes)
    gen = torch.Generator(device=dev).manual_seed(seed)
    sets = []
    for _ in range(n_sets):
        q = torch.randn((B, H, D), generator=gen, device=dev, dtype=torch.float16)
        k = torch.randn((B, Hkv, S, D), generator=gen, device=dev, dtype=torch.float16)
        v = torch.randn((B, Hkv, S, D), generator=gen, device=dev, dtype=torch.float16)
        if fmt != "fp16":
            k[..., [3, 37, 71, 105]] *= 10
        if fmt == "fp16":
            sets.append((q, k, v))
        elif fmt == "int8":
            sets.append((q, *llmik.quantize_per_token(k), *llmik.quantize_per_token(v)))
        else:
            sets.append((q, *llmik.quantize_k_per_channel_groupwise_int4(k, gs),
                         *llmik.quantize_v_per_token_int4(v)))
        del k, v
    # correctness gate on the first set (first <= 8 sequences)
    gb = min(B, 8)
    if fmt == "fp16":
        q0, k0, v0 = sets[0]
        got = llmik.decode_attention(q0, k0, v0, scale)
        kd, vd = k0[:gb], v0[:gb]
    elif fmt == "int8":
        q0, kq, ks, vq, vs = sets[0]
        got = llmik.decode_attention_int8(q0, kq, ks, vq, vs, scale)
        kd = kq[:gb].float() * ks[:gb].float()[..., None]
        vd = vq[:gb].float() * vs[:gb].float()[..., None]
    else:
        q0, kq, ks, vq, vs = sets[0]
        got = llmik.decode_attention_int4(q0, kq, ks, vq, vs, gs, scale)
        kd = unpack_int4(kq[:gb]).float() * ks[:gb].float().repeat_interleave(gs, dim=2)[:, :, :S]
        vd = unpack_int4(vq[:gb]).float() * vs[:gb].float()[..., None]
    ref = torch_attention_ref(q0[:gb], kd, vd, scale)
    err = gate(f"{fmt} attention B={B} S={S}", got[:gb], ref)
    excess = excess_over_output_rounding(got[:gb], ref)
    del kd, vd, got, ref

    if fmt == "fp16":
        fns = [lambda s=s: llmik.decode_attention(s[0], s[1], s[2], scale) for s in sets]
    elif fmt == "int8":
        fns = [lambda s=s: llmik.decode_attention_int8(s[0], s[1], s[2], s[3], s[4], scale)
               for s in sets]
    else:
        fns = [lambda s=s: llmik.decode_attention_int4(s[0], s[1], s[2], s[3], s[4], gs, scale)
               for s in sets]
    info = {}
    us = time_steps(fns, warmup, steps, all_sets=not exact_steps, info=info)
    dist = sample_steps(fns)
    del sets, fns
    torch.cuda.empty_cache()
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"name": f"attn_{fmt}" + (f"_g{gs}" if fmt == "int4" else ""), "B": B, "S": S,
            "us": round(us, 3), "bytes": nbytes, "GBps": round(gbs, 1),
            "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4), "max_abs_err": err,
            "max_err_minus_out_half_ulp": excess, "sets": n_sets,
            "rotated_MB": round(n_sets * nbytes / 1e6, 1), "dist": dist,
            "warmup_calls": info["warmup_calls"]}


def unpack_int4(p):
    import torch
    x = p.to(torch.int32) & 0xFF
    lo = ((x & 0x0F) << 28) >> 28
    hi = ((x & 0xF0) << 24) >> 28
    return torch.stack([lo, hi], dim=-1).reshape(*p.shape[:-1], 2 * p.shape[-1])


def bench_w4a16(llmik, M: int, K: int, N: int, steps: int, warmup: int, gs: int = 128,
                seed: int = 0):
    import torch
    dev = torch.device("cuda:0")
    nbytes = w4a16_bytes(M, K, N, gs)
    n_sets = n_sets_for(nbytes)
    gen = torch.Generator(device=dev).manual_seed(seed)
    sets = []
    for _ in range(n_sets):
        # random packed words: every nibble pattern, codes in [-8, 7]
        w = torch.randint(-2 ** 31, 2 ** 31 - 1, (K // 8, N), generator=gen, device=dev,
                          dtype=torch.int32)
        sc = (torch.rand((K // gs, N), generator=gen, device=dev) * 0.004 + 0.001).half()
        a = torch.randn((M, K), generator=gen, device=dev, dtype=torch.float16)
        sets.append((a, w, sc))
    a0, w0, s0 = sets[0]
    got = llmik.w4a16_gemm_f32out(a0, w0, s0, gs)
    ref = a0.double() @ unpack_w4(w0).double().mul(s0.double().repeat_interleave(gs, dim=0))
    err = gate(f"w4a16 M={M} K={K} N={N}", got, ref)
    del ref, got
    fns = [lambda s=s: llmik.w4a16_gemm(s[0], s[1], s[2], gs) for s in sets]
    us = time_steps(fns, warmup, steps)
    dist = sample_steps(fns)
    del sets, fns
    torch.cuda.empty_cache()
    gbs = nbytes / (us * 1e-6) / 1e9
    flops = 2.0 * M * K * N
    tf = flops / (us * 1e-6) / 1e12
    return {"name": "w4a16", "M": M, "K": K, "N": N, "us": round(us, 3), "bytes": nbytes,
            "GBps": round(gbs, 1), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
            "TFLOPs": round(tf, 2), "frac_mfma_fp16_peak": round(tf / MFMA_FP16_PEAK_TFLOPS, 4),
            "max_abs_err_f32out": err, "sets": n_sets,
            "rotated_MB": round(n_sets * nbytes / 1e6, 1), "dist": dist}


def bench_prefill(llmik, M: int, K: int, N: int, steps: int, warmup: int, gs: int = 128,
                  seed: int = 0):
    """Prefill-sized W4A16 (M >= 256): the reference's layer switches to
    w4a16_dequantize + F.linear at 256 rows (integration/w4a16_patch.py:89-116).
    Times that path (dequantise into a fresh fp16 [K, N], then torch.matmul,
    i.e. hipBLASLt) beside w4a16_gemm on the same inputs."""
    import torch
    dev = torch.device("cuda:0")
    kern = bench_w4a16(llmik, M, K, N, steps, warmup, gs, seed)
    nbytes = w4a16_bytes(M, K, N, gs)
    n_sets = n_sets_for(nbytes)
    gen = torch.Generator(device=dev).manual_seed(seed + 1)
    sets = []
    for _ in range(n_sets):
        w = torch.randint(-2 ** 31, 2 ** 31 - 1, (K // 8, N), generator=gen, device=dev,
                          dtype=torch.int32)
        sc = (torch.rand((K // gs, N), generator=gen, device=dev) * 0.004 + 0.001).half()
        a = torch.randn((M, K), generator=gen, device=dev, dtype=torch.float16)
        sets.append((a, w, sc))
    a0, w0, s0 = sets[0]
    got = torch.matmul(a0, llmik.w4a16_dequantize(w0, s0, gs))
    ref = a0.float() @ unpack_w4(w0).float().mul(s0.float().repeat_interleave(gs, dim=0))
    err = float((got.float() - ref).abs().max())
    del got, ref
    fns = [lambda s=s: torch.matmul(s[0], llmik.w4a16_dequantize(s[1], s[2], gs)) for s in sets]
    us = time_steps(fns, warmup, steps)
    del sets, fns
    torch.cuda.empty_cache()
    kern.update({"name": "w4a16_prefill", "dequant_matmul_us": round(us, 3),
                 "dequant_matmul_max_abs_err": err,
                 "dequant_matmul_TFLOPs": round(2.0 * M * K * N / (us * 1e-6) / 1e12, 2)})
    return kern


def bench_fp16_library_gemm(llmik, M: int, K: int, N: int, steps: int, warmup: int, gs: int = 128,
                            seed: int = 0) -> dict:
    """A reference point for the MFMA-bound W4A16 rows: the same product with
    the weights already dequantised to fp16 (w4a16_dequantize, outside the
    timed region) and multiplied by torch.matmul (hipBLASLt) over rotating
    sets of fp16 weights (4x the int4 weight bytes per call). It is the
    vendor library's time for the GEMM alone, with no dequantisation cost."""
    import torch
    dev = torch.device("cuda:0")
    nbytes = 2 * K * N + 2 * M * K + 2 * M * N
    n_sets = n_sets_for(nbytes)
    gen = torch.Generator(device=dev).manual_seed(seed + 2)
    sets = []
    for _ in range(n_sets):
        w = torch.randint(-2 ** 31, 2 ** 31 - 1, (K // 8, N), generator=gen, device=dev,
                          dtype=torch.int32)
        sc = (torch.rand((K // gs, N), generator=gen, device=dev) * 0.004 + 0.001).half()
        sets.append((torch.randn((M, K), generator=gen, device=dev, dtype=torch.float16),
                     llmik.w4a16_dequantize(w, sc, gs)))
        del w, sc
    fns = [lambda s=s: torch.matmul(s[0], s[1]) for s in sets]
    us = time_steps(fns, warmup, steps)
    del sets, fns
    torch.cuda.empty_cache()
    return {"fp16_library_gemm_us": round(us, 3),
            "fp16_library_gemm_TFLOPs": round(2.0 * M * K * N / (us * 1e-6) / 1e12, 2)}


def bench_decode_layer(llmik, n_layers: int, B: int, ctx: int, steps: int, warmup: int,
                       fused: bool = True) -> dict:
    """A decode step through `n_layers` Llama-3-8B layers (llmik_cuda.decode_layer:
    rmsnorm, W4A16 q/k/v/o/gate/up/down, rope, fp16 cache write, split-K
    attention over `ctx` tokens, silu_mul, residual adds), launched eagerly
    from Python and replayed from one HIP graph; `fused` picks the merged
    step (a DecodeStack: 7 launches per layer plus one) or the op-by-op
    17-launch one. Four layers hold ~950 MB of weights and caches, so the
    replays read HBM, not the Infinity Cache."""
    import torch
    from llmik_cuda.decode_layer import DecodeLayer, DecodeStack
    dev = torch.device("cuda:0")
    layers = []
    for i in range(n_layers):
        layer = DecodeLayer(4096, 32, 8, 14336, B, ctx, device=dev, seed=20 + i, fused=fused)
        g = torch.Generator(device=dev).manual_seed(40 + i)
        layer.kbuf.normal_(generator=g)
        layer.vbuf.normal_(generator=g)
        layers.append(layer)
    pos = ctx - 1
    x = torch.randn((B, 4096), generator=torch.Generator(device=dev).manual_seed(60), device=dev,
                    dtype=torch.float16)

    if fused:
        # the merged layers hand (h, mlp) on; the residual add rides in the
        # next layer's first RMSNorm launch
        stack = DecodeStack(layers)

        def model_step(inp):
            return stack.step(inp, pos)
    else:
        def model_step(inp):
            for layer in layers:
                inp = layer.step(inp, pos)
            return inp

    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for _ in range(warmup):
            model_step(x)
        stream.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(steps):
            model_step(x)
        end.record(stream)
    torch.cuda.synchronize()
    eager_us = start.elapsed_time(end) * 1000.0 / steps
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for _ in range(steps):
            model_step(x)
    with torch.cuda.stream(stream):
        graph.replay()
        torch.cuda.synchronize()
        start.record(stream)
        graph.replay()
        end.record(stream)
    torch.cuda.synchronize()
    graph_us = start.elapsed_time(end) * 1000.0 / steps
    del graph
    hidden, kv, inter, gs = 4096, 1024, 14336, 128
    w_elems = hidden * (2 * hidden + 2 * kv) + 3 * hidden * inter
    nbytes = w_elems // 2 + 2 * (w_elems // gs) + 2 * 2 * B * 8 * ctx * 128
    del layers
    torch.cuda.empty_cache()
    gbs = nbytes * n_layers / (graph_us * 1e-6) / 1e9
    return {"name": "decode_layer_step" if fused else "decode_layer_step_op_by_op",
            "layers": n_layers, "B": B, "ctx": ctx,
            "eager_us_per_layer": round(eager_us / n_layers, 3),
            "graph_us_per_layer": round(graph_us / n_layers, 3),
            "bytes_per_layer": nbytes, "graph_GBps": round(gbs, 1),
            "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}


def unpack_w4(w):
    import torch
    shifts = torch.arange(8, device=w.device, dtype=torch.int32).view(1, 8, 1) * 4
    x = (w.unsqueeze(1) << (28 - shifts)) >> 28
    return x.reshape(w.shape[0] * 8, w.shape[1])


def bench_writers(llmik, B: int, S: int, steps: int, warmup: int, seed: int = 0):
    import torch
    dev = torch.device("cuda:0")
    out = []
    gen = torch.Generator(device=dev).manual_seed(seed)
    x_bytes = B * 8 * S * 128 * 2
    n_sets = n_sets_for(x_bytes)
    xs = [torch.randn((B, 8, S, 128), generator=gen, device=dev, dtype=torch.float16)
          for _ in range(n_sets)]
    cases = [
        ("quantize_per_token_int8", lambda x: llmik.quantize_per_token(x),
         x_bytes + B * 8 * S * 128 + B * 8 * S * 2),
        ("quantize_k_groupwise_int4_g128", lambda x: llmik.quantize_k_per_channel_groupwise_int4(x, 128),
         x_bytes + B * 8 * S * 64 + B * 8 * ((S + 127) // 128) * 128 * 2),
        ("quantize_v_per_token_int4", lambda x: llmik.quantize_v_per_token_int4(x),
         x_bytes + B * 8 * S * 64 + B * 8 * S * 2),
    ]
    for name, fn, nbytes in cases:
        fns = [lambda x=x, fn=fn: fn(x) for x in xs]
        us = time_steps(fns, warmup, steps)
        gbs = nbytes / (us * 1e-6) / 1e9
        out.append({"name": name, "B": B, "S": S, "us": round(us, 3), "bytes": nbytes,
                    "GBps": round(gbs, 1), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)})
    del xs
    torch.cuda.empty_cache()
    return out


def bench_wquant(llmik, steps: int, warmup: int, seed: int = 0, gs: int = 128):
    """The offline weight path: quantize_pack_weights_int4 on an fp32 [K, N]
    weight (QuantizedLinear's convention), at the three Llama shapes. Bytes:
    the fp32 weight read once, the packed words and fp16 scales written.
    Gated bit-for-bit against a torch restatement of the reference's
    quantiser on the GPU (reference/quant_matmul_ref.py:39-88)."""
    import torch
    dev = torch.device("cuda:0")
    out = []
    gen = torch.Generator(device=dev).manual_seed(seed)
    for K, N in ((4096, 4096), (4096, 14336), (14336, 4096)):
        nbytes = K * N * 4 + K * N // 2 + (K // gs) * N * 2
        n_sets = n_sets_for(nbytes)
        ws = [torch.randn((K, N), generator=gen, device=dev) * 0.02 for _ in range(n_sets)]
        packed, s16 = llmik.quantize_pack_weights_int4(ws[0], gs)
        wg = ws[0].view(K // gs, gs, N)
        # Tensor / tensor: torch's GPU division by a Python scalar multiplies
        # by the reciprocal, which is not the reference's CPU true division.
        amax = wg.abs().amax(dim=1)
        scale = (amax / torch.full_like(amax, 7.0)).clamp(min=1e-8)
        q = (wg / scale.unsqueeze(1)).round().clamp(-7, 7).to(torch.int64).view(K, N)
        shifts = torch.arange(8, device=dev, dtype=torch.int64).view(1, 8, 1) * 4
        ref = ((q.view(K // 8, 8, N) & 0xF) << shifts).sum(dim=1)
        if not (torch.equal(packed.to(torch.int64) & 0xFFFFFFFF, ref) and
                torch.equal(s16, scale.half())):
            raise SystemExit(f"correctness gate failed for w4 quantiser K={K} N={N}")
        del packed, s16, wg, scale, q, ref
        fns = [lambda w=w: llmik.quantize_pack_weights_int4(w, gs) for w in ws]
        us = time_steps(fns, warmup, steps)
        gbs = nbytes / (us * 1e-6) / 1e9
        out.append({"name": "w4_quantize_pack_fp32", "K": K, "N": N, "us": round(us, 3),
                    "bytes": nbytes, "GBps": round(gbs, 1), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)})
        del ws, fns
        torch.cuda.empty_cache()
    return out


def bench_append(llmik, B: int, S: int, steps: int, warmup: int, seed: int = 0):
    """One decode step's KV append at cache length S (B batches, 8 kv heads,
    one new token): the cat-free caches (in-place writers) next to the
    reference cache's decode step (re-quantise the fp16 residual and
    torch.cat the whole packed cache, integration/kv_int4_cache.py:168-206),
    run on the GPU with the same kernels."""
    import torch
    from llmik_cuda.kv_cache import Int4KIVICache, Int8KVCache
    dev = torch.device("cuda:0")
    g = 128
    gen = torch.Generator(device=dev).manual_seed(seed)
    Hkv = 8
    n_new = max(steps, warmup) + 4
    k_pre = torch.randn((B, Hkv, S, 128), generator=gen, device=dev, dtype=torch.float16)
    v_pre = torch.randn((B, Hkv, S, 128), generator=gen, device=dev, dtype=torch.float16)
    toks = [(torch.randn((B, Hkv, 1, 128), generator=gen, device=dev, dtype=torch.float16),
             torch.randn((B, Hkv, 1, 128), generator=gen, device=dev, dtype=torch.float16))
            for _ in range(4)]
    out = []
    # cat-free INT4 KIVI and INT8: the cache holds S tokens, each step appends one
    for name, cache in (("kivi_int4_append_inplace", Int4KIVICache(B, Hkv, S + 2 * n_new + g, g, device=dev)),
                        ("int8_append_inplace", Int8KVCache(B, Hkv, S + 2 * n_new + g, device=dev))):
        cache.append(k_pre, v_pre)
        fns = [lambda c=cache, t=t: c.append(t[0], t[1]) for t in toks]
        us = time_steps(fns, warmup, steps)
        out.append({"name": name, "B": B, "S": S, "new_tokens": 1, "us": round(us, 3)})
        del cache
    # reference-style KIVI decode step: quantised full groups + an fp16
    # residual of r tokens, re-quantised and concatenated every step
    k_full, ks_full = llmik.quantize_k_per_channel_groupwise_int4(k_pre, g)
    v_full, vs_full = llmik.quantize_v_per_token_int4(v_pre)
    r = 37
    k_res = torch.randn((B, Hkv, r, 128), generator=gen, device=dev, dtype=torch.float16)
    v_res = torch.randn((B, Hkv, r, 128), generator=gen, device=dev, dtype=torch.float16)

    def cat_step():
        kq, ks = llmik.quantize_k_per_channel_groupwise_int4(k_res, g)
        vq, vs = llmik.quantize_v_per_token_int4(v_res)
        return (torch.cat([k_full, kq], dim=2), torch.cat([ks_full, ks], dim=2),
                torch.cat([v_full, vq], dim=2), torch.cat([vs_full, vs], dim=2))
    us = time_steps([cat_step], warmup, steps)
    out.append({"name": "kivi_int4_reference_cat_step", "B": B, "S": S, "residual_tokens": r,
                "us": round(us, 3)})
    del k_pre, v_pre, k_full, v_full
    torch.cuda.empty_cache()
    return out


# -------------------------------------------------------------- CPU baseline

def _timed_median(fn, budget_s: float, min_calls: int = 10, warmup: int = 3,
                  max_calls: int = 50):
    """Median microseconds of fn() after `warmup` calls: at least `min_calls`
    calls, more while the budget lasts (at most `max_calls`)."""
    for _ in range(warmup):
        fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < min_calls or (time.perf_counter() < t_end and len(times) < max_calls):
        t0 = time.perf_counter_ns()
        fn()
        times.append((time.perf_counter_ns() - t0) / 1e3)
    times.sort()
    return times[len(times) // 2], len(times)


def cpu_baseline(budget_s: float = 12.0):
    """The reference's eager fp32 decode attention (attention_ref.py:43-80,
    restated with torch CPU ops in oracle/torch_ref.py) at the headline shape
    on the host cores."""
    import torch
    from oracle import torch_ref as tr
    threads = tr.host_threads()
    torch.set_num_threads(threads)
    gen = torch.Generator().manual_seed(0)
    B, H, Hkv, S, D = 8, 32, 8, 4096, 128
    q = torch.randn((B, H, D), generator=gen).half()
    k = torch.randn((B, Hkv, S, D), generator=gen).half()
    v = torch.randn((B, Hkv, S, D), generator=gen).half()
    med, n = _timed_median(lambda: tr.eager_decode_attention(q, k, v, 1.0 / math.sqrt(D)), budget_s)
    return {"value": round(med, 1), "unit": "us", "cores": threads, "kind": "port",
            "sample": f"{n} full calls (after 3 warm-up) of oracle/torch_ref.py eager_decode_attention "
                      f"(torch CPU: repeat_interleave GQA, fp32 matmul, softmax, matmul, .to(fp16)) "
                      f"at B=8 H=32 Hkv=8 D=128 S=4096, median; torch.set_num_threads({threads}) "
                      f"from os.sched_getaffinity capped by OMP_NUM_THREADS"}


def cpu_details(budget_s: float = 3.0):
    """The reference's other CPU paths restated with torch ops
    (oracle/torch_ref.py): the KV quantisers on x.float() at B=8, S=4096,
    quantized_matmul_ref (with its per-call fp32 dequant) at M=1 on the three
    Llama shapes, and the numpy port of the attention for comparison; median
    of >= 10 calls after 3 warm-up calls each."""
    import numpy as np
    import torch
    from oracle import attention as oa
    from oracle import torch_ref as tr
    threads = tr.host_threads()
    torch.set_num_threads(threads)
    gen = torch.Generator().manual_seed(0)
    out = []
    x = torch.randn((8, 8, 4096, 128), generator=gen).half().float()
    for name, fn in (("quantize_per_token_int8", lambda: tr.quantize_per_token(x, 8)),
                     ("quantize_k_groupwise_int4_g128",
                      lambda: tr.quantize_per_channel_groupwise(x, 4, 128)),
                     ("quantize_v_per_token_int4", lambda: tr.quantize_per_token(x, 4))):
        us, n = _timed_median(fn, budget_s)
        out.append({"name": name, "B": 8, "S": 4096, "cpu_us": round(us, 1), "calls": n,
                    "cores": threads, "impl": "torch"})
    del x
    for K, N in ((4096, 4096), (4096, 14336), (14336, 4096)):
        q = torch.randint(-7, 8, (K, N), generator=gen, dtype=torch.int8)
        sc = (torch.rand((K // 128, N), generator=gen) * 0.004 + 0.001).half()
        act = torch.randn((1, K), generator=gen).half()
        us, n = _timed_median(lambda: tr.quantized_matmul_ref(act, q, sc, 128), budget_s)
        out.append({"name": "w4a16", "M": 1, "K": K, "N": N, "cpu_us": round(us, 1), "calls": n,
                    "cores": threads, "impl": "torch"})
        del q, sc, act
    rng = np.random.default_rng(0)
    qn = rng.standard_normal((8, 32, 128)).astype(np.float16)
    kn = rng.standard_normal((8, 8, 4096, 128)).astype(np.float16)
    vn = rng.standard_normal((8, 8, 4096, 128)).astype(np.float16)
    us, n = _timed_median(lambda: oa.decode_attention_expanded(qn, kn, vn), budget_s, min_calls=5)
    out.append({"name": "attn_fp16", "B": 8, "S": 4096, "cpu_us": round(us, 1), "calls": n,
                "impl": "numpy port (oracle/attention.py decode_attention_expanded)"})
    return out


# ------------------------------------------------------------------ floors

FLOOR_SIZES = (
    ("w4a16 (4096, 4096) M=1", w4a16_bytes(1, 4096, 4096)),
    ("w4a16 (4096, 14336) M=1", w4a16_bytes(1, 4096, 14336)),
    ("attention INT4 g128 B=8 S=4096", attn_bytes("int4", 8, 32, 8, 4096)),
    ("attention INT8 B=8 S=4096", attn_bytes("int8", 8, 32, 8, 4096)),
    ("attention A16 K and V", 2 * 8 * 8 * 4096 * 128 * 2),
    ("1 GiB", 1 << 30),
)
FLOOR_GRIDS = (256, 1024, 2048)
FLOOR_LOADS = (4, 8, 16)
# Read + write streams of the KV writers at B=8, S=4096 (one fp16 tensor in,
# codes out; the scales' 0.5 MB are left out): (name, bytes read, bytes
# written per 16 read).
FLOOR_RW = (
    ("INT8 per-token writer stream", 8 * 8 * 4096 * 128 * 2, 8),
    ("INT4 writer stream", 8 * 8 * 4096 * 128 * 2, 4),
)
FLOOR_RW_LOADS = (4, 8)


def bench_floors(steps: int, warmup: int) -> list:
    """What one launch costs before it does any work, and what the plainest
    read of a product kernel's bytes costs (llmik_diag_empty /
    llmik_diag_read of libllmik_diag.so, csrc_diag/diag.hip), timed like
    every other row: graph
    replay of `steps` calls over rotating windows of one buffer (>= 768 MiB
    in all). Each read size runs at every grid in FLOOR_GRIDS (workgroups of
    8 waves) and every depth in FLOOR_LOADS (16-byte loads per lane in
    flight); the empty kernel at 256 and 1024 workgroups. Rows are printed
    in the order their dispatches run; "calls" counts a row's dispatches
    (time_steps' untimed calls, then the timed replay of "reps" calls, which
    are the row's last). A last row per size names the fastest read."""
    import torch
    from llmik_cuda._lib import diag_check as check
    from llmik_cuda._lib import diag_lib
    lib = diag_lib()
    dev = torch.device("cuda:0")
    rows = []

    def stream_ptr():
        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    for nwg in (256, 1024):
        fn = (lambda n=nwg: check(lib.llmik_diag_empty(n, stream_ptr())))
        info = {}
        us = time_steps([fn], warmup, steps, info=info)
        rows.append({"name": f"empty kernel, {nwg} x 512 threads", "n_workgroups": nwg,
                     "calls": info["warmup_calls"] + steps, "reps": steps, "us": round(us, 3)})
        log(rows[-1])
    for name, nbytes in FLOOR_SIZES:
        nbytes = (nbytes + 255) // 256 * 256
        n_sets = n_sets_for(nbytes)
        buf = torch.randint(0, 256, (n_sets * nbytes,), dtype=torch.uint8, device=dev)
        size_rows = []
        for nwg in FLOOR_GRIDS:
            sink = torch.zeros(nwg * 8, dtype=torch.int32, device=dev)
            for L in FLOOR_LOADS:
                fns = [(lambda i=i, n=nwg, sk=sink, L=L:
                        check(lib.llmik_diag_read(ctypes.c_void_p(buf.data_ptr() + i * nbytes), nbytes,
                                                  ctypes.c_void_p(sk.data_ptr()), n, L, stream_ptr())))
                       for i in range(n_sets)]
                info = {}
                us = time_steps(fns, warmup, steps, info=info)
                reps = max(steps, n_sets)
                size_rows.append({"name": f"read {name}", "bytes": nbytes, "n_workgroups": nwg,
                                  "loads_per_lane": L, "windows": n_sets,
                                  "calls": info["warmup_calls"] + reps, "reps": reps,
                                  "us": round(us, 3), "TBps": round(nbytes / us / 1e6, 3)})
                log(size_rows[-1])
        best = min(size_rows, key=lambda r: r["us"])
        rows.extend(size_rows)
        rows.append({"name": f"fastest read {name}", "bytes": nbytes, "us": best["us"],
                     "TBps": best["TBps"], "n_workgroups": best["n_workgroups"],
                     "loads_per_lane": best["loads_per_lane"]})
        del buf
        torch.cuda.synchronize()
    for name, nbytes, wb in FLOOR_RW:
        out_bytes = nbytes // 16 * wb
        n_sets = n_sets_for(nbytes + out_bytes)
        src = torch.randint(0, 256, (n_sets * nbytes,), dtype=torch.uint8, device=dev)
        dst = torch.empty((n_sets * out_bytes,), dtype=torch.uint8, device=dev)
        size_rows = []
        for nwg in FLOOR_GRIDS:
            for L in FLOOR_RW_LOADS:
                fns = [(lambda i=i, n=nwg, L=L:
                        check(lib.llmik_diag_read_write(ctypes.c_void_p(src.data_ptr() + i * nbytes), nbytes,
                                                        ctypes.c_void_p(dst.data_ptr() + i * out_bytes), wb,
                                                        n, L, stream_ptr())))
                       for i in range(n_sets)]
                info = {}
                us = time_steps(fns, warmup, steps, info=info)
                reps = max(steps, n_sets)
                size_rows.append({"name": f"read+write {name}", "bytes_read": nbytes,
                                  "bytes_written": out_bytes, "n_workgroups": nwg, "loads_per_lane": L,
                                  "windows": n_sets, "calls": info["warmup_calls"] + reps, "reps": reps,
                                  "us": round(us, 3), "TBps": round((nbytes + out_bytes) / us / 1e6, 3)})
                log(size_rows[-1])
        best = min(size_rows, key=lambda r: r["us"])
        rows.extend(size_rows)
        rows.append({"name": f"fastest read+write {name}", "bytes_read": nbytes, "bytes_written": out_bytes,
                     "us": best["us"], "TBps": best["TBps"], "n_workgroups": best["n_workgroups"],
                     "loads_per_lane": best["loads_per_lane"]})
        del src, dst
        torch.cuda.synchronize()
    return rows


# ------------------------------------------------------------- HBM traffic

PMC_WORKLOADS = ("attn:fp16", "attn:int8", "attn:int4", "attn:int4g32", "attn:int4b64",
                 "w4a16:1", "w4a16:16", "w4a16:128", "w4a16:256", "w4a16:2048")


def pmc_workload(llmik, name: str, steps: int) -> None:
    """The program the rocprofv3 --pmc passes run: `steps` eager calls of one
    kernel family over rotating HBM-resident input sets (>= 768 MiB), then
    five plain 256 MiB device copies (torch copy_, a read and a write of
    known size) whose counter readings give the scale factor.

      attn:fp16 / attn:int8 / attn:int4 / attn:int4g32   B=8, S=4096 (the
          headline shape; INT4 at group 128 or 32, K with outlier channels)
      attn:int4b64                     INT4 g128 at B=64, S=8192
      w4a16:M                          M rows on (4096,4096), (4096,14336),
                                       (14336,4096), `steps` calls each, in
                                       that order
    """
    import torch
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(1)
    kind, arg = name.split(":")
    if kind == "attn":
        fmt = {"fp16": "fp16", "int8": "int8"}.get(arg, "int4")
        gs = 32 if arg == "int4g32" else 128
        B, S = (64, 8192) if arg == "int4b64" else (8, 4096)
        H, Hkv, D = 32, 8, 128
        n_sets = n_sets_for(attn_bytes(fmt, B, H, Hkv, S, D, gs))
        calls = []
        for _ in range(n_sets):
            q = torch.randn((B, H, D), generator=gen, device=dev, dtype=torch.float16)
            k = torch.randn((B, Hkv, S, D), generator=gen, device=dev, dtype=torch.float16)
            v = torch.randn((B, Hkv, S, D), generator=gen, device=dev, dtype=torch.float16)
            if fmt == "fp16":
                calls.append(lambda q=q, k=k, v=v: llmik.decode_attention(q, k, v, D ** -0.5))
                continue
            k[..., [3, 37, 71, 105]] *= 10
            if fmt == "int8":
                t = (q, *llmik.quantize_per_token(k), *llmik.quantize_per_token(v))
                calls.append(lambda t=t: llmik.decode_attention_int8(*t, D ** -0.5))
            else:
                t = (q, *llmik.quantize_k_per_channel_groupwise_int4(k, gs),
                     *llmik.quantize_v_per_token_int4(v))
                calls.append(lambda t=t: llmik.decode_attention_int4(*t, gs, D ** -0.5))
            del k, v
        torch.cuda.synchronize()
        log(f"pmc workload {name}: B={B} S={S} {fmt}" + (f" g{gs}" if fmt == "int4" else "")
            + f", {n_sets} input sets, {steps} calls")
        for i in range(steps):
            calls[i % n_sets]()
    elif kind == "w4a16":
        M = int(arg)
        for K, N in ((4096, 4096), (4096, 14336), (14336, 4096)):
            n_sets = n_sets_for(w4a16_bytes(M, K, N))
            sets = [(torch.randn((M, K), generator=gen, device=dev, dtype=torch.float16),
                     torch.randint(-2 ** 31, 2 ** 31 - 1, (K // 8, N), generator=gen, device=dev,
                                   dtype=torch.int32),
                     (torch.rand((K // 128, N), generator=gen, device=dev) * 0.004 + 0.001).half())
                    for _ in range(n_sets)]
            torch.cuda.synchronize()
            log(f"pmc workload {name}: M={M} K={K} N={N}, {n_sets} input sets, {steps} calls")
            for i in range(steps):
                llmik.w4a16_gemm(*sets[i % n_sets], 128)
            torch.cuda.synchronize()
            del sets
    else:
        raise SystemExit(f"unknown --pmc-workload {name}; one of {PMC_WORKLOADS}")
    torch.cuda.synchronize()
    src = torch.randint(0, 255, (256 << 20,), dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"pmc workload {name} done; 5 x 256 MiB copies")


def read_traffic():
    """HBM bytes per headline launch from the committed rocprofv3 --pmc
    summary (FETCH_SIZE + WRITE_SIZE, scaled by the copy kernel's readings),
    or None when the summary is absent."""
    if not TRAFFIC_FILE.exists():
        return None
    vals = {}
    for line in TRAFFIC_FILE.read_text().splitlines():
        parts = line.strip().strip("`").split()
        if len(parts) == 2 and parts[0] in ("fetch_bytes_per_launch", "write_bytes_per_launch"):
            vals[parts[0]] = int(parts[1])
    if len(vals) != 2:
        return None
    return vals["fetch_bytes_per_launch"] + vals["write_bytes_per_launch"]


# ------------------------------------------------------- compact JSON rows

_SHAPE_KEYS = ("fmt", "M", "K", "N", "B", "S", "layers", "ctx", "new_tokens", "residual_tokens")
_VALUE_KEYS = (("us", "us"), ("frac_hbm_peak", "frac"), ("frac_mfma_fp16_peak", "mfma_frac"),
               ("fp16_library_gemm_us", "lib_us"), ("dequant_matmul_us", "deq_lib_us"),
               ("eager_us_per_layer", "eager_us"), ("graph_us_per_layer", "graph_us"),
               ("max_abs_err", "err"), ("max_abs_err_f32out", "err"), ("cpu_us", "cpu_us"))


def compact(rows) -> dict:
    """{row key: {short value keys}} for the one-line JSON, so that every
    config's time and roofline fraction fits in a few KB (the full rows, with
    their distributions and byte counts, go to stderr as they are measured).
    The key is the row name followed by its shape, e.g. "attn_int8 B8 S4096"."""
    out = {}
    for r in rows or []:
        key = " ".join([r["name"]] + [f"{k}{r[k]}" for k in _SHAPE_KEYS if k in r])
        out[key] = {short: r[k] for k, short in _VALUE_KEYS if k in r and r[k] is not None}
    return out


# ---------------------------------------------------------------------- main

def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    # 16000 untimed calls (160 replays of the 100-call graph, ~0.4 s at A16):
    # the sustained-load warm-up time_steps asks for ("warmup_calls" adds the
    # eager call per input set and the settling replay).
    ap.add_argument("--warmup", type=int, default=16000)
    ap.add_argument("--no-details", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default="",
                    help="comma list: int8,int4,w4a16,prefill,layer,writers,append,sweep,wquant")
    ap.add_argument("--floors", action="store_true",
                    help="time the empty-kernel and plain-read floors (csrc_diag/diag.hip), print one "
                         "JSON line per row and exit")
    ap.add_argument("--pmc-workload", nargs="?", const="attn:fp16", default=None,
                    choices=PMC_WORKLOADS,
                    help="run a counter-collection program (one kernel family's calls, then "
                         "calibration copies) and exit; default attn:fp16, the headline")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; multi-GPU runs are out of scope "
                                   "(bench.py --gpus must be 1)"}))
        sys.exit(2)

    import torch
    import llmik_cuda as llmik
    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a GPU")
    log(f"device {torch.cuda.get_device_name(0)}; library {llmik.LIB_PATH}")
    if args.pmc_workload:
        pmc_workload(llmik, args.pmc_workload, args.steps)
        return
    if args.floors:
        for row in bench_floors(args.steps, args.warmup):
            print(json.dumps(row), flush=True)
        return

    only = set(filter(None, args.only.split(",")))
    want = (lambda k: not only or k in only)

    t_wall = time.perf_counter()
    head = bench_attention(llmik, "fp16", 8, 4096, args.steps, args.warmup, seed=1,
                           exact_steps=True)
    log(f"headline {head}")
    details = []
    if not args.no_details:
        if want("int8"):
            details.append(bench_attention(llmik, "int8", 8, 4096, 100, 10, seed=2))
            log(details[-1])
        if want("int4"):
            for B, S in ((8, 4096), (64, 8192)):
                details.append(bench_attention(llmik, "int4", B, S, 100 if B == 8 else 30, 10,
                                               gs=128, seed=3))
                log(details[-1])
            # group 32: the integration's default (integration/kv_int4_cache.py:73)
            details.append(bench_attention(llmik, "int4", 8, 4096, 100, 10, gs=32, seed=3))
            log(details[-1])
            details.append(bench_attention(llmik, "fp16", 64, 8192, 20, 5, seed=4))
            log(details[-1])
        if want("sweep"):
            for B, S in ((8, 1024), (8, 16384), (8, 32768), (1, 4096), (64, 4096)):
                details.append(bench_attention(llmik, "fp16", B, S, 50, 5, seed=5))
                log(details[-1])
        if want("w4a16"):
            for M in (1, 16, 128):
                for K, N in ((4096, 4096), (4096, 14336), (14336, 4096)):
                    details.append(bench_w4a16(llmik, M, K, N, 100 if M < 128 else 30, 10, seed=6))
                    if M == 128:
                        details[-1].update(bench_fp16_library_gemm(llmik, M, K, N, 30, 10, seed=6))
                    log(details[-1])
        if want("prefill"):
            for M in (256, 2048):
                for K, N in ((4096, 4096), (4096, 14336), (14336, 4096)):
                    details.append(bench_prefill(llmik, M, K, N, 20, 3, seed=10))
                    log(details[-1])
        if want("layer"):
            details.append(bench_decode_layer(llmik, 4, 8, 4096, 10, 3))
            details.append(bench_decode_layer(llmik, 4, 8, 4096, 10, 3, fused=False))
            log(details[-2:])
        if want("writers"):
            details.extend(bench_writers(llmik, 8, 4096, 50, 5, seed=7))
            log(details[-3:])
        if want("append"):
            details.extend(bench_append(llmik, 8, 4096, 50, 5, seed=8))
            log(details[-3:])
        if want("wquant"):
            details.extend(bench_wquant(llmik, 20, 3, seed=9))
            log(details[-3:])
    gpu_wall = time.perf_counter() - t_wall

    cpu = None
    cpu_more = None
    if not args.no_cpu:
        cpu = cpu_baseline()
        log(f"cpu baseline {cpu}")
        if not args.no_details:
            cpu_more = cpu_details()
            log(f"cpu details {cpu_more}")

    achieved = head["GBps"]
    line = {
        "metric": "decode-attn µs + % HBM peak; W4A16 GEMV µs at Llama-3-8B shapes",
        "value": head["us"],
        "unit": "us",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_calls": head["warmup_calls"],
        "ms_per_step": round(head["us"] / 1000.0, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {"workload": "fp16 split-K GQA decode attention (Llama-3-8B heads)",
                   "batch": 8, "n_heads": 32, "n_kv_heads": 8, "head_dim": 128,
                   "seqlen_kv": 4096, "kv_layout": "[B, Hkv, S, D] fp16 contiguous",
                   "input_sets_rotated": head["sets"]},
        # per-call distribution over 100 graph replays of >= 20 calls each
        "dist": head["dist"],
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": read_traffic(),
                     "traffic_source": ("profiles/" + TRAFFIC_FILE.name + ": rocprofv3 --pmc FETCH_SIZE "
                                        "+ WRITE_SIZE per headline launch, scaled by a copy of known "
                                        "size; committed, not measured in this run"),
                     "algorithmic_bytes_per_launch": head["bytes"]},
        "cpu_baseline": cpu,
        # every other config: {row: {us, frac of 8 TB/s, ...}}; full rows on stderr
        "details": compact(details),
        "cpu_details": compact(cpu_more),
        "gpu_wall_s": round(gpu_wall, 1),
    }
    print(json.dumps(line, separators=(",", ":")))


if __name__ == "__main__":
    main()
