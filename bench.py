"""Benchmark: affine 4-bit quantized matmul (MLX format) on one MI355X.

Metric: Q4 GEMV GB/s (% of HBM peak) at M=1; Q4 GEMM TFLOPS (% MFMA peak) at M=2048.

A step is one pass of the decode hot path over one decoder layer: the seven
projections q, k, v, o, gate, up, down of the Gemma-style 12B layer (hidden 3840,
16 q heads x 256, 8 KV heads x 256, FFN 15360), all 4-bit group-64 affine, at
batch M=1.  They run as the model's data dependencies allow: q|k|v as one fused
projection (weights concatenated along N at load, all read the same x), then o,
then gate|up fused, then down.  Weights are synthetic (N(0, 0.02) rounded to bf16,
then quantized), activations N(0, 1) in bf16.  `value` is algorithmic bytes per
step (packed W + bf16 scales/biases + bf16 x + bf16 y, see algo_bytes) / measured
step time, with the weights already resident in HBM, timed over graph replays of
the step.  The loop rotates over enough distinct weight copies (>= 512 MiB) that
the 256 MiB Infinity Cache cannot serve them.

Also reported: the dominant kernel's roofline (the fused gate|up GEMV, timed per
launch from graph replays of back-to-back launches), every projection at M = 1, 4,
8, the lm_head at M = 1, 8, 16, the prefill GEMM at M=2048, and the CPU baseline
(the oracle's fp32 loop on the host cores, on a bounded sample of the same work).

    python bench.py [--steps K] [--warmup W] [--no-cpu] [--no-gemm]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "Q4 GEMV GB/s (% of HBM peak) at M=1; Q4 GEMM TFLOPS (% MFMA peak) at M=2048"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
HIDDEN = 3840
# (name, N, K) of one decoder layer
LAYER = [
    ("q_proj", 4096, 3840),
    ("k_proj", 2048, 3840),
    ("v_proj", 2048, 3840),
    ("o_proj", 3840, 4096),
    ("gate_proj", 15360, 3840),
    ("up_proj", 15360, 3840),
    ("down_proj", 3840, 15360),
]
# launches of one decode step: projections sharing x are fused along N
STEP = [("qkv_proj", ("q_proj", "k_proj", "v_proj")), ("o_proj", ("o_proj",)),
        ("gate_up_proj", ("gate_proj", "up_proj")), ("down_proj", ("down_proj",))]
SEED_BASE = 20260630
ROTATE_BYTES = 512 << 20


def algo_bytes(m: int, n: int, k: int, y_bytes: int = 2) -> int:
    """Packed W + bf16 scales and biases + bf16 x + y."""
    return n * k // 2 + 4 * n * (k // 64) + 2 * m * k + y_bytes * m * n


def algo_flops(m: int, n: int, k: int) -> int:
    return 2 * m * n * k


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def quantized_layer():
    """The seven projections, quantized on the host from seeded weights."""
    from oracle import affine as A
    from oracle import c_oracle as C

    host = {}
    for i, (name, n, k) in enumerate(LAYER):
        rng = np.random.Generator(np.random.PCG64(SEED_BASE + 1000 + i))
        w = rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)
        host[name] = C.quantize(A.round_to_bf16(w))
    return host


def fused_triple(host, names):
    parts = [host[n] for n in names]
    return tuple(np.ascontiguousarray(np.concatenate([p[j] for p in parts], axis=0)) for j in range(3))


def graph_ms(torch, fn, replays: int, warmup: int) -> float:
    """Captures fn() in a HIP graph, replays it warmup + replays times on the
    current stream and returns ms per replay over exactly `replays` timed replays
    (HIP events on the stream the kernels run on, synchronized on both sides)."""
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        fn()  # eager warm-up on the capture stream
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        fn()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    cur = torch.cuda.current_stream()
    t0.record(cur)
    for _ in range(replays):
        g.replay()
    t1.record(cur)
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / replays
    del g
    return ms


def kernel_us(torch, Q, triple, m: int, k: int, n: int, xdev, reps_per_graph: int = 40) -> float:
    """Average duration of one forward launch: back-to-back launches over rotated
    weight copies, captured in a graph and replayed."""
    wbytes = n * k // 2 + 4 * n * (k // 64)
    copies = max(2, -(-ROTATE_BYTES // wbytes))
    lins = [Q.QuantizedLinear(*triple) for _ in range(copies)]
    y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    launches = max(copies, (reps_per_graph // copies) * copies)

    def fn():
        for i in range(launches):
            lins[i % copies].forward(xdev[:m], out=y)

    ms = graph_ms(torch, fn, replays=10, warmup=2)
    for lin in lins:
        lin.close()
    return ms * 1e3 / launches


def cpu_baseline(host, target_s: float = 12.0) -> dict:
    """The oracle's fp32 qmm loop (OpenMP over rows) on this host's cores, on a
    bounded sample: whole decoder-layer steps at M=1, repeated until ~target_s."""
    from oracle import affine as A
    from oracle import c_oracle as C

    threads = min(os.cpu_count() or 1, 16)
    xs = {k: A.make_activations(1, k, seed=SEED_BASE + k) for k in {k for _, _, k in LAYER}}
    outs = {name: np.empty((1, n), np.float32) for name, n, _ in LAYER}
    step_bytes = sum(algo_bytes(1, n, k) for _, n, k in LAYER)

    def one_step():
        for name, n, k in LAYER:
            C.qmm_f32(xs[k], *host[name], threads=threads, out=outs[name])

    one_step()
    t0 = time.perf_counter()
    reps = 0
    while True:
        one_step()
        reps += 1
        el = time.perf_counter() - t0
        if el >= target_s or reps >= 2000:
            break
    return {
        "value": round(step_bytes * reps / el / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{reps} decoder-layer steps (7 projections, M=1) in {el:.1f} s; C restatement of the "
                  f"fp32 dequantize-and-dot loop (oracle/q4_oracle.c), OpenMP over rows, {threads} threads",
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-gemm", action="store_true")
    ap.add_argument("--quick", action="store_true", help="headline only (skip the per-shape sweeps)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        return 2

    import torch

    import helios_amd
    from helios_amd import qmm as Q
    from oracle import affine as A

    helios_amd.load_library()
    torch.cuda.set_device(0)
    log("quantizing one decoder layer")
    host = quantized_layer()
    fused = {name: fused_triple(host, parts) for name, parts in STEP}
    fused_nk = {name: (sum(dict((l[0], l[1]) for l in LAYER)[p] for p in parts), dict((l[0], l[2]) for l in LAYER)[parts[0]])
                for name, parts in STEP}
    layer_w_bytes = sum(n * k // 2 + 4 * n * (k // 64) for _, n, k in LAYER)
    copies = max(2, -(-ROTATE_BYTES // layer_w_bytes))
    log(f"uploading {copies} copies of the layer ({copies * layer_w_bytes / 2**20:.0f} MiB)")
    layers = [{name: Q.QuantizedLinear(*fused[name]) for name, _ in STEP} for _ in range(copies)]

    xs = {k: torch.from_numpy(A.make_activations(16, k, seed=SEED_BASE + k).view(np.int16)).view(torch.bfloat16).cuda()
          for k in {k for _, _, k in LAYER}}
    ys = {name: torch.empty((16, n), dtype=torch.bfloat16, device="cuda") for name, (n, _) in fused_nk.items()}

    def step_fn(m):
        def fn():
            for c in range(copies):
                for name, _ in STEP:
                    n, k = fused_nk[name]
                    layers[c][name].forward(xs[k][:m], out=ys[name][:m])
        return fn

    # --- headline: one decoder layer's projections at M=1 (4 launches), graph-replayed ---
    log(f"timing decode step M=1 ({args.warmup} warmup + {args.steps} timed replays)")
    ms_step = graph_ms(torch, step_fn(1), args.steps, args.warmup) / copies
    step_bytes = sum(algo_bytes(1, n, k) for _, n, k in LAYER)
    value = step_bytes / (ms_step * 1e-3) / 1e9
    step_by_m = {}
    for m in ((4, 8) if not args.quick else ()):
        ms_m = graph_ms(torch, step_fn(m), max(10, args.steps // 4), 2) / copies
        step_by_m[f"m{m}"] = {"ms_per_step": round(ms_m, 5),
                              "GBps": round(sum(algo_bytes(m, n, k) for _, n, k in LAYER) / (ms_m * 1e-3) / 1e9, 1)}
    for lin_set in layers:
        for lin in lin_set.values():
            lin.close()
    del layers

    # --- dominant kernel: fused gate|up GEMV at M=1 ---
    n_gu, k_gu = fused_nk["gate_up_proj"]
    us_gu = kernel_us(torch, Q, fused["gate_up_proj"], 1, k_gu, n_gu, xs[k_gu])
    gu_bytes = algo_bytes(1, n_gu, k_gu)
    gu_gbs = gu_bytes / (us_gu * 1e-6) / 1e9
    roofline = {
        "bound": "hbm",
        "achieved": round(gu_gbs, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(gu_gbs / HBM_PEAK_GBS, 4),
        "traffic": None,
        "kernel": f"decode_stream_kernel<1,4> gate|up fused N={n_gu} K={k_gu} M=1",
        "algo_bytes_per_launch": gu_bytes,
        "avg_launch_us": round(us_gu, 3),
    }

    per_proj = {}
    lm = None
    if not args.quick:
        for m in (1, 4, 8):
            for name, n, k in LAYER:
                us = kernel_us(torch, Q, host[name], m, k, n, xs[k])
                per_proj[f"{name}_m{m}"] = {"us": round(us, 2), "GBps": round(algo_bytes(m, n, k) / (us * 1e-6) / 1e9, 1)}
            for name, _ in STEP:
                if len(dict(STEP)[name]) > 1:
                    n, k = fused_nk[name]
                    us = kernel_us(torch, Q, fused[name], m, k, n, xs[k])
                    per_proj[f"{name}_m{m}"] = {"us": round(us, 2),
                                                "GBps": round(algo_bytes(m, n, k) / (us * 1e-6) / 1e9, 1)}
        try:
            from oracle import c_oracle as C

            log("quantizing lm_head 262144x3840")
            rng = np.random.Generator(np.random.PCG64(SEED_BASE + 3000))
            lm_w = rng.standard_normal((262144, HIDDEN), dtype=np.float32) * np.float32(0.02)
            lm_triple = C.quantize(A.round_to_bf16(lm_w))
            del lm_w
            lm = {}
            for m in (1, 8, 16):
                us = kernel_us(torch, Q, lm_triple, m, HIDDEN, 262144, xs[HIDDEN], reps_per_graph=4)
                lm[f"m{m}"] = {"us": round(us, 1), "GBps": round(algo_bytes(m, 262144, HIDDEN) / (us * 1e-6) / 1e9, 1)}
            del lm_triple
        except Exception as e:  # memory or build problems should not hide the headline
            lm = {"error": str(e)}

    # --- prefill GEMM at M=2048 (gate shape) ---
    gemm = None
    if not args.no_gemm:
        xm = torch.from_numpy(A.make_activations(2048, HIDDEN, seed=SEED_BASE + 2, outliers=True).view(np.int16)) \
            .view(torch.bfloat16).cuda()
        ym = torch.empty((2048, 15360), dtype=torch.bfloat16, device="cuda")
        lin = Q.QuantizedLinear(*host["gate_proj"])
        ms = graph_ms(torch, lambda: lin.forward(xm, out=ym), replays=5, warmup=1)
        lin.close()
        tflops = algo_flops(2048, 15360, HIDDEN) / (ms * 1e-3) / 1e12
        gemm = {"shape": "gate_proj M=2048 N=15360 K=3840", "ms": round(ms, 4), "TFLOPS": round(tflops, 1),
                "frac_bf16_peak": round(tflops / BF16_PEAK_TFLOPS, 4)}

    cpu = None
    if not args.no_cpu:
        log("CPU baseline")
        cpu = cpu_baseline(host)

    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "one Gemma-style 12B decoder layer's 7 projections (q,k,v,o,gate,up,down) at decode M=1, "
                        "4-bit group-64 affine, hidden 3840, FFN 15360; launched as qkv, o, gate_up, down",
            "global_batch": 1,
            "parallelism": "none (1 GPU)",
            "weight_copies_rotated": copies,
        },
        "pct_hbm_peak": round(value / HBM_PEAK_GBS * 100, 2),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "decode_step_by_m": step_by_m,
        "decode_per_projection": per_proj,
        "lm_head": lm,
        "prefill_gemm": gemm,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
