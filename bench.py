"""Benchmark: affine 4-bit quantized matmul (MLX format) on one MI355X.

Metric: Q4 GEMV GB/s (% of HBM peak) at M=1; Q4 GEMM TFLOPS (% MFMA peak) at M=2048.

A step is one pass of the decode hot path over one decoder layer: the seven
projections q, k, v, o, gate, up, down of the Gemma-style 12B layer (hidden 3840,
16 q heads x 256, 8 KV heads x 256, FFN 15360), all 4-bit group-64 affine, at
batch M=1.  Weights are synthetic (N(0, 0.02) rounded to bf16, then quantized),
activations N(0, 1) in bf16.  `value` is algorithmic bytes per step (packed W +
bf16 scales/biases + bf16 x + bf16 y, see ALGO_BYTES) / measured time, with the
weights already resident in HBM.  The timing loop rotates over enough distinct
weight copies (>= 512 MiB) that the 256 MiB Infinity Cache cannot serve them.

Also reported: the dominant kernel's roofline (gate_proj GEMV, HIP-event timed
per launch), the prefill GEMM at M=2048, and the CPU baseline (the oracle's
fp32 loop on the host cores, on a bounded sample of the same workload).

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
SEED_BASE = 20260630
ROTATE_BYTES = 512 << 20


def algo_bytes(m: int, n: int, k: int, y_bytes: int = 2) -> int:
    """Packed W + bf16 scales and biases + bf16 x + y."""
    return n * k // 2 + 4 * n * (k // 64) + 2 * m * k + y_bytes * m * n


def algo_flops(m: int, n: int, k: int) -> int:
    return 2 * m * n * k


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def make_layer(torch, lib_mod, copies: int):
    """Quantize the layer once on the host (C oracle's quantizer, seeded), upload
    `copies` independent device copies."""
    from oracle import affine as A

    host = []
    for i, (name, n, k) in enumerate(LAYER):
        rng = np.random.Generator(np.random.PCG64(SEED_BASE + 1000 + i))
        w = rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)
        from oracle import c_oracle as C

        host.append(C.quantize(A.round_to_bf16(w)))
    layers = []
    for c in range(copies):
        layers.append([lib_mod.QuantizedLinear(*h) for h in host])
    return host, layers


def time_graph(torch, fn, steps: int, warmup: int):
    """Captures `fn` (one step) in a CUDA/HIP graph, replays warmup + steps, returns
    ms per step over exactly `steps` timed replays."""
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        fn()  # eager warm call on the capture stream
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
    for _ in range(steps):
        g.replay()
    t1.record(cur)
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / steps, g


def per_launch_ms(torch, launch, reps: int) -> float:
    """Average kernel duration from HIP events bracketing each single launch on the
    stream it runs on (the launches are issued one at a time, so each event pair
    covers one kernel)."""
    stream = torch.cuda.current_stream()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for i in range(reps):
        evs[i][0].record(stream)
        launch(i)
        evs[i][1].record(stream)
    torch.cuda.synchronize()
    d = sorted(a.elapsed_time(b) for a, b in evs)
    return float(np.mean(d[len(d) // 10: len(d) - len(d) // 10]))  # trimmed mean


def cpu_baseline(host, target_s: float = 12.0) -> dict:
    """The oracle's fp32 qmm loop (OpenMP over rows) on this host's cores, on a
    bounded sample: whole decoder-layer steps at M=1, repeated until ~target_s."""
    from oracle import affine as A
    from oracle import c_oracle as C

    threads = min(os.cpu_count() or 1, 16)
    xs = {k: A.make_activations(1, k, seed=SEED_BASE + k) for k in {k for _, _, k in LAYER}}
    outs = [np.empty((1, n), np.float32) for _, n, _ in LAYER]
    step_bytes = sum(algo_bytes(1, n, k) for _, n, k in LAYER)

    def one_step():
        for (name, n, k), h, o in zip(LAYER, host, outs):
            C.qmm_f32(xs[k], *h, threads=threads, out=o)

    one_step()
    t0 = time.perf_counter()
    reps = 0
    while True:
        one_step()
        reps += 1
        el = time.perf_counter() - t0
        if el >= target_s or reps >= 200:
            break
    return {
        "value": round(step_bytes * reps / el / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{reps} decoder-layer steps (7 projections, M=1) in {el:.1f} s; "
                  f"C restatement of the fp32 dequantize-and-dot loop, OpenMP over rows",
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-gemm", action="store_true")
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
    layer_w_bytes = sum(n * k // 2 + 4 * n * (k // 64) for _, n, k in LAYER)
    copies = max(2, -(-ROTATE_BYTES // layer_w_bytes))
    log(f"quantizing one decoder layer, {copies} device copies ({copies * layer_w_bytes / 2**20:.0f} MiB)")
    host, layers = make_layer(torch, Q, copies)

    xs = {k: torch.from_numpy(A.make_activations(16, k, seed=SEED_BASE + k).view(np.int16)).view(torch.bfloat16).cuda()
          for k in {k for _, _, k in LAYER}}
    ys = [torch.empty((16, n), dtype=torch.bfloat16, device="cuda") for _, n, _ in LAYER]

    def decode_step_fn(m):
        def fn():
            for c in range(copies):
                for (name, n, k), lin, y in zip(LAYER, layers[c], ys):
                    lin.forward(xs[k][:m], out=y[:m])
        return fn

    # --- headline: one decoder layer's projections at M=1, graph-replayed ---
    log("timing decode step M=1")
    ms_all, g1 = time_graph(torch, decode_step_fn(1), args.steps, args.warmup)
    ms_step = ms_all / copies
    step_bytes = sum(algo_bytes(1, n, k) for _, n, k in LAYER)
    value = step_bytes / (ms_step * 1e-3) / 1e9
    del g1

    per_proj = {}
    for m in (1, 4, 8):
        for i, (name, n, k) in enumerate(LAYER):
            ms = per_launch_ms(torch, lambda r, i=i, k=k, m=m: layers[r % copies][i].forward(xs[k][:m], out=ys[i][:m]),
                               reps=60)
            per_proj[f"{name}_m{m}"] = {"us": round(ms * 1e3, 2),
                                        "GBps": round(algo_bytes(m, n, k) / (ms * 1e-3) / 1e9, 1)}
    gate = per_proj["gate_proj_m1"]
    gate_bytes = algo_bytes(1, 15360, 3840)
    roofline = {
        "bound": "hbm",
        "achieved": gate["GBps"],
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(gate["GBps"] / HBM_PEAK_GBS, 4),
        "traffic": None,
        "kernel": "decode_kernel<1,4> gate_proj N=15360 K=3840 M=1",
        "algo_bytes_per_launch": gate_bytes,
        "avg_launch_us": gate["us"],
    }

    # --- lm_head decode (566 MB, naturally HBM resident) ---
    lm = None
    try:
        from oracle import c_oracle as C

        rng = np.random.Generator(np.random.PCG64(SEED_BASE + 3000))
        log("quantizing lm_head 262144x3840")
        lm_w = rng.standard_normal((262144, HIDDEN), dtype=np.float32) * np.float32(0.02)
        lm_lin = Q.QuantizedLinear(*C.quantize(A.round_to_bf16(lm_w)))
        del lm_w
        y_lm = torch.empty((16, 262144), dtype=torch.bfloat16, device="cuda")
        lm = {}
        for m in (1, 8, 16):
            ms = per_launch_ms(torch, lambda r, m=m: lm_lin.forward(xs[HIDDEN][:m], out=y_lm[:m]), reps=20)
            lm[f"m{m}"] = {"us": round(ms * 1e3, 1), "GBps": round(algo_bytes(m, 262144, HIDDEN) / (ms * 1e-3) / 1e9, 1)}
        lm_lin.close()
    except Exception as e:  # memory or build problems should not hide the headline
        lm = {"error": str(e)}

    # --- prefill GEMM at M=2048 (gate shape) ---
    gemm = None
    if not args.no_gemm:
        xm = torch.from_numpy(A.make_activations(2048, HIDDEN, seed=SEED_BASE + 2, outliers=True).view(np.int16)) \
            .view(torch.bfloat16).cuda()
        ym = torch.empty((2048, 15360), dtype=torch.bfloat16, device="cuda")
        lin = layers[0][4]
        ms = per_launch_ms(torch, lambda r: lin.forward(xm, out=ym), reps=5)
        tflops = algo_flops(2048, 15360, HIDDEN) / (ms * 1e-3) / 1e12
        gemm = {"shape": "gate_proj M=2048 N=15360 K=3840", "ms": round(ms, 3), "TFLOPS": round(tflops, 1),
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
                        "4-bit group-64 affine, hidden 3840, FFN 15360",
            "global_batch": 1,
            "parallelism": "none (1 GPU)",
            "weight_copies_rotated": copies,
        },
        "pct_hbm_peak": round(value / HBM_PEAK_GBS * 100, 2),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "decode_per_projection": per_proj,
        "lm_head": lm,
        "prefill_gemm": gemm,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
