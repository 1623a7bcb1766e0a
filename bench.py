"""Benchmark: affine 4-bit quantized matmul (MLX format) on one MI355X.

Metric: Q4 GEMV GB/s (% of HBM peak) at M=1; Q4 GEMM TFLOPS (% MFMA peak) at M=2048.

A step is one pass of the decode hot path over one decoder layer: the seven
projections q, k, v, o, gate, up, down of the Gemma-style 12B layer (hidden 3840,
16 q heads x 256, 8 KV heads x 256, FFN 15360), all 4-bit group-64 affine, at
batch M=1.  They run as the model's data dependencies allow: q|k|v as one fused
projection (weights concatenated along N at load, all read the same x), then o,
then gate and up as one pair with the GeGLU epilogue (gemma4_qgeglu_forward, whose
output h feeds down), then down.  Weights are synthetic (N(0, 0.02) rounded to bf16,
then quantized), activations N(0, 1) in bf16.  `value` is algorithmic bytes per
step (packed W + bf16 scales/biases + bf16 x + bf16 y of the seven projections,
see algo_bytes) / measured step time, with the weights already resident in HBM, timed over graph replays of
the step.  The loop rotates over enough distinct weight copies (>= 512 MiB) that
the 256 MiB Infinity Cache cannot serve them.

The headline replays run `--warmup` times, then untimed for `--settle-ms` of wall
time (the GPU's clock ramps for a few milliseconds once it gets busy, so a handful of
replays would time the ramp), then exactly `--steps` timed replays.

Also reported: the single GEMV of gate_proj's shape at M=1 (x [1, 3840], W [15360, 3840])
as its own field, the dominant kernel's roofline (the gate|up GeGLU pair at M=1, timed per launch
from graph replays of back-to-back launches), every projection at M = 1, 4, 8, the
lm_head at M = 1, 8, 16, the prefill GEMM at M = 256 (the reference's long-context
chunk), 512 and 2048 (the seven projections, the GeGLU pair and the real 12B's
full-attention shapes), practical peaks (a 1 GiB copy, a read-only streaming kernel,
hipBLASLt on the gate shape), and the CPU baseline (the oracle's fp32 loop on the host
cores, on bounded samples of that GEMV, one decoder layer at M = 1, the lm_head at M = 1
and one layer's prefill at M = 512, all threads and one thread).

    python bench.py [--steps K] [--warmup W] [--no-cpu] [--no-gemm] [--quick]
    python bench.py --roofline-only   # the dominant kernel and a 1 GiB copy only (for rocprofv3)
    python bench.py --prefill-only    # the prefill GEMM sweep only (for rocprofv3 kernel traces)

`roofline.traffic` is the HBM bytes one launch of the dominant kernel moves, from
rocprofv3 FETCH_SIZE and WRITE_SIZE passes over `--roofline-only`, each scaled by
what the same counter reads for the 1 GiB copy; it is read from
profiles/gate_up_decode_m1_traffic.json when that file describes the same launch.
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
# launches of one decode step: projections sharing x are fused along N; gate and up
# form the GeGLU pair (output h [M, 15360])
STEP = [("qkv_proj", ("q_proj", "k_proj", "v_proj")), ("o_proj", ("o_proj",)),
        ("gate_up_geglu", ("gate_proj", "up_proj")), ("down_proj", ("down_proj",))]
PAIR = "gate_up_geglu"
SEED_BASE = 20260630
ROTATE_BYTES = 512 << 20
COPY_BYTES = 1 << 30
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gate_up_decode_m1_traffic.json")
# launches of the same step under the reference's own call structure (q, k and v
# each their own quantized_linear, native_model.cc:993, :1005, :1009; gate and up as
# the GeGLU pair; down)
STEP_UNFUSED = [("q_proj", ("q_proj",)), ("k_proj", ("k_proj",)), ("v_proj", ("v_proj",)), ("o_proj", ("o_proj",)),
                ("gate_up_geglu", ("gate_proj", "up_proj")), ("down_proj", ("down_proj",))]
# the kernel that runs the gate|up GeGLU pair at M = 1: the int8 matrix-core decode
# kernel, 1920 row blocks dealt round a grid of three 8-wave workgroups per CU with
# one chunk in flight per wave
DOM_KERNEL = "decode_limb_kernel"
DOM_INSTANCE = "decode_limb_kernel<1,8,true>"


def weight_bytes(n: int, k: int) -> int:
    """Resident bytes of one 4-bit projection: codes plus bf16 scale and bias per group."""
    return n * k // 2 + 4 * n * (k // 64)


def algo_bytes(m: int, n: int, k: int, y_bytes: int = 2) -> int:
    """Packed W + bf16 scales and biases + bf16 x + y."""
    return n * k // 2 + 4 * n * (k // 64) + 2 * m * k + y_bytes * m * n


def pair_algo_bytes(m: int, f: int, k: int) -> int:
    """The GeGLU pair: both packed weights with scales and biases + bf16 x + bf16 h."""
    return 2 * f * k // 2 + 2 * 4 * f * (k // 64) + 2 * m * k + 2 * m * f


def algo_flops(m: int, n: int, k: int) -> int:
    return 2 * m * n * k


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def synthetic_weights(n: int, k: int, seed: int):
    """MLX-format triple (host numpy: uint32 codes, bf16 scale and bias bits) of a
    seeded W ~ N(0, 0.02) [n, k] rounded to bf16, quantized 4-bit group-64 with the
    package's quantizer (on the GPU when there is one)."""
    import torch
    from helios_amd.quantize import quantize

    rng = np.random.Generator(np.random.PCG64(seed))
    w = torch.from_numpy(rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
    if torch.cuda.is_available():
        w = w.cuda()
    wq, s, b = quantize(w.bfloat16())
    return (wq.cpu().numpy().view(np.uint32), s.view(torch.int16).cpu().numpy().view(np.uint16),
            b.view(torch.int16).cpu().numpy().view(np.uint16))


def synthetic_activations(m: int, k: int, seed: int, outliers: bool = False) -> np.ndarray:
    """bf16 bits of a seeded x ~ N(0, 1) [m, k]; with ``outliers`` 1% of the entries
    are scaled by 20 (the prefill workloads' activation outliers)."""
    import torch

    rng = np.random.Generator(np.random.PCG64(seed))
    x = rng.standard_normal((m, k), dtype=np.float32)
    if outliers:
        x = np.where(rng.random((m, k)) < 0.01, x * np.float32(20), x).astype(np.float32)
    return torch.from_numpy(x).bfloat16().view(torch.int16).numpy().view(np.uint16)


def quantized_layer():
    """The seven projections from seeded weights."""
    return {name: synthetic_weights(n, k, SEED_BASE + 1000 + i) for i, (name, n, k) in enumerate(LAYER)}


def fused_triple(host, names):
    parts = [host[n] for n in names]
    return tuple(np.ascontiguousarray(np.concatenate([p[j] for p in parts], axis=0)) for j in range(3))


def settle(torch, replay, settle_ms: float) -> int:
    """Replays untimed until settle_ms of wall time have passed (the GPU's clock ramps
    for a few milliseconds once it gets busy); returns the replays spent.  Batches are
    synchronized, so the wall time is the GPU's."""
    t0 = time.perf_counter()
    n, batch = 0, 1
    while (time.perf_counter() - t0) * 1e3 < settle_ms:
        t1 = time.perf_counter()
        for _ in range(batch):
            replay()
        torch.cuda.synchronize()
        n += batch
        if (time.perf_counter() - t1) * 1e3 < 2.0:
            batch *= 2
    return n


def graph_ms(torch, fn, replays: int, warmup: int, settle_ms: float = 0.0, info: dict | None = None) -> float:
    """Captures fn() in a HIP graph, replays it `warmup` times, then (settle_ms > 0)
    untimed until settle_ms of wall time have passed, and returns ms per replay over
    exactly `replays` timed replays (HIP events on the stream the kernels run on,
    synchronized on both sides)."""
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
    if settle_ms > 0:
        n = settle(torch, g.replay, settle_ms)
        if info is not None:
            info["settle_replays"] = n
            info["settle_ms"] = settle_ms
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


def graph_ms_steady(torch, fn, settle_ms: float = 50.0, time_ms: float = 20.0) -> float:
    """graph_ms for the per-shape sweeps: the clock ramps for a few milliseconds once
    the GPU gets busy, so replays run untimed for about settle_ms first and the timed
    replays cover about time_ms (both from a first estimate of one replay)."""
    est = max(graph_ms(torch, fn, replays=3, warmup=1), 1e-3)
    return graph_ms(torch, fn, replays=max(10, int(time_ms / est) + 1), warmup=max(2, int(settle_ms / est) + 1))


def kernel_us(torch, make, m: int, k: int, n: int, xdev, wbytes: int, reps_per_graph: int = 40) -> float:
    """Average duration of one forward launch (of make(), output [m, n]): back-to-back
    launches over rotated weight copies, captured in a graph and replayed."""
    copies = max(2, -(-ROTATE_BYTES // wbytes))
    lins = [make() for _ in range(copies)]
    y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    launches = max(copies, (reps_per_graph // copies) * copies)

    def fn():
        for i in range(launches):
            lins[i % copies].forward(xdev[:m], out=y)

    ms = graph_ms_steady(torch, fn)
    for lin in lins:
        lin.close()
    return ms * 1e3 / launches


def copy_gbs(torch, nbytes: int = COPY_BYTES, reps: int = 20) -> float:
    """Practical HBM rate: a plain device-to-device copy of nbytes (read + write
    counted), timed with events on the current stream."""
    src = torch.ones(nbytes // 2, dtype=torch.bfloat16, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(reps):
        dst.copy_(src)
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / reps
    del src, dst
    return 2 * nbytes / (ms * 1e-3) / 1e9


def read_gbs(torch, nbytes: int = COPY_BYTES, reps: int = 20) -> dict:
    """Practical HBM read rate: the read-only streaming kernel of libhbm_probe.so
    (each wave one contiguous 8 KiB run per step, neighbouring waves neighbouring
    runs) over nbytes, the best over a few grid sizes; graph-replayed after a wall-time
    settle, timed with events on the replay stream."""
    import ctypes

    from helios_amd import build as hbuild

    lib = ctypes.CDLL(hbuild.PROBE_PATH)
    lib.hbm_read_probe.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    lib.hbm_read_probe.restype = ctypes.c_int
    buf = torch.ones(nbytes // 4, dtype=torch.int32, device="cuda")
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    best = None
    for per_cu in (2, 4, 8):
        wgs = cus * per_cu
        sink = torch.empty(wgs * 4, dtype=torch.int32, device="cuda")

        def fn():
            st = torch.cuda.current_stream().cuda_stream
            if lib.hbm_read_probe(buf.data_ptr(), nbytes, sink.data_ptr(), wgs, ctypes.c_void_p(st)) != 0:
                raise RuntimeError("hbm_read_probe launch failed")

        ms = graph_ms(torch, fn, replays=reps, warmup=2, settle_ms=30.0)
        gbs = nbytes / (ms * 1e-3) / 1e9
        if best is None or gbs > best["GBps"]:
            best = {"GBps": round(gbs, 1), "workgroups_per_cu": per_cu, "bytes": nbytes}
        del sink
    del buf
    return best


def dense_gemm_tflops(torch, m: int, n: int, k: int, reps: int = 20) -> float:
    """Practical bf16 MFMA rate on the same GEMM shape: torch's bf16 linear (hipBLASLt)
    on a dense bf16 weight."""
    a = torch.randn(m, k, dtype=torch.bfloat16, device="cuda")
    w = torch.randn(n, k, dtype=torch.bfloat16, device="cuda")
    for _ in range(3):
        torch.nn.functional.linear(a, w)
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(reps):
        torch.nn.functional.linear(a, w)
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / reps
    del a, w
    return algo_flops(m, n, k) / (ms * 1e-3) / 1e12


def recorded_traffic(kernel: str, algo: int):
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3
    counter passes, if they describe this launch."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None, None
    if t.get("kernel") != kernel or t.get("algo_bytes_per_launch") != algo:
        return None, None
    return t.get("traffic_bytes_per_launch"), t


def _csv_rows(d: str, suffix: str):
    import csv
    import glob

    files = sorted(glob.glob(os.path.join(d, "**", "*" + suffix), recursive=True))
    if not files:
        raise SystemExit(f"no *{suffix} under {d}")
    with open(files[0], newline="") as f:
        return list(csv.DictReader(f))


def summarize_profiles(stats_dir: str, fetch_dir: str, write_dir: str, line_file: str, command: str) -> None:
    """Turns rocprofv3 output over `bench.py --roofline-only` into the committed
    summaries: the kernel-trace statistics (average launch duration of the dominant
    kernel, to compare with the bench's own HIP-event figure) and the HBM traffic per
    launch from the FETCH_SIZE / WRITE_SIZE passes, each scaled by what the same
    counter reads for the 1 GiB copy."""
    with open(line_file) as f:
        line = json.loads([l for l in f if l.startswith("{")][-1])
    stats = _csv_rows(stats_dir, "kernel_stats.csv")

    def short(name: str) -> str:
        return name.replace("void ", "").replace("(anonymous namespace)::", "").split("(")[0][:90]

    def per_dispatch(rows, counter, match, largest=False):
        vals = [float(r["Counter_Value"]) for r in rows if r["Counter_Name"] == counter and match(r["Kernel_Name"])]
        if not vals:
            raise SystemExit(f"no {counter} rows for the kernel")
        if largest:  # the 1 GiB copies, not the runtime's small blits (handle creation's)
            vals = [v for v in vals if v >= 0.5 * max(vals)]
        return sum(vals) / len(vals), len(vals)

    is_dom = lambda n: DOM_KERNEL in n  # noqa: E731
    # the runtime's blit kernel of the 1 GiB device copy (torch's own dtype-conversion
    # kernels also carry "copy" in their names)
    is_copy = lambda n: "rocclr_copybuffer" in n.lower()  # noqa: E731
    fetch_rows = _csv_rows(fetch_dir, "counter_collection.csv")
    write_rows = _csv_rows(write_dir, "counter_collection.csv")
    f_dom, n_fd = per_dispatch(fetch_rows, "FETCH_SIZE", is_dom)
    f_cpy, n_fc = per_dispatch(fetch_rows, "FETCH_SIZE", is_copy, largest=True)
    w_dom, n_wd = per_dispatch(write_rows, "WRITE_SIZE", is_dom)
    w_cpy, n_wc = per_dispatch(write_rows, "WRITE_SIZE", is_copy, largest=True)
    f_scale = line["copy_bytes"] / (f_cpy * 1024)
    w_scale = line["copy_bytes"] / (w_cpy * 1024)
    # a second, independent calibration of the read counter: the read-only probe
    # kernel reads exactly read_probe_bytes per dispatch and writes 4 bytes per wave
    is_probe = lambda n: "hbm_read_kernel" in n  # noqa: E731
    try:
        f_prb, n_fp = per_dispatch(fetch_rows, "FETCH_SIZE", is_probe)
        f_scale_probe = line["read_probe_bytes"] / (f_prb * 1024)
    except (SystemExit, KeyError):
        f_prb, n_fp, f_scale_probe = None, 0, None
    fetch_b = f_dom * 1024 * f_scale
    write_b = w_dom * 1024 * w_scale
    dom_stats = [r for r in stats if is_dom(r["Name"])]
    avg_ns = float(dom_stats[0]["AverageNs"]) if dom_stats else None
    traffic = {
        "kernel": line["kernel"],
        "algo_bytes_per_launch": line["algo_bytes_per_launch"],
        "traffic_bytes_per_launch": int(round(fetch_b + write_b)),
        "fetch_bytes_per_launch": int(round(fetch_b)),
        "write_bytes_per_launch": int(round(write_b)),
        "traffic_over_algo": round((fetch_b + write_b) / line["algo_bytes_per_launch"], 4),
        "fetch_size_kib_per_dispatch": round(f_dom, 1),
        "write_size_kib_per_dispatch": round(w_dom, 1),
        "copy_fetch_kib": round(f_cpy, 1),
        "copy_write_kib": round(w_cpy, 1),
        "fetch_scale": round(f_scale, 5),
        "write_scale": round(w_scale, 5),
        "fetch_scale_read_probe": round(f_scale_probe, 5) if f_scale_probe else None,
        "read_probe_fetch_kib": round(f_prb, 1) if f_prb else None,
        "fetch_bytes_per_launch_by_probe_scale": int(round(f_dom * 1024 * f_scale_probe)) if f_scale_probe else None,
        "dispatches": {"fetch": n_fd, "write": n_wd, "copy_fetch": n_fc, "copy_write": n_wc, "probe_fetch": n_fp},
        "rocprof_avg_launch_us": round(avg_ns / 1e3, 3) if avg_ns else None,
        "bench_avg_launch_us": line["avg_launch_us"],
        "source": "rocprofv3 --pmc FETCH_SIZE and --pmc WRITE_SIZE over bench.py --roofline-only",
        "command": command,
    }
    os.makedirs(os.path.dirname(TRAFFIC_FILE), exist_ok=True)
    with open(TRAFFIC_FILE, "w") as f:
        json.dump(traffic, f, indent=1)
        f.write("\n")
    md = [f"# Dominant decode kernel: {line['kernel']}", "", "Command (from the repository root):", "",
          "```", command, "```", "", "bench.py --roofline-only line:", "", "```", json.dumps(line), "```", "",
          "rocprofv3 --kernel-trace --stats (kernel_stats.csv):", "",
          "| kernel | calls | avg us | min us | max us |", "|---|---:|---:|---:|---:|"]
    for r in sorted(stats, key=lambda r: -float(r["TotalDurationNs"]))[:8]:
        md.append(f"| {short(r['Name'])} | {r['Calls']} | {float(r['AverageNs']) / 1e3:.3f} | "
                  f"{float(r['MinNs']) / 1e3:.3f} | {float(r['MaxNs']) / 1e3:.3f} |")
    md += ["", "HBM traffic per launch (FETCH_SIZE, WRITE_SIZE in KiB per dispatch, scaled by the 1 GiB copy; "
           "the read-only probe over 1 GiB gives a second, independent scale for FETCH_SIZE):", "",
           "```", json.dumps(traffic, indent=1), "```", ""]
    with open(os.path.join(ROOT, "profiles", "gate_up_decode_m1.md"), "w") as f:
        f.write("\n".join(md))
    print(json.dumps(traffic))


PREFILL_MS = (64, 256, 512, 2048)


def prefill_sweep_names(ms=PREFILL_MS):
    """The forwards of `--prefill-only` in the order it runs them."""
    names = []
    for m in ms:
        names += [f"{n}_m{m}" for n, _, _ in list(LAYER) + list(FULL_ATTENTION)] + [f"{PAIR}_m{m}"]
    return names


def variants_run(torch, Q, host) -> dict:
    """The 8-bit affine variant and a LoRA adapter on the gate_proj shape (N = 15360,
    K = 3840): decode at M = 1 (HBM rate over the variant's own algorithmic bytes:
    8-bit codes are 1 byte per weight plus the bf16 scales and biases) and prefill at
    M = 2048 (TFLOPS), and the LoRA forward (rank 16, delta added to the bf16 output)
    against the plain forward on the same handle."""
    import torch as _t
    from helios_amd.quantize import quantize

    n, k = 15360, HIDDEN
    rng = np.random.Generator(np.random.PCG64(SEED_BASE + 7000))
    w = _t.from_numpy(rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).cuda().bfloat16()
    wq8, s8, b8 = quantize(w, bits=8)
    del w
    out = {}
    x1 = torch.from_numpy(synthetic_activations(1, k, seed=SEED_BASE + 11).view(np.int16)).view(torch.bfloat16).cuda()
    x2 = torch.from_numpy(synthetic_activations(2048, k, seed=SEED_BASE + 12, outliers=True).view(np.int16)) \
        .view(torch.bfloat16).cuda()
    w8bytes = n * k + 4 * n * (k // 64)
    us = kernel_us(torch, lambda: Q.QuantizedLinear(wq8, s8, b8, bits=8), 1, k, n, x1, w8bytes)
    b1 = w8bytes + 2 * k + 2 * n
    out["q8_gate_m1"] = {"us": round(us, 2), "GBps": round(b1 / (us * 1e-6) / 1e9, 1),
                         "algo_bytes": b1, "resident_bytes_per_weight": 1.125}
    lin8 = Q.QuantizedLinear(wq8, s8, b8, bits=8)
    y2 = torch.empty((2048, n), dtype=torch.bfloat16, device="cuda")
    ms = graph_ms_steady(torch, lambda: lin8.forward(x2, out=y2))
    out["q8_gate_m2048"] = {"us": round(ms * 1e3, 1),
                            "TFLOPS": round(algo_flops(2048, n, k) / (ms * 1e-3) / 1e12, 1)}
    lin8.close()
    # LoRA: rank 16, scale 2 (alpha 32), A [16, K], B [N, 16]
    r = 16
    a = (rng.standard_normal((r, k)) * 0.02).astype(np.float32)
    bm = (rng.standard_normal((n, r)) * 0.02).astype(np.float32)
    lora = Q.LoraAdapter(a, bm, 2.0)
    lin = Q.QuantizedLinear(*host["gate_proj"])
    for m, x in ((1, x1), (2048, x2)):
        y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
        t_plain = graph_ms_steady(torch, lambda: lin.forward(x, out=y)) * 1e3
        t_lora = graph_ms_steady(torch, lambda: lin.forward_lora(x, lora, out=y)) * 1e3
        out[f"lora_r16_gate_m{m}"] = {"us_plain": round(t_plain, 2), "us_lora": round(t_lora, 2),
                                      "overhead_us": round(t_lora - t_plain, 2)}
    lin.close()
    lora.close()
    return out


def summarize_gemm(stats_dir: str, pmc_dir: str, line_file: str, command: str) -> None:
    """Turns rocprofv3 output over `bench.py --gemm-only` into the headline GEMM's
    committed summary (profiles/gate_prefill_m2048.md): the kernel-trace statistics
    (the GEMM kernel's average duration and the TFLOPS it implies), and the counters of
    one --pmc pass per dispatch of the GEMM kernel (median over dispatches), with the
    matrix cores' busy share: SQ_VALU_MFMA_BUSY_CYCLES per SIMD over the kernel's
    cycles (GRBM_GUI_ACTIVE counts once per XCD)."""
    import statistics

    with open(line_file) as f:
        line = json.loads([l for l in f if l.startswith("{")][-1])
    stats = _csv_rows(stats_dir, "kernel_stats.csv")
    rows = _csv_rows(pmc_dir, "counter_collection.csv")

    def short(name: str) -> str:
        return name.replace("void ", "").replace("(anonymous namespace)::", "").split("(")[0][:90]

    is_gemm = lambda n: "gemm_kernel" in n  # noqa: E731
    per = {}
    for r in rows:
        if is_gemm(r["Kernel_Name"]):
            per.setdefault(r["Counter_Name"], {}).setdefault(r["Dispatch_Id"], 0.0)
            per[r["Counter_Name"]][r["Dispatch_Id"]] += float(r["Counter_Value"])
    med = {c: statistics.median(v.values()) for c, v in per.items()}
    g = [r for r in stats if is_gemm(r["Name"])]
    avg_us = float(g[0]["AverageNs"]) / 1e3 if g else None
    m, n, k = 2048, 15360, HIDDEN
    md = [f"# Prefill GEMM: {short(g[0]['Name']) if g else 'gemm_kernel'} gate_proj M=2048 N=15360 K=3840 (bf16 out)", "",
          "Command (from the repository root):", "", "```", command, "```", "",
          f"Unprofiled line (`bench.py --gemm-only`): {json.dumps(line)}", "",
          "rocprofv3 --kernel-trace --stats (kernel_stats.csv):", "",
          "| kernel | calls | avg us | min us | max us |", "|---|---:|---:|---:|---:|"]
    for r in sorted((r for r in stats if "q4::" in r["Name"]), key=lambda r: -float(r["TotalDurationNs"]))[:6]:
        md.append(f"| {short(r['Name'])} | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                  f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} |")
    if avg_us:
        tf = algo_flops(m, n, k) / (avg_us * 1e-6) / 1e12
        md += ["", f"GEMM kernel alone: {tf:.0f} TFLOPS at the rocprof average ({avg_us:.1f} us), "
                   f"{tf / BF16_PEAK_TFLOPS:.1%} of {BF16_PEAK_TFLOPS / 1e3:.1f} PF dense bf16."]
    md += ["", "Counters per dispatch of the GEMM kernel (median over dispatches; SQ counters summed over the chip):",
           "", "| counter | value |", "|---|---:|"]
    for c in sorted(med):
        md.append(f"| {c} | {med[c]:.0f} |")
    if {"SQ_INSTS_MFMA", "SQ_INSTS_VALU"} <= med.keys():
        mf, va = med["SQ_INSTS_MFMA"], med["SQ_INSTS_VALU"]
        md += ["", f"- MFMA instructions {mf / 1e6:.2f} M; other VALU instructions (SQ_INSTS_VALU counts the MFMAs "
                   f"too) {(va - mf) / 1e6:.2f} M, {(va - mf) / mf:.2f} per MFMA."]
    if {"SQ_VALU_MFMA_BUSY_CYCLES", "GRBM_GUI_ACTIVE"} <= med.keys():
        # the profiled GPU's SIMD count, from the agent description rocprofv3 writes
        agents = [r for r in _csv_rows(pmc_dir, "agent_info.csv") if int(r.get("Simd_Count") or 0) > 0]
        simds = int(agents[0]["Simd_Count"]) if agents else 1024
        busy = med["SQ_VALU_MFMA_BUSY_CYCLES"] / simds
        cyc = med["GRBM_GUI_ACTIVE"] / 8
        md.append(f"- Matrix-core busy cycles per SIMD: {busy / 1e3:.0f} K of {cyc / 1e3:.0f} K kernel cycles "
                  f"(GRBM_GUI_ACTIVE / 8 XCDs): {busy / cyc:.0%} busy.")
    with open(os.path.join(ROOT, "profiles", "gate_prefill_m2048.md"), "w") as f:
        f.write("\n".join(md) + "\n")
    print("\n".join(md))


def summarize_trace(db_path: str, out_md: str, command: str) -> None:
    """Per-shape kernel durations of `bench.py --prefill-only` from a rocprofv3
    --kernel-trace database (rocpd SQLite).  Each shape's handles are created (repack
    launches) before its forwards, which split the trace into the sweep's shapes in
    order; a GEMM-path forward launches the GEMM (after xaug_kernel, the group-sum
    pre-pass, or xprep_kernel, the fp16 form's, for the 256-row tile) and, when K is
    split, the split-K reduction; a
    decode-path forward one decode kernel.  Reported: the median
    duration of each kernel and of the whole forward (first launch start to last
    launch end) over the shape's forwards."""
    import re
    import sqlite3

    rows = list(sqlite3.connect(db_path).execute(
        "select name, grid_x, grid_y, workgroup_x, duration, start from kernels order by start"))

    def short(n):
        n = n.replace("(anonymous namespace)::", "").replace("void ", "").replace("q4::", "")
        return re.sub(r"\(.*", "", n)

    shapes = _trace_forwards(rows, short)  # per shape: list of forwards, each a list of launches
    names = prefill_sweep_names()
    md = ["# Prefill GEMM sweep: kernel durations per forward", "", "Command (from the repository root):", "",
          "```", command, "```", "",
          "Per shape: the launches of one forward (kernel: workgroups x K splits, or x 16-row slabs for the decode "
          "kernels) and their median durations over the shape's forwards (back-to-back forwards over rotated weight "
          "copies in a replayed graph); the forward's span runs from its first launch's start to its last launch's "
          "end.", "",
          "| shape | launches | forwards | median us per kernel | forward span us |", "|---|---|---:|---|---:|"]
    for name, fwds in zip(names, shapes):
        if not fwds:
            continue
        sig = max(set(tuple((short(p[0]), p[1] // max(p[3], 1), p[2]) for p in f) for f in fwds),
                  key=lambda k: sum(1 for f in fwds if len(f) == len(k)))
        same = [f for f in fwds if len(f) == len(sig)]
        cols = list(zip(*[[p[4] for p in f] + [f[-1][5] + f[-1][4] - f[0][5]] for f in same]))
        med = [sorted(c)[len(c) // 2] / 1e3 for c in cols]
        desc = ", ".join(f"{k} {g}x{y}" for k, g, y in sig)
        md.append(f"| {name} | {desc} | {len(same)} | {' / '.join(f'{x:.2f}' for x in med[:-1])} | "
                  f"{med[-1]:.2f} |")
    if len(shapes) != len(names):
        md += ["", f"(trace holds {len(shapes)} shapes, the sweep {len(names)}: labels may not line up)"]
    with open(out_md, "w") as f:
        f.write("\n".join(md) + "\n")
    print("\n".join(md))


# launches of `--decode-only`, in the order it runs them: (launch, rows)
DECODE_PROFILE = [("k_proj", 1), ("q_proj", 1), ("o_proj", 1), ("qkv_proj", 1), ("gate_proj", 1), ("down_proj", 1),
                  ("gate_up_geglu", 1), ("qkv_proj", 8), ("o_proj", 8), ("gate_proj", 8), ("down_proj", 8),
                  ("gate_up_geglu", 8)]


def _trace_forwards(rows, short):
    """Kernel launches of a trace in start order, grouped per shape (each shape's
    handles are created, with repack launches, before its forwards) and per forward (a
    GEMM-path forward starts with the GEMM, or its pre-pass for the 256-row tile; a
    decode-path forward is one decode kernel)."""
    shapes = []
    for r in rows:
        if "q4::" not in r[0]:
            continue
        s = short(r[0])
        if s.startswith("repack"):
            if not shapes or shapes[-1]:
                shapes.append([])
        elif shapes and (s.startswith(("xaug", "xprep")) or s.startswith("decode") or
                         (s.startswith("gemm_kernel") and
                          not (shapes[-1] and short(shapes[-1][-1][-1][0]).startswith(("xaug", "xprep"))))):
            shapes[-1].append([r])
        elif shapes and shapes[-1]:
            shapes[-1][-1].append(r)
    return shapes


def summarize_decode(db_path: str, fetch_dir: str, write_dir: str, line_file: str, out_md: str, command: str) -> None:
    """Per-launch summary of `bench.py --decode-only` from a rocprofv3 kernel trace
    (rocpd SQLite) and FETCH_SIZE / WRITE_SIZE passes (csv): the median duration of
    each decode launch and its HBM bytes per dispatch, each counter scaled by what it
    reads for the run's 1 GiB copy, against the launch's algorithmic bytes."""
    import re
    import sqlite3

    def short(n):
        n = n.replace("(anonymous namespace)::", "").replace("void ", "").replace("q4::", "")
        return re.sub(r"\(.*", "", n)

    with open(line_file) as f:
        line = json.loads([l for l in f if l.startswith("{")][-1])
    rows = list(sqlite3.connect(db_path).execute(
        "select name, grid_x, grid_y, workgroup_x, duration, start from kernels order by start"))
    shapes = _trace_forwards(rows, short)

    def counter_shapes(d, counter):
        """per shape (split at repack dispatches, in dispatch order): the mean counter
        value of its decode dispatches, and the copy kernel's value"""
        recs = [r for r in _csv_rows(d, "counter_collection.csv") if r["Counter_Name"] == counter]
        recs.sort(key=lambda r: int(r.get("Dispatch_Id") or r.get("Correlation_Id") or 0))
        per, cpy = [], []
        for r in recs:
            n = r["Kernel_Name"]
            if "rocclr_copybuffer" in n.lower():
                cpy.append(float(r["Counter_Value"]))
            elif "q4::" not in n:
                continue
            elif short(n).startswith("repack"):
                if not per or per[-1]:
                    per.append([])
            elif short(n).startswith("decode") and per:
                per[-1].append(float(r["Counter_Value"]))
        # the 1 GiB copies, not the runtime's small blits (handle creation's)
        cpy = [c for c in cpy if c >= 0.5 * max(cpy)] if cpy else cpy
        return [sum(v) / len(v) if v else None for v in per], (sum(cpy) / len(cpy) if cpy else None)

    fetch, f_cpy = counter_shapes(fetch_dir, "FETCH_SIZE")
    write, w_cpy = counter_shapes(write_dir, "WRITE_SIZE")
    f_scale = line["copy_bytes"] / (f_cpy * 1024) if f_cpy else None
    w_scale = line["copy_bytes"] / (w_cpy * 1024) if w_cpy else None
    md = ["# Decode launches at M = 1 and 8: durations and HBM traffic", "", "Command (from the repository root):", "",
          "```", command, "```", "", "bench.py --decode-only line (HIP-event timing, no profiler):", "", "```",
          json.dumps(line), "```", "",
          "Per launch: the kernel (workgroups x 16-row slabs), its median duration over the launch's dispatches in "
          "the kernel trace (back-to-back launches over rotated weight copies in a replayed graph), the bench's own "
          "figure, and HBM bytes per dispatch from FETCH_SIZE + WRITE_SIZE (KiB per dispatch, scaled by what each "
          f"counter reads for the 1 GiB copy: fetch x{f_scale:.4f}, write x{w_scale:.4f}) against the algorithmic "
          "bytes.", "",
          "| launch | kernel | dispatches | median us (trace) | us (bench) | algorithmic MB | HBM MB | ratio | GB/s |",
          "|---|---|---:|---:|---:|---:|---:|---:|---:|"]
    for i, (name, m) in enumerate(DECODE_PROFILE):
        key = f"{name}_m{m}"
        if i >= len(shapes) or not shapes[i]:
            continue
        fwds = shapes[i]
        k0 = short(fwds[0][0][0])
        durs = sorted(p[4] for f in fwds for p in f if short(p[0]) == k0)
        med = durs[len(durs) // 2] / 1e3
        rec = line["launches"][key]
        hbm = None
        if i < len(fetch) and i < len(write) and fetch[i] is not None and write[i] is not None:
            hbm = fetch[i] * 1024 * f_scale + write[i] * 1024 * w_scale
        md.append(f"| {key} | {k0} {fwds[0][0][1] // max(fwds[0][0][3], 1)}x{fwds[0][0][2]} | {len(durs)} | "
                  f"{med:.2f} | {rec['us']:.2f} | {rec['algo_bytes'] / 1e6:.2f} | "
                  f"{(hbm / 1e6) if hbm else float('nan'):.2f} | "
                  f"{(hbm / rec['algo_bytes']) if hbm else float('nan'):.3f} | {rec['algo_bytes'] / (med * 1e3):.0f} |")
    if len(shapes) != len(DECODE_PROFILE):
        md += ["", f"(trace holds {len(shapes)} launches, the run {len(DECODE_PROFILE)}: labels may not line up)"]
    with open(out_md, "w") as f:
        f.write("\n".join(md) + "\n")
    print("\n".join(md))


def build_decoder(torch, Q, layers: int = 48, seed: int = SEED_BASE + 5):
    """Weights of the 48-layer Gemma-style 12B decoder's quantized projections, made on
    the device: random 4-bit codes with bf16 scales in [0.002, 0.005) and biases
    -7.5 * scale + U(-0.002, 0.002), so that the weights are centred (a N(0, 0.02)
    weight's size; 6.6 GB, far beyond the 256 MiB Infinity Cache).  Each layer holds q|k|v as one handle (8192 x 3840, q, k, v
    concatenated along N), o, the gate|up GeGLU pair and down, plus per-layer RMSNorm
    weights; one greedy lm_head (262144 x 3840) follows."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)

    def triple(n, k):
        w = torch.randint(-2**31, 2**31 - 1, (n, k // 8), dtype=torch.int32, device="cuda", generator=g)
        s = torch.rand((n, k // 64), device="cuda", generator=g) * 0.003 + 0.002
        b = -7.5 * s + (torch.rand((n, k // 64), device="cuda", generator=g) - 0.5) * 0.004
        return w, s.bfloat16(), b.bfloat16()

    net = []
    for _ in range(layers):
        net.append({"qkv": Q.QuantizedLinear(*triple(8192, HIDDEN)), "o": Q.QuantizedLinear(*triple(HIDDEN, 4096)),
                    "mlp": Q.QuantizedGeGLU(triple(15360, HIDDEN), triple(15360, HIDDEN)),
                    "down": Q.QuantizedLinear(*triple(HIDDEN, 15360)),
                    "norm": (torch.rand((2, HIDDEN), device="cuda", generator=g) * 0.2 - 0.1).bfloat16()})
    lm = Q.QuantizedLinear(*triple(262144, HIDDEN))
    torch.cuda.synchronize()
    return net, lm


def free_decoder(net, lm) -> None:
    for L in net:
        for name in ("qkv", "o", "mlp", "down"):
            L[name].close()
    lm.close()


def rms_norm(torch, x, w, eps: float = 1e-6):
    """Gemma RMSNorm in fp32, rounded to bf16: x / sqrt(mean(x^2) + eps) * (1 + w)."""
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * (1.0 + w.float())).bfloat16()


def decoder_forward_m1(torch, net, lm, x0, states=None):
    """One decode token through the chained decoder, every projection on the library:
    per layer RMSNorm -> q|k|v -> attention over the token's own position (one key, so
    each query head's output is the value of its KV head; RoPE at position 0 is the
    identity) -> o -> residual add -> RMSNorm -> gate|up GeGLU -> down -> residual add;
    then the greedy lm_head (softcap 30) on the final RMSNorm.  Attention and norms are
    plain torch bf16/fp32 ops.  Returns the token tensor [1] (int32); with `states` (a
    list) the residual stream after every layer is appended to it."""
    x = x0
    for L in net:
        h = rms_norm(torch, x, L["norm"][0])
        qkv = L["qkv"].forward(h)
        v = qkv[:, 6144:8192].reshape(1, 8, 256)
        attn = v.repeat_interleave(2, dim=1).reshape(1, 4096)  # 16 query heads over 8 KV heads
        x = (x.float() + L["o"].forward(attn).float()).bfloat16()
        hh = L["mlp"].forward(rms_norm(torch, x, L["norm"][1]))
        x = (x.float() + L["down"].forward(hh).float()).bfloat16()
        if states is not None:
            states.append(x)
    token = lm.forward_greedy(rms_norm(torch, x, net[-1]["norm"][0]), softcap=30.0)
    return token if isinstance(token, torch.Tensor) else token[0]


def decoder_check(torch, net, lm, replays: int = 3, seed: int = SEED_BASE + 6) -> dict:
    """The chained decode forward run eagerly and as a HIP graph replayed `replays`
    times (with eager work and synchronizations between replays): whether every
    residual state and the token are finite / equal bit for bit across them."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    x0 = torch.randn((1, HIDDEN), device="cuda", generator=g).bfloat16()
    eager_states = []
    eager_tok = decoder_forward_m1(torch, net, lm, x0, eager_states).clone()
    torch.cuda.synchronize()
    finite = all(bool(torch.isfinite(s).all()) for s in eager_states)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        decoder_forward_m1(torch, net, lm, x0)  # warms the capture stream's scratch
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    cap_states = []
    with torch.cuda.graph(graph, stream=stream):
        cap_tok = decoder_forward_m1(torch, net, lm, x0, cap_states)
    equal, tokens = True, []
    for _ in range(replays):
        graph.replay()
        torch.cuda.synchronize()
        equal &= all(torch.equal(a, b) for a, b in zip(eager_states, cap_states))
        tokens.append(int(cap_tok.item()))
        # eager work between replays (the program's own use of the stream)
        decoder_forward_m1(torch, net, lm, x0)
        torch.cuda.synchronize()
    del graph
    return {"finite": finite, "graph_equals_eager": bool(equal), "token": int(eager_tok.item()),
            "replay_tokens": tokens, "token_stable": all(t == int(eager_tok.item()) for t in tokens),
            "final_rms": round(float(eager_states[-1].float().pow(2).mean().sqrt()), 4)}


def model_run(torch, Q, decode_steps: int = 128, prefill_tokens: int = 16384, chunk: int = 2048,
              layers: int = 48) -> dict:
    """The 48-layer Gemma-style 12B decoder's quantized matmuls, timed alone (the other
    ops of the model are not in the timed region): 16K-token chunked prefill (M = 2048
    chunks) then 128 decode steps at M = 1, each layer as qkv, o, the gate|up GeGLU
    pair and down, then the greedy lm_head on the last position.  Inputs of the timed
    passes are fixed N(0, 1) activations.  Timed with events around the launches only.
    Then `decoder_check`: the chained forward (norms, attention and residuals between
    the projections) checked eager against graph replays."""
    net, lm = build_decoder(torch, Q, layers)
    g = torch.Generator(device="cuda")
    g.manual_seed(SEED_BASE + 7)
    # each projection's input and output, contiguous [chunk, width]; a pass over M rows
    # uses the first M rows of each
    xin = {k: torch.randn((chunk, k), device="cuda", generator=g).bfloat16() for k in (HIDDEN, 4096, 15360)}
    yout = {n: torch.empty((chunk, n), device="cuda", dtype=torch.bfloat16) for n in (8192, HIDDEN, 15360)}

    def step(m):
        for L in net:
            L["qkv"].forward(xin[HIDDEN][:m], out=yout[8192][:m])
            L["o"].forward(xin[4096][:m], out=yout[HIDDEN][:m])
            L["mlp"].forward(xin[HIDDEN][:m], out=yout[15360][:m])
            L["down"].forward(xin[15360][:m], out=yout[HIDDEN][:m])

    step(chunk)
    step(1)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    # prefill: 8 chunks of 2048 through every layer, then the head on the last row
    e0.record()
    for _ in range(prefill_tokens // chunk):
        step(chunk)
    lm.forward_greedy(xin[HIDDEN][:1], softcap=30.0)
    e1.record()
    torch.cuda.synchronize()
    prefill_ms = e0.elapsed_time(e1)
    # decode: a graph of one token (every layer + the greedy head), replayed
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        step(1)
        lm.forward_greedy(xin[HIDDEN][:1], softcap=30.0)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        step(1)
        lm.forward_greedy(xin[HIDDEN][:1], softcap=30.0)
    graph.replay()
    torch.cuda.synchronize()
    e0.record()
    for _ in range(decode_steps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    decode_ms = e0.elapsed_time(e1) / decode_steps
    del graph
    check = decoder_check(torch, net, lm)
    layer_w = sum(n * k // 2 + 4 * n * (k // 64) for _, n, k in LAYER)
    lm_w = 262144 * HIDDEN // 2 + 4 * 262144 * (HIDDEN // 64)
    step_bytes = layers * sum(algo_bytes(1, n, k) for _, n, k in LAYER) + algo_bytes(1, 262144, HIDDEN)
    prefill_flops = layers * sum(algo_flops(prefill_tokens, n, k) for _, n, k in LAYER) + algo_flops(1, 262144, HIDDEN)
    free_decoder(net, lm)
    return {
        "workload": f"{layers}-layer Gemma-style 12B decoder, quantized matmuls only: {prefill_tokens}-token prefill "
                    f"in chunks of {chunk}, then {decode_steps} decode steps (each layer qkv, o, gate|up GeGLU pair, "
                    "down; greedy lm_head with softcap)",
        "weights_bytes": layers * layer_w + lm_w,
        "decode_ms_per_token": round(decode_ms, 4),
        "decode_tokens_per_s": round(1e3 / decode_ms, 1),
        "decode_GBps": round(step_bytes / (decode_ms * 1e-3) / 1e9, 1),
        "prefill_ms": round(prefill_ms, 2),
        "prefill_TFLOPS": round(prefill_flops / (prefill_ms * 1e-3) / 1e12, 1),
        "prefill_tokens_per_s": round(prefill_tokens / (prefill_ms * 1e-3), 1),
        "chained_forward_check": check,
    }


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(host, lm_triple=None, scale: float = 1.0) -> dict:
    """The oracle's fp32 qmm loop (dequantize a row's groups, then dot; OpenMP over
    rows) on this host's cores, on bounded samples of four workloads, each timed
    on all threads and on 1 thread: the single GEMV (gate_proj shape, M = 1), the
    decoder layer's seven projections at M = 1 (the headline's workload and `value`),
    the lm_head at M = 1, and the seven projections at the prefill chunk M = 512.
    Samples that would take long on one thread use the first rows of each weight
    (the rate per byte or per flop does not depend on which rows).  Threads: the
    OMP_NUM_THREADS of the environment (the host's CPU share), else os.cpu_count()."""
    from oracle import c_oracle as C

    env_threads = os.environ.get("OMP_NUM_THREADS", "")
    threads = int(env_threads) if env_threads.isdigit() and int(env_threads) > 0 else (os.cpu_count() or 1)
    xs = {(m, k): synthetic_activations(m, k, seed=SEED_BASE + 7 * m + k) for m in (1, 512)
          for k in {k for _, _, k in LAYER}}

    def rows(tri, r):
        return tuple(np.ascontiguousarray(a[:r]) for a in tri) if r < tri[0].shape[0] else tri

    def timed(fn, target):
        fn()  # warm (page in, thread pool up)
        t0 = time.perf_counter()
        reps = 0
        while True:
            fn()
            reps += 1
            el = time.perf_counter() - t0
            if el >= target:
                return reps, el

    def run(parts, m, nthreads, target, row_frac=1.0):
        """parts: [(triple, k)]; returns (reps, seconds, bytes per rep, flops per rep)."""
        work = [(rows(tri, max(16, int(tri[0].shape[0] * row_frac))), k) for tri, k in parts]
        outs = [np.empty((m, t[0].shape[0]), np.float32) for t, _ in work]

        def fn():
            for (t, k), o in zip(work, outs):
                C.qmm_f32(xs[(m, k)], *t, threads=nthreads, out=o)

        reps, el = timed(fn, target * scale)
        nb = sum(algo_bytes(m, t[0].shape[0], k) for t, k in work)
        fl = sum(algo_flops(m, t[0].shape[0], k) for t, k in work)
        return reps, el, nb, fl

    layer = [(host[name], k) for name, _, k in LAYER]
    cases = [("gemv_gate_m1", [(host["gate_proj"], HIDDEN)], 1, 2.0, 1.0, 1.0, "GB/s"),
             ("layer_m1", layer, 1, 4.0, 2.0, 1.0, "GB/s"),
             ("layer_prefill_m512", layer, 512, 4.0, 2.0, 1 / 32, "GFLOP/s")]
    if lm_triple is not None:
        cases.insert(2, ("lm_head_m1", [(lm_triple, HIDDEN)], 1, 3.0, 1.5, 1 / 16, "GB/s"))
    out = {}
    for name, parts, m, t_all, t_one, frac_one, unit in cases:
        res = {}
        for label, nthr, target, frac in (("all_threads", threads, t_all, 1.0), ("one_thread", 1, t_one, frac_one)):
            reps, el, nb, fl = run(parts, m, nthr, target, frac)
            rate = nb * reps / el / 1e9 if unit == "GB/s" else fl * reps / el / 1e9
            res[label] = {"value": round(rate, 3), "reps": reps, "seconds": round(el, 2),
                          "rows_fraction": frac}
        res["unit"] = unit
        out[name] = res
    head = out["layer_m1"]["all_threads"]
    return {
        "value": head["value"],
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{head['reps']} decoder-layer steps (7 projections, M=1) in {head['seconds']} s on {threads} "
                  "threads; C restatement of the fp32 dequantize-and-dot loop (oracle/q4_oracle.c), OpenMP over "
                  "rows; 1-thread and other workloads under 'workloads'",
        "cpu_model": cpu_model(),
        "threads_source": "OMP_NUM_THREADS" if env_threads.isdigit() else "os.cpu_count()",
        "host_cpus": os.cpu_count(),
        "workloads": out,
    }


# the real 12B's full-attention layers (native_model.cc:795-798, :820-827): q 3840 -> 8192,
# k 3840 -> 512 (no v_proj: k doubles as v), o 8192 -> 3840
FULL_ATTENTION = [("full_q_proj", 8192, 3840), ("full_k_proj", 512, 3840), ("full_o_proj", 3840, 8192)]


def prefill_sweep(torch, Q, host, ms, shapes, pair: bool, full_attention: bool) -> dict:
    """Prefill GEMM lines: each projection of `shapes` (and, optionally, the gate|up
    GeGLU pair and the full-attention shapes) at every M of ms; activations N(0, 1)
    with 1% outliers x20.  Timed as the decode lines are (kernel_us): back-to-back
    forwards over rotated weight copies in one graph, replayed after a wall-time
    settle, so a line is one forward's launches and the gaps between them, not the
    launch of a one-forward graph (~7-10 us per replay)."""
    out = {}
    extra = {}
    if full_attention:
        for i, (name, n, k) in enumerate(FULL_ATTENTION):
            extra[name] = synthetic_weights(n, k, SEED_BASE + 6000 + i)
    all_shapes = list(shapes) + (list(FULL_ATTENTION) if full_attention else [])
    for m in ms:
        xk = {k: torch.from_numpy(synthetic_activations(m, k, seed=SEED_BASE + 2 + k, outliers=True).view(np.int16))
              .view(torch.bfloat16).cuda() for k in {k for _, _, k in all_shapes}}
        for name, n, k in all_shapes:
            tri = host[name] if name in host else extra[name]
            us = kernel_us(torch, lambda: Q.QuantizedLinear(*tri), m, k, n, xk[k], weight_bytes(n, k))
            tflops = algo_flops(m, n, k) / (us * 1e-6) / 1e12
            out[f"{name}_m{m}"] = {"us": round(us, 1), "TFLOPS": round(tflops, 1),
                                   "frac_bf16_peak": round(tflops / BF16_PEAK_TFLOPS, 4)}
        if pair:  # the GeGLU pair: gate and up in one GEMM, h = geglu(gate, up)
            f, k = 15360, HIDDEN
            us = kernel_us(torch, lambda: Q.QuantizedGeGLU(host["gate_proj"], host["up_proj"]), m, k, f, xk[k],
                           2 * weight_bytes(f, k))
            tflops = algo_flops(m, 2 * f, k) / (us * 1e-6) / 1e12
            out[f"{PAIR}_m{m}"] = {"us": round(us, 1), "TFLOPS": round(tflops, 1),
                                   "frac_bf16_peak": round(tflops / BF16_PEAK_TFLOPS, 4)}
        del xk
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-gemm", action="store_true")
    ap.add_argument("--quick", action="store_true", help="headline only (skip the per-shape sweeps)")
    ap.add_argument("--gemm-only", action="store_true",
                    help="the headline prefill GEMM (gate_proj, M=2048) only, one JSON line (for rocprofv3)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="the prefill GEMM sweep only (the seven projections at M = 64, 256, 512, 2048 and the "
                         "full-attention shapes), one JSON line (for rocprofv3 kernel traces)")
    ap.add_argument("--settle-ms", type=float, default=100.0,
                    help="untimed wall time of headline replays after the warm-up replays (the clock ramps)")
    ap.add_argument("--roofline-only", action="store_true",
                    help="time only the dominant kernel and a 1 GiB copy (the program rocprofv3 passes run)")
    ap.add_argument("--summarize-profiles", nargs=5, metavar=("STATS_DIR", "FETCH_DIR", "WRITE_DIR", "LINE", "CMD"),
                    help="write the profiles/ summaries from rocprofv3 output over --roofline-only (no GPU)")
    ap.add_argument("--summarize-gemm", nargs=4, metavar=("STATS_DIR", "PMC_DIR", "LINE", "CMD"),
                    help="write profiles/gate_prefill_m2048.md from rocprofv3 output over --gemm-only")
    ap.add_argument("--summarize-trace", nargs=3, metavar=("RESULTS_DB", "OUT_MD", "CMD"),
                    help="write a per-shape summary of a rocprofv3 kernel trace of --prefill-only (no GPU)")
    ap.add_argument("--decode-only", action="store_true",
                    help="the decode launches of DECODE_PROFILE (M = 1 and 8) and a 1 GiB copy, one JSON line "
                         "(for rocprofv3 kernel traces and counter passes)")
    ap.add_argument("--summarize-decode", nargs=6,
                    metavar=("RESULTS_DB", "FETCH_DIR", "WRITE_DIR", "LINE", "OUT_MD", "CMD"),
                    help="write the per-launch summary of rocprofv3 output over --decode-only (no GPU)")
    args = ap.parse_args()
    if args.summarize_profiles:
        summarize_profiles(*args.summarize_profiles)
        return 0
    if args.summarize_trace:
        summarize_trace(*args.summarize_trace)
        return 0
    if args.summarize_gemm:
        summarize_gemm(*args.summarize_gemm)
        return 0
    if args.summarize_decode:
        summarize_decode(*args.summarize_decode)
        return 0
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        return 2

    import torch

    import helios_amd
    from helios_amd import qmm as Q

    helios_amd.load_library()
    torch.cuda.set_device(0)
    log("quantizing one decoder layer")
    host = quantized_layer()
    dims = {name: (n, k) for name, n, k in LAYER}
    launches = dict(STEP + STEP_UNFUSED)
    fused = {name: fused_triple(host, parts) for name, parts in launches.items() if name != PAIR}
    # N of each launch's output and its K
    step_nk = {name: (sum(dims[p][0] for p in parts) if name != PAIR else dims[parts[0]][0], dims[parts[0]][1])
               for name, parts in launches.items()}
    wbytes_of = {name: sum(dims[p][0] * dims[p][1] // 2 + 4 * dims[p][0] * (dims[p][1] // 64) for p in parts)
                 for name, parts in launches.items()}

    def maker(name):
        if name == PAIR:
            return lambda: Q.QuantizedGeGLU(host["gate_proj"], host["up_proj"])
        return lambda: Q.QuantizedLinear(*fused[name])

    xs = {k: torch.from_numpy(synthetic_activations(16, k, seed=SEED_BASE + k).view(np.int16)).view(torch.bfloat16).cuda()
          for k in {k for _, _, k in LAYER}}
    f_gu, k_gu = step_nk[PAIR]
    gu_bytes = pair_algo_bytes(1, f_gu, k_gu)
    gu_kernel = f"{DOM_INSTANCE} gate|up GeGLU pair F={f_gu} K={k_gu} M=1"

    def pair_us(m):
        return kernel_us(torch, maker(PAIR), m, k_gu, f_gu, xs[k_gu], wbytes_of[PAIR])

    if args.gemm_only:
        n_g, k_g = step_nk_gate = (15360, HIDDEN)
        xg = torch.from_numpy(synthetic_activations(2048, k_g, seed=SEED_BASE + 2 + k_g, outliers=True).view(np.int16)) \
            .view(torch.bfloat16).cuda()
        yg = torch.empty((2048, n_g), dtype=torch.bfloat16, device="cuda")
        lin = Q.QuantizedLinear(*host["gate_proj"])
        ms = graph_ms_steady(torch, lambda: lin.forward(xg, out=yg))
        lin.close()
        print(json.dumps({"shape": "gate_proj M=2048 N=15360 K=3840", "us": round(ms * 1e3, 1),
                          "TFLOPS": round(algo_flops(2048, n_g, k_g) / (ms * 1e-3) / 1e12, 1)}), flush=True)
        return 0

    if args.prefill_only:
        print(json.dumps(prefill_sweep(torch, Q, host, PREFILL_MS, LAYER, pair=True, full_attention=True)),
              flush=True)
        return 0

    if args.decode_only:
        res = {}
        for name, m in DECODE_PROFILE:
            if name in step_nk:
                n, k = step_nk[name]
                make, wb = maker(name), wbytes_of[name]
            else:  # a projection the step fuses with others (gate_proj)
                n, k = dims[name]
                make, wb = (lambda nm=name: Q.QuantizedLinear(*host[nm])), weight_bytes(n, k)
            us = kernel_us(torch, make, m, k, n, xs[k], wb)
            ab = pair_algo_bytes(m, n, k) if name == PAIR else algo_bytes(m, n, k)
            res[f"{name}_m{m}"] = {"us": round(us, 3), "algo_bytes": ab, "GBps": round(ab / (us * 1e-6) / 1e9, 1)}
        cgbs = copy_gbs(torch)
        print(json.dumps({"launches": res, "copy_bytes": COPY_BYTES, "copy_GBps": round(cgbs, 1)}), flush=True)
        return 0

    if args.roofline_only:
        us_gu = pair_us(1)
        cgbs = copy_gbs(torch)
        rd = read_gbs(torch, reps=10)
        print(json.dumps({"kernel": gu_kernel, "algo_bytes_per_launch": gu_bytes, "avg_launch_us": round(us_gu, 3),
                          "achieved_GBps": round(gu_bytes / (us_gu * 1e-6) / 1e9, 1),
                          "copy_bytes": COPY_BYTES, "copy_GBps": round(cgbs, 1),
                          "read_probe_bytes": rd["bytes"], "read_probe_GBps": rd["GBps"]}), flush=True)
        return 0

    layer_w_bytes = sum(wbytes_of[name] for name, _ in STEP)
    copies = max(2, -(-ROTATE_BYTES // layer_w_bytes))
    log(f"uploading {copies} copies of the layer ({copies * layer_w_bytes / 2**20:.0f} MiB)")
    layers = [{name: maker(name)() for name, _ in STEP} for _ in range(copies)]
    ys = {name: torch.empty((16, n), dtype=torch.bfloat16, device="cuda") for name, (n, _) in step_nk.items()}

    def step_fn(m, step=STEP, sets=None):
        sets = layers if sets is None else sets

        def fn():
            for c in range(copies):
                for name, _ in step:
                    n, k = step_nk[name]
                    sets[c][name].forward(xs[k][:m], out=ys[name][:m])
        return fn

    # --- headline: one decoder layer's projections at M=1 (4 launches), graph-replayed ---
    log(f"timing decode step M=1 ({args.warmup} warmup replays, {args.settle_ms:.0f} ms settle, "
        f"{args.steps} timed replays)")
    settle_info = {}
    ms_step = graph_ms(torch, step_fn(1), args.steps, args.warmup, settle_ms=args.settle_ms, info=settle_info) / copies
    step_bytes = sum(algo_bytes(1, n, k) for _, n, k in LAYER)
    value = step_bytes / (ms_step * 1e-3) / 1e9
    step_by_m = {}
    for m in ((4, 8, 16) if not args.quick else ()):
        ms_m = graph_ms(torch, step_fn(m), max(10, args.steps // 4), 2, settle_ms=50.0) / copies
        step_by_m[f"m{m}"] = {"ms_per_step": round(ms_m, 5),
                              "GBps": round(sum(algo_bytes(m, n, k) for _, n, k in LAYER) / (ms_m * 1e-3) / 1e9, 1)}
    for lin_set in layers:
        for lin in lin_set.values():
            lin.close()
    del layers
    # the same step under the reference's call structure: q, k and v as three launches
    unfused = None
    if not args.quick:
        sets = [{name: maker(name)() for name, _ in STEP_UNFUSED} for _ in range(copies)]
        ms_u = graph_ms(torch, step_fn(1, STEP_UNFUSED, sets), max(10, args.steps // 4), 2, settle_ms=50.0) / copies
        unfused = {"launches": [name for name, _ in STEP_UNFUSED], "ms_per_step": round(ms_u, 5),
                   "GBps": round(step_bytes / (ms_u * 1e-3) / 1e9, 1)}
        for lin_set in sets:
            for lin in lin_set.values():
                lin.close()
        del sets

    # --- dominant kernel: the gate|up GeGLU pair at M=1 ---
    us_gu = pair_us(1)
    gu_gbs = gu_bytes / (us_gu * 1e-6) / 1e9
    traffic, traffic_rec = recorded_traffic(gu_kernel, gu_bytes)
    roofline = {
        "bound": "hbm",
        "achieved": round(gu_gbs, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(gu_gbs / HBM_PEAK_GBS, 4),
        "traffic": traffic,
        "kernel": gu_kernel,
        "algo_bytes_per_launch": gu_bytes,
        "avg_launch_us": round(us_gu, 3),
    }
    if traffic_rec is not None:
        roofline["traffic_source"] = traffic_rec.get("source")

    # --- the single GEMV of gate_proj's shape (x [1, 3840], W [15360, 3840]) ---
    n1, k1 = dims["gate_proj"]
    us1 = kernel_us(torch, lambda: Q.QuantizedLinear(*host["gate_proj"]), 1, k1, n1, xs[k1],
                    n1 * k1 // 2 + 4 * n1 * (k1 // 64))
    gbs1 = algo_bytes(1, n1, k1) / (us1 * 1e-6) / 1e9
    gemv1 = {"shape": f"x [1, {k1}] . W[{n1}, {k1}]^T (gate_proj), 4-bit group 64, bf16 y", "us": round(us1, 2),
             "GBps": round(gbs1, 1), "frac_hbm_peak": round(gbs1 / HBM_PEAK_GBS, 4),
             "algo_bytes": algo_bytes(1, n1, k1)}

    per_proj = {}
    lm = None
    lm_triple = None
    if not args.quick:
        for m in (1, 4, 8):
            for name, n, k in LAYER:
                us = kernel_us(torch, lambda: Q.QuantizedLinear(*host[name]), m, k, n, xs[k],
                               n * k // 2 + 4 * n * (k // 64))
                per_proj[f"{name}_m{m}"] = {"us": round(us, 2), "GBps": round(algo_bytes(m, n, k) / (us * 1e-6) / 1e9, 1)}
            n, k = step_nk["qkv_proj"]
            us = kernel_us(torch, maker("qkv_proj"), m, k, n, xs[k], wbytes_of["qkv_proj"])
            per_proj[f"qkv_proj_m{m}"] = {"us": round(us, 2), "GBps": round(algo_bytes(m, n, k) / (us * 1e-6) / 1e9, 1)}
            us = pair_us(m)
            per_proj[f"{PAIR}_m{m}"] = {"us": round(us, 2),
                                        "GBps": round(pair_algo_bytes(m, f_gu, k_gu) / (us * 1e-6) / 1e9, 1)}
        try:
            log("quantizing lm_head 262144x3840")
            lm_triple = synthetic_weights(262144, HIDDEN, SEED_BASE + 3000)
            lm = {}
            for m in (1, 8, 16):
                us = kernel_us(torch, lambda: Q.QuantizedLinear(*lm_triple), m, HIDDEN, 262144, xs[HIDDEN],
                               262144 * HIDDEN // 2 + 4 * 262144 * (HIDDEN // 64), reps_per_graph=4)
                lm[f"m{m}"] = {"us": round(us, 1), "GBps": round(algo_bytes(m, 262144, HIDDEN) / (us * 1e-6) / 1e9, 1)}
        except Exception as e:  # memory or build problems should not hide the headline
            lm = {"error": str(e)}

    # --- prefill GEMM: the seven projections at M = 64, 256, 512, 2048 (gate at M=2048 headlines) ---
    gemm = None
    peaks = None
    if not args.no_gemm:
        if args.quick:
            gemm = prefill_sweep(torch, Q, host, (2048,), [l for l in LAYER if l[0] == "gate_proj"], pair=False,
                                 full_attention=False)
        else:
            gemm = prefill_sweep(torch, Q, host, PREFILL_MS, LAYER, pair=True, full_attention=True)
        head = gemm["gate_proj_m2048"]
        gemm["headline"] = {"shape": "gate_proj M=2048 N=15360 K=3840", **head}
        if not args.quick:
            log("practical peaks: 1 GiB copy, 1 GiB read, dense bf16 GEMM (hipBLASLt) on the gate shape")
            dense = dense_gemm_tflops(torch, 2048, 15360, HIDDEN)
            cg = copy_gbs(torch)
            rd = read_gbs(torch)
            peaks = {"copy_GBps": round(cg, 1), "read_GBps": rd["GBps"], "read_probe": rd,
                     "dense_bf16_gemm_TFLOPS_gate_m2048": round(dense, 1),
                     "roofline_frac_of_read": round(gu_gbs / rd["GBps"], 4),
                     "gemv_gate_m1_frac_of_read": round(gbs1 / rd["GBps"], 4),
                     "gemm_frac_of_dense": round(head["TFLOPS"] / dense, 4)}

    variants = None
    if not args.quick:
        log("8-bit and LoRA variants on the gate_proj shape")
        try:
            variants = variants_run(torch, Q, host)
        except Exception as e:  # memory or build problems should not hide the headline
            variants = {"error": str(e)}

    model = None
    if not args.quick:
        log("48-layer decoder: 16K prefill + 128 decode steps (quantized matmuls only)")
        try:
            model = model_run(torch, Q)
        except Exception as e:  # memory or build problems should not hide the headline
            model = {"error": str(e)}

    cpu = None
    if not args.no_cpu:
        log("CPU baseline")
        cpu = cpu_baseline(host, lm_triple)

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
                        "4-bit group-64 affine, hidden 3840, FFN 15360; launched as qkv, o, gate|up GeGLU pair, down",
            "global_batch": 1,
            "parallelism": "none (1 GPU)",
            "weight_copies_rotated": copies,
        },
        "pct_hbm_peak": round(value / HBM_PEAK_GBS * 100, 2),
        "headline_settle": settle_info,
        "gemv_gate_m1": gemv1,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "decode_step_by_m": step_by_m,
        "decode_step_unfused_m1": unfused,
        "decode_per_projection": per_proj,
        "lm_head": lm,
        "prefill_gemm": gemm,
        "variants_8bit_lora": variants,
        "model_48_layers": model,
        "practical_peaks": peaks,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
