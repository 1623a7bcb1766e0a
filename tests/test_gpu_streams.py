"""Concurrent use and graph capture of the C ABI on the GPU.

A handle is immutable after create, so forward may run on several streams and host
threads at once; per-call scratch comes from a stream-ordered pool and goes back on
the caller's stream.  Every kernel is deterministic (split-K partial sums are added in
split order), so concurrent results must equal the serial ones bit for bit:

  * four host threads, each on its own stream (default priority), run the decode
    path, the split-K GEMM, the gate|up pair and the greedy head on shared handles
    with their own inputs, interleaved; every output equals the serial result on the
    default stream;
  * the same calls captured once in a graph and replayed five times, the inputs
    rewritten by eager work between replays: every replay equals the eager result
    for its inputs.  Captured on a stream whose scratch memory is too small, the
    calls' scratch becomes allocation nodes of the graph; captured on a stream warmed
    up first, they use that stream's memory (no allocation nodes: asserted on the
    graph's node types); no memset nodes either way;
  * hipStreamPerThread from two threads at once: each thread's own stream and
    scratch;
  * gemma4_qmm_release_scratch returns a stream's memory.
"""

import threading

import numpy as np
import pytest

from oracle import affine as A
from test_gpu_parity import dev_triple, dev_x, random_triple

pytestmark = pytest.mark.gpu

K = 1024
N = 4096
F = 2048
# decode at 1 and 5 rows; 512 rows (32 slabs of 4M weights) take the GEMM
ROWS = (1, 5, 512)


def _handles(gpu_lib):
    lin = gpu_lib.QuantizedLinear(*dev_triple(*random_triple(N, K, 11)))
    pair = gpu_lib.QuantizedGeGLU(dev_triple(*random_triple(F, K, 12)), dev_triple(*random_triple(F, K, 13)))
    head = gpu_lib.QuantizedLinear(*dev_triple(*random_triple(20000, K, 14)))
    return lin, pair, head


def _run(lin, pair, head, xs, torch):
    """Every call of one round on the current stream: outputs in a list."""
    outs = []
    for x in xs:
        outs.append(lin.forward(x))
        outs.append(lin.forward(x, out_dtype=torch.float32))
        outs.append(pair.forward(x))
        if x.shape[0] <= 16:
            tok, val, logits = head.forward_greedy(x, softcap=30.0, return_logits=True)
            outs += [tok, val, logits]
    return outs


def _inputs(seed):
    return [dev_x(A.make_activations(m, K, seed=seed + m, outliers=True)) for m in ROWS]


def _same(a, b):
    import torch

    return (a.shape == b.shape and a.dtype == b.dtype
            and torch.equal(a.contiguous().view(torch.uint8), b.contiguous().view(torch.uint8)))


def test_threads_on_own_streams_match_serial(gpu_lib):
    import torch

    lin, pair, head = _handles(gpu_lib)
    threads_n, rounds = 4, 6
    inputs = [[_inputs(1000 * t + 10 * r) for r in range(rounds)] for t in range(threads_n)]
    # serial reference on the default stream
    want = [[_run(lin, pair, head, inputs[t][r], torch) for r in range(rounds)] for t in range(threads_n)]
    torch.cuda.synchronize()

    got = [[None] * rounds for _ in range(threads_n)]
    errors = []
    start = threading.Barrier(threads_n)

    def worker(t):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                start.wait(timeout=60)
                for r in range(rounds):
                    got[t][r] = _run(lin, pair, head, inputs[t][r], torch)
            s.synchronize()
        except Exception as e:  # reported below, with the thread
            errors.append((t, repr(e)))

    ts = [threading.Thread(target=worker, args=(t,), daemon=True) for t in range(threads_n)]
    for th in ts:
        th.start()
    for th in ts:
        th.join(timeout=120)
    assert not any(th.is_alive() for th in ts), "a worker thread did not finish"
    assert not errors, errors
    torch.cuda.synchronize()
    for t in range(threads_n):
        for r in range(rounds):
            for i, (a, b) in enumerate(zip(got[t][r], want[t][r])):
                assert _same(a, b), f"thread {t} round {r} output {i} differs from the serial result"
    for h in (lin, pair, head):
        h.close()


def test_graph_replays_match_eager(gpu_lib):
    import torch

    lin, pair, head = _handles(gpu_lib)
    xs = _inputs(5000)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _run(lin, pair, head, xs, torch)  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = _run(lin, pair, head, xs, torch)
    torch.cuda.synchronize()
    for rep in range(5):
        # eager work between replays: new inputs written into the captured buffers
        for i, m in enumerate(ROWS):
            xs[i].copy_(dev_x(A.make_activations(m, K, seed=7000 + 100 * rep + m, outliers=True)))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        want = _run(lin, pair, head, xs, torch)
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(outs, want)):
            assert _same(a, b), f"replay {rep}: output {i} differs from the eager result"
    del g
    for h in (lin, pair, head):
        h.close()


def test_per_thread_default_stream(gpu_lib):
    """hipStreamPerThread (the handle value 2) names a different stream in every
    thread: two threads issuing split-K GEMMs on it at once, each with its own
    inputs, match the serial results bit for bit (their scratch must not be shared)."""
    import torch

    lin = gpu_lib.QuantizedLinear(*dev_triple(*random_triple(N, K, 21)))
    m, rounds = 512, 8
    xs = [[dev_x(A.make_activations(m, K, seed=9000 + 100 * t + r)) for r in range(rounds)] for t in range(2)]
    want = [[lin.forward(x) for x in row] for row in xs]
    torch.cuda.synchronize()
    got = [[torch.empty_like(want[t][r]) for r in range(rounds)] for t in range(2)]
    errors = []
    start = threading.Barrier(2)

    def worker(t):
        try:
            start.wait(timeout=60)
            for r in range(rounds):
                lin.forward_raw(xs[t][r].data_ptr(), m, got[t][r].data_ptr(), stream_ptr=2)
            torch.cuda.synchronize()
        except Exception as e:  # reported below, with the thread
            errors.append((t, repr(e)))

    ts = [threading.Thread(target=worker, args=(t,), daemon=True) for t in range(2)]
    for th in ts:
        th.start()
    for th in ts:
        th.join(timeout=120)
    assert not any(th.is_alive() for th in ts), "a worker thread did not finish"
    assert not errors, errors
    torch.cuda.synchronize()
    for t in range(2):
        for r in range(rounds):
            assert _same(got[t][r], want[t][r]), f"thread {t} round {r} differs from the serial result"
    lin.close()


def test_graph_on_warmed_stream_matches_eager(gpu_lib):
    """Warm-up and capture on the same stream: the captured calls take their scratch
    from that stream's workspace (no allocation nodes).  Replays on that stream, with
    new inputs written between them, match the eager result; eager calls on another
    stream in between use their own workspace."""
    import torch

    lin, pair, head = _handles(gpu_lib)
    xs = _inputs(6000)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _run(lin, pair, head, xs, torch)  # grows s's workspace
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        outs = _run(lin, pair, head, xs, torch)
    torch.cuda.synchronize()
    for rep in range(4):
        for i, m in enumerate(ROWS):
            xs[i].copy_(dev_x(A.make_activations(m, K, seed=8000 + 100 * rep + m, outliers=True)))
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize()
        want = _run(lin, pair, head, xs, torch)  # the default stream
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(outs, want)):
            assert _same(a, b), f"replay {rep}: output {i} differs from the eager result"
    del g
    for h in (lin, pair, head):
        h.close()


def test_release_scratch(gpu_lib):
    """gemma4_qmm_release_scratch frees a stream's scratch memory (the device's free
    memory grows by at least what the split plan took), later calls on the stream
    allocate again and give the same bits, and a stream the library never used is a
    no-op."""
    import torch

    import hip_graph_nodes as G

    # k_proj's shape at 512 rows: 64-row tiles with K split four ways (partial planes)
    lin = gpu_lib.QuantizedLinear(*dev_triple(*random_triple(2048, 3840, 31)))
    x = dev_x(A.make_activations(512, 3840, seed=32))
    need = lin.scratch_bytes(512)
    assert need > 0
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        y1 = lin.forward(x)
    torch.cuda.synchronize()
    free0 = G.free_device_bytes()
    gpu_lib.release_scratch(s)
    assert G.free_device_bytes() >= free0 + need
    with torch.cuda.stream(s):
        y2 = lin.forward(x)
    torch.cuda.synchronize()
    assert _same(y1, y2)
    gpu_lib.release_scratch(s)
    gpu_lib.release_scratch(torch.cuda.Stream())
    lin.close()


def test_warmed_stream_capture_node_types(gpu_lib):
    """The node types behind the graph tests' claims: on a stream whose workspace was
    grown by the same calls, a capture of the decode path, the split-K GEMM, the pair
    and the greedy head holds kernel nodes only; on a cold stream the scratch-taking
    calls add allocation and free nodes; never a memset node."""
    import ctypes

    import torch

    import hip_graph_nodes as G

    lin, pair, head = _handles(gpu_lib)
    xs = _inputs(6500)
    lib = gpu_lib.load_library()
    outs = []
    for x in xs:
        m = x.shape[0]
        outs.append((x, torch.empty((m, N), dtype=torch.bfloat16, device="cuda"),
                     torch.empty((m, F), dtype=torch.bfloat16, device="cuda"),
                     torch.empty((m,), dtype=torch.int32, device="cuda"),
                     torch.empty((m,), dtype=torch.float32, device="cuda")))

    def issue(s):
        for x, y, h, tok, val in outs:
            m = x.shape[0]
            lin.forward(x, out=y, stream=s)
            pair.forward(x, out=h, stream=s)
            if m <= 16:
                st = lib.gemma4_qlinear_forward_greedy(head._handle, ctypes.c_void_p(s.cuda_stream),
                                                       ctypes.c_void_p(x.data_ptr()), m, 30.0, None,
                                                       gpu_lib.DTYPE_BF16, ctypes.c_void_p(tok.data_ptr()),
                                                       ctypes.c_void_p(val.data_ptr()))
                assert st == 0, gpu_lib.last_error()

    cold = torch.cuda.Stream()
    types_cold = G.capture_node_types(cold, lambda: issue(cold))
    assert G.MEM_ALLOC in types_cold and G.MEM_FREE in types_cold, types_cold
    assert G.MEMSET not in types_cold, types_cold
    warm = torch.cuda.Stream()
    issue(warm)
    torch.cuda.synchronize()
    types_warm = G.capture_node_types(warm, lambda: issue(warm))
    assert types_warm and all(t == G.KERNEL for t in types_warm), types_warm
    for h in (lin, pair, head):
        h.close()
