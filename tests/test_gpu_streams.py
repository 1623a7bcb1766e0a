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
    up first, they use that stream's memory (no allocation nodes); no memset nodes
    either way;
  * hipStreamPerThread from two threads at once: each thread's own stream and
    scratch.
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
