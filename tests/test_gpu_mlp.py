"""GPU parity of gemma4_qmlp_forward, the MLP block in one call (gate|up -> GeGLU ->
down; native_model.cc:1318-1321 at decode, :934-949 in prefill), through the C ABI.

It queues the gate|up pair's launch and then down's, so it must give the bits of the
two separate calls (gemma4_qgeglu_forward, then gemma4_qlinear_forward on its h) on
every path: one row (the int8 decode kernels), decode slabs, the GEMM, 8-bit handles
and the bf16 kernels pinned.  Against the oracle (bars of test_gpu_geglu.py and
test_gpu_parity.py): h against geglu_ops of the correctly rounded exact gate and up
products; y against the float64 product of down with the call's own h (one rounding
of a value within ACC_REL * RMS of it).  Repeated calls and graph replays with new
inputs between them give the eager bits; argument errors are reported.
"""

import numpy as np
import pytest

from oracle import affine as A
from oracle import c_oracle as C

from test_gpu_geglu import _check, _exact_gu
from test_gpu_parity import assert_rounded, dev_triple, dev_x, host_bits, random_triple

pytestmark = pytest.mark.gpu

F, K, N = 15360, 3840, 3840


def _mlp(gpu_lib, f, k, n, seed, bits=4):
    if bits == 4:
        gate, up, down = random_triple(f, k, seed), random_triple(f, k, seed + 1), random_triple(n, f, seed + 2)
    else:
        rng = np.random.default_rng(seed)
        gate, up, down = (C.quantize(A.round_to_bf16((rng.standard_normal(s) * 0.02).astype(np.float32)), bits=8)
                          for s in ((f, k), (f, k), (n, f)))
    pair = gpu_lib.QuantizedGeGLU(dev_triple(*gate), dev_triple(*up), bits=bits)
    d = gpu_lib.QuantizedLinear(*dev_triple(*down), bits=bits)
    return gate, up, down, pair, d


def _two_calls(pair, d, xd):
    h = pair.forward(xd)
    return d.forward(h), h


@pytest.mark.parametrize("f,k,n,m", [(F, K, N, 1), (F, K, N, 8), (F, K, N, 512), (64, 192, 48, 1),
                                     (192, 64, 40, 3), (1024, 640, 136, 40)])
def test_mlp_block(gpu_lib, f, k, n, m):
    import torch

    gate, up, down, pair, d = _mlp(gpu_lib, f, k, n, seed=7100 + f + k + m)
    x = A.make_activations(m, k, seed=7200 + f + m, outliers=True)
    xd = dev_x(x)
    y, h = pair.forward_mlp(d, xd)
    y2, h2 = _two_calls(pair, d, xd)
    torch.cuda.synchronize()
    assert tuple(y.shape) == (m, n) and tuple(h.shape) == (m, f)
    assert torch.equal(h, h2) and torch.equal(y, y2)
    rows = np.unique(np.linspace(0, m - 1, min(m, 6)).astype(np.int64))
    rt = torch.from_numpy(rows).cuda()
    _check(h[rt], *_exact_gu(x, gate, up, rows), f"h F={f} K={k} M={m}")
    y_exact = C.qmm_f64(np.ascontiguousarray(host_bits(h)[rows]), *down)
    assert_rounded(y[rt].contiguous(), y_exact, f"y F={f} K={k} N={n} M={m}")
    for obj in (pair, d):
        obj.close()


def test_mlp_block_pinned_bf16_kernels_and_8bit(gpu_lib):
    import torch

    _, _, _, pair, d = _mlp(gpu_lib, 1024, 640, 136, seed=7900)
    xd = dev_x(A.make_activations(1, 640, seed=7901))
    with gpu_lib.decode_kernel(2):
        y, h = pair.forward_mlp(d, xd)
        y2, h2 = _two_calls(pair, d, xd)
    torch.cuda.synchronize()
    assert torch.equal(h, h2) and torch.equal(y, y2)
    _, _, _, p8, d8 = _mlp(gpu_lib, 256, 640, 136, seed=7902, bits=8)
    y, h = p8.forward_mlp(d8, xd)
    y2, h2 = _two_calls(p8, d8, xd)
    torch.cuda.synchronize()
    assert torch.equal(h, h2) and torch.equal(y, y2)
    for obj in (pair, d, p8, d8):
        obj.close()


def test_mlp_block_graph_replays(gpu_lib):
    """A graph of three one-row MLP calls replayed five times with new inputs written
    between replays: every replay equals the eager result bit for bit."""
    import torch

    _, _, _, pair, d = _mlp(gpu_lib, F, K, N, seed=7300)
    xs = [dev_x(A.make_activations(1, K, seed=7500 + i)) for i in range(3)]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for x in xs:
            pair.forward_mlp(d, x)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        outs = [pair.forward_mlp(d, x) for x in xs]
    torch.cuda.synchronize()
    for rep in range(5):
        for i, x in enumerate(xs):
            x.copy_(dev_x(A.make_activations(1, K, seed=7600 + 10 * rep + i)))
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize()
        for i, x in enumerate(xs):
            y, h = pair.forward_mlp(d, x)
            torch.cuda.synchronize()
            assert torch.equal(outs[i][1], h), f"replay {rep} call {i}: h differs from eager"
            assert torch.equal(outs[i][0], y), f"replay {rep} call {i}: y differs from eager"
    del g
    for obj in (pair, d):
        obj.close()


def test_mlp_block_argument_errors(gpu_lib):
    import ctypes

    import torch

    _, _, _, pair, d = _mlp(gpu_lib, 64, 192, 48, seed=8200)
    wrong = gpu_lib.QuantizedLinear(*dev_triple(*random_triple(48, 128, 8201)))  # K != F
    lib = gpu_lib.load_library()
    x = dev_x(A.make_activations(1, 192, seed=8202))
    h = torch.empty((1, 64), dtype=torch.bfloat16, device="cuda")
    y = torch.empty((1, 48), dtype=torch.bfloat16, device="cuda")
    P = gpu_lib._dev_ptr

    def call(a, b, dtype=gpu_lib.DTYPE_BF16, hp=None):
        return lib.gemma4_qmlp_forward(a._handle, b._handle, None, P(x), 1, hp or P(h), P(y), dtype)

    assert call(pair, wrong) == gpu_lib.Status.INVALID_ARGUMENT and "in_features" in gpu_lib.last_error()
    assert call(d, d) == gpu_lib.Status.INVALID_ARGUMENT and "gate|up pair" in gpu_lib.last_error()
    assert call(pair, pair) == gpu_lib.Status.INVALID_ARGUMENT and "one projection" in gpu_lib.last_error()
    assert call(pair, d, gpu_lib.DTYPE_F32) == gpu_lib.Status.UNSUPPORTED_CONFIG
    assert call(pair, d, hp=ctypes.c_void_p(h.data_ptr() + 2)) == gpu_lib.Status.INVALID_ARGUMENT
    assert call(pair, d) == gpu_lib.Status.OK
    torch.cuda.synchronize()
    for obj in (pair, d, wrong):
        obj.close()
