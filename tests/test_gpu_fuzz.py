"""Seeded random shapes through the C ABI on the GPU, against the oracle.

Each case draws N (or F for a gate|up pair), K (a multiple of 64), M from one of eight
row ranges (0, 1, 2, 3-4, 5-16, 17-31, 32-64, 65-300), 4 or 8 bits, a bf16 or fp32
output, and the automatic path choice or the GEMM pinned from 32 rows.  Between them
the cases reach every decode variant (row, per-row-block, streaming, global-x; 16-row
slabs), the GEMM's 256-, 128- and 64-row tiles with and without a K split, and the
ragged edges (N not a multiple of 16, K not a multiple of 128, a last row block or
group pair partly empty).  Sampled rows are checked with the bars of
test_gpu_parity.py (bf16 max |err| <= 1e-2 RMS + ulp/2, fp32 <= 2e-3 RMS) and, for
pairs, test_gpu_geglu.py.
"""

import numpy as np
import pytest

from oracle import affine as A
from oracle import c_oracle as C
from test_gpu_geglu import _check as check_geglu
from test_gpu_parity import assert_close, dev_triple, dev_x

pytestmark = pytest.mark.gpu

M_RANGES = [(0, 0), (1, 1), (2, 2), (3, 4), (5, 16), (17, 31), (32, 64), (65, 300)]
MAX_WEIGHTS = 12_000_000  # per case (both halves of a pair, both planes at 8 bits)
SAMPLE_ROWS = 12


def _cases(count=40, seed=20261202):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(count):
        lo, hi = M_RANGES[i % len(M_RANGES)]
        m = int(rng.integers(lo, hi + 1))
        pair = bool(rng.random() < 0.3)
        bits = 8 if rng.random() < 0.25 else 4
        f32 = bool(rng.random() < 0.4)
        pin = bool(rng.random() < 0.5)
        k = 64 * int(rng.integers(1, 129))
        per_row = k * (2 if bits == 8 else 1) * (2 if pair else 1)
        n_max = max(1, min(6000 if not pair else 3000, MAX_WEIGHTS // per_row))
        n = int(rng.integers(1, n_max + 1))
        cases.append(dict(i=i, n=n, k=k, m=m, pair=pair, bits=bits, f32=f32, pin=pin, outliers=i % 3 != 0))
    return cases


def _gemm_cases(count=16, seed=20261203):
    """Cases on the GEMM: M of 32-300 rows (half of them <= 64: the 64-row tile), the
    GEMM pinned, pairs more often."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(count):
        m = int(rng.integers(32, 65)) if i % 2 == 0 else int(rng.integers(65, 301))
        pair = bool(rng.random() < 0.4)
        bits = 8 if rng.random() < 0.25 else 4
        f32 = bool(rng.random() < 0.4)
        k = 64 * int(rng.integers(1, 129))
        per_row = k * (2 if bits == 8 else 1) * (2 if pair else 1)
        n_max = max(1, min(6000 if not pair else 3000, MAX_WEIGHTS // per_row))
        n = int(rng.integers(1, n_max + 1))
        cases.append(dict(i=100 + i, n=n, k=k, m=m, pair=pair, bits=bits, f32=f32, pin=True, outliers=i % 3 != 0))
    return cases


CASES = _cases() + _gemm_cases()


def _triple(n, k, bits, seed):
    rng = np.random.default_rng(seed)
    w = A.round_to_bf16((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    return C.quantize(w, bits=bits) if bits == 8 else C.quantize(w)


def _rows(m, seed):
    if m <= SAMPLE_ROWS:
        return np.arange(m)
    rows = np.random.default_rng(seed).choice(m, SAMPLE_ROWS - 1, replace=False)
    return np.unique(np.concatenate([rows, [m - 1]]))


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c['i']}-{'pair' if c['pair'] else 'lin'}{c['bits']}"
                         f"-N{c['n']}-K{c['k']}-M{c['m']}{'-f32' if c['f32'] else ''}{'-gemm' if c['pin'] and c['m'] >= 32 else ''}")
def test_random_shapes(gpu_lib, case):
    import torch

    n, k, m, bits = case["n"], case["k"], case["m"], case["bits"]
    what = f"case {case['i']}: {'pair' if case['pair'] else 'linear'} bits={bits} N={n} K={k} M={m} f32={case['f32']}"
    print(what, flush=True)
    x = A.make_activations(m, k, seed=1000 + case["i"], outliers=case["outliers"]) if m > 0 else \
        np.zeros((0, k), np.uint16)
    dtype = torch.float32 if case["f32"] else torch.bfloat16
    seed = 77_000 + 10 * case["i"]
    with gpu_lib.gemm_min_rows(32 if case["pin"] else 0):
        if case["pair"]:
            gate, up = _triple(n, k, bits, seed), _triple(n, k, bits, seed + 1)
            obj = gpu_lib.QuantizedGeGLU(dev_triple(*gate), dev_triple(*up), bits=bits)
        else:
            tri = _triple(n, k, bits, seed)
            obj = gpu_lib.QuantizedLinear(*dev_triple(*tri), bits=bits)
        y = obj.forward(dev_x(x), out_dtype=dtype)
        torch.cuda.synchronize()
    obj.close()
    assert tuple(y.shape) == (m, n) and y.dtype == dtype, what
    if m == 0:
        return
    rows = _rows(m, seed)
    xs = np.ascontiguousarray(x[rows])
    rt = torch.from_numpy(rows).cuda()
    if case["pair"]:
        g = C.qmm_f64(xs, *gate, bits=bits).astype(np.float32)
        u = C.qmm_f64(xs, *up, bits=bits).astype(np.float32)
        check_geglu(y[rt], g, u, what)
    else:
        assert_close(y[rt], C.qmm_f64(xs, *tri, bits=bits), what)
