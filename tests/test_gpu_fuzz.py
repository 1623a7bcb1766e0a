"""Seeded random shapes through the C ABI on the GPU, against the oracle.

Each projection case draws N (or F for a gate|up pair), K (a multiple of 64), M from one of eight
row ranges (0, 1, 2, 3-4, 5-16, 17-31, 32-64, 65-300; GEMM cases also 300-2100), 4 or 8 bits, a bf16 or fp32
output, and the automatic path choice or the GEMM pinned from 32 rows.  Between them
the cases reach every decode variant (row, per-row-block, streaming, global-x; 16-row
slabs), the GEMM's 256-, 128- and 64-row tiles with and without a K split, and the
ragged edges (N not a multiple of 16, K not a multiple of 128, a last row block or
group pair partly empty).  Sampled rows are checked with the bars of
test_gpu_parity.py (bf16 max |err| <= 1e-2 RMS + ulp/2, fp32 <= 2e-3 RMS) and, for
pairs, test_gpu_geglu.py.  LoRA (rank 1-96) and the greedy head (M 1-16, softcap 0
or 30) get random shapes of their own, with the bars of test_gpu_lora.py and
test_gpu_greedy.py.  The int8 decode kernels, pinned, get random shapes of 1-8 rows
of their own (every output checked).
"""

import numpy as np
import pytest

from oracle import affine as A
from oracle import c_oracle as C
from test_gpu_geglu import _check as check_geglu
from test_gpu_parity import BF16_REL, F32_REL, assert_close, dev_triple, dev_x, host_bits

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


def _gemm_cases_tall(count=8, seed=20261209):
    """The GEMM at 300-2100 rows (the 64-row tile unsplit or split, the 128- and
    256-row tiles; N up to 3000 keeps the oracle rows cheap)."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(count):
        pair = bool(rng.random() < 0.3)
        bits = 8 if rng.random() < 0.25 else 4
        k = 64 * int(rng.integers(8, 129))
        per_row = k * (2 if bits == 8 else 1) * (2 if pair else 1)
        n_max = max(16, min(3000 if not pair else 1500, MAX_WEIGHTS // per_row))
        cases.append(dict(i=150 + i, n=int(rng.integers(16, n_max + 1)), k=k, m=int(rng.integers(300, 2101)),
                          pair=pair, bits=bits, f32=bool(rng.random() < 0.4), pin=True, outliers=i % 3 != 0))
    return cases


CASES = _cases() + _gemm_cases() + _gemm_cases_tall()


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


def _limb_cases(count=24, seed=20261206):
    """The int8 matrix-core decode kernels pinned (gemma4_qmm_set_decode_kernel 1) on
    random shapes of 1-8 rows: every launch shape of the one-row and the 2-8 row
    kernels, 4 and 8 bits, pairs, bf16 and fp32; every fourth case wide enough (more
    than 4096 row blocks) for the phased launch at 3-8 rows."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(count):
        m = 1 + i % 8
        pair = bool(rng.random() < 0.25)
        bits = 8 if rng.random() < 0.25 else 4
        f32 = bool(rng.random() < 0.4)
        if i % 4 == 3:
            k = 64 * int(rng.integers(1, 9))
            n = int(rng.integers(65_600, 80_001)) // (2 if pair else 1)
            bits = 4
        else:
            k = 64 * int(rng.integers(1, 129))
            per_row = k * (2 if bits == 8 else 1) * (2 if pair else 1)
            n = int(rng.integers(1, max(2, min(6000 if not pair else 3000, MAX_WEIGHTS // per_row)) + 1))
        cases.append(dict(i=400 + i, n=n, k=k, m=m, pair=pair, bits=bits, f32=f32, outliers=i % 3 != 0))
    return cases


@pytest.mark.parametrize("case", _limb_cases(), ids=lambda c: f"{c['i']}-{'pair' if c['pair'] else 'lin'}{c['bits']}"
                         f"-N{c['n']}-K{c['k']}-M{c['m']}{'-f32' if c['f32'] else ''}")
def test_random_shapes_int8_kernels(gpu_lib, case):
    import torch

    n, k, m, bits = case["n"], case["k"], case["m"], case["bits"]
    what = f"int8 case {case['i']}: {'pair' if case['pair'] else 'linear'} bits={bits} N={n} K={k} M={m} f32={case['f32']}"
    print(what, flush=True)
    x = A.make_activations(m, k, seed=2000 + case["i"], outliers=case["outliers"])
    dtype = torch.float32 if case["f32"] else torch.bfloat16
    seed = 66_000 + 10 * case["i"]
    with gpu_lib.decode_kernel(1):
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
    if case["pair"]:
        g = C.qmm_f64(x, *gate, bits=bits).astype(np.float32)
        u = C.qmm_f64(x, *up, bits=bits).astype(np.float32)
        check_geglu(y, g, u, what)
    else:
        assert_close(y, C.qmm_f64(x, *tri, bits=bits), what)


def _lora_cases(count=12, seed=20261204):
    """LoRA on random shapes: rank 1-96 (the fused one-launch path up to M = 4 and
    rank 64, the two-kernel path otherwise), M 1-200."""
    rng = np.random.default_rng(seed)
    ranges = [(1, 1), (2, 2), (3, 4), (5, 16), (17, 64), (65, 200)]
    cases = []
    for i in range(count):
        lo, hi = ranges[i % len(ranges)]
        k = 64 * int(rng.integers(1, 65))
        cases.append(dict(i=200 + i, n=int(rng.integers(1, 4001)), k=k, m=int(rng.integers(lo, hi + 1)),
                          r=int(rng.integers(1, 97)), f32=bool(rng.random() < 0.4),
                          scale=float(rng.choice([0.5, 2.0]))))
    return cases


@pytest.mark.parametrize("case", _lora_cases(), ids=lambda c: f"{c['i']}-N{c['n']}-K{c['k']}-M{c['m']}-r{c['r']}"
                         f"{'-f32' if c['f32'] else ''}")
def test_random_lora(gpu_lib, case):
    import torch

    from test_gpu_lora import check_bf16_two_roundings

    n, k, m, r = case["n"], case["k"], case["m"], case["r"]
    what = f"LoRA case {case['i']}: N={n} K={k} M={m} r={r} f32={case['f32']}"
    print(what, flush=True)
    seed = 88_000 + 10 * case["i"]
    tri = _triple(n, k, 4, seed)
    rng = np.random.default_rng(seed + 1)
    a = (rng.standard_normal((r, k)) * 0.02).astype(np.float32)
    b = (rng.standard_normal((n, r)) * 0.02).astype(np.float32)
    x = A.make_activations(m, k, seed=seed + 2, outliers=True)
    lin = gpu_lib.QuantizedLinear(*dev_triple(*tri))
    lora = gpu_lib.LoraAdapter(a, b, case["scale"])
    dt = torch.float32 if case["f32"] else torch.bfloat16
    y = lin.forward_lora(dev_x(x), lora, out_dtype=dt)
    torch.cuda.synchronize()
    lin.close()
    lora.close()
    rows = _rows(m, seed)
    xs = np.ascontiguousarray(x[rows])
    base = C.qmm_f64(xs, *tri).astype(np.float32)
    want = A.lora_ops(xs, a, b, case["scale"], base, bf16=not case["f32"]).astype(np.float64)
    got = host_bits(y[torch.from_numpy(rows).cuda()])
    if case["f32"]:
        ok, worst = A.check_f32_output(got, want, F32_REL)
    else:
        ok, worst = check_bf16_two_roundings(got, want)
    assert ok, f"{what}: worst error / RMS = {worst:.3e}"


def _greedy_cases(count=10, seed=20261205):
    """The greedy head (softcap + first argmax) on random shapes, M 1-16."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(count):
        k = 64 * int(rng.integers(1, 65))
        m = int(rng.integers(1, 17))
        n = int(rng.integers(2, min(30000, 200_000_000 // (m * k)) + 1))
        cases.append(dict(i=300 + i, n=n, k=k, m=m, cap=float(rng.choice([0.0, 30.0])),
                          f32=bool(rng.random() < 0.4)))
    return cases


@pytest.mark.parametrize("case", _greedy_cases(), ids=lambda c: f"{c['i']}-N{c['n']}-K{c['k']}-M{c['m']}"
                         f"-cap{int(c['cap'])}{'-f32' if c['f32'] else ''}")
def test_random_greedy(gpu_lib, case):
    import torch

    from test_gpu_greedy import _check_token

    n, k, m, cap = case["n"], case["k"], case["m"], case["cap"]
    what = f"greedy case {case['i']}: N={n} K={k} M={m} cap={cap} f32={case['f32']}"
    print(what, flush=True)
    seed = 99_000 + 10 * case["i"]
    tri = _triple(n, k, 4, seed)
    x = A.make_activations(m, k, seed=seed + 1, outliers=True)
    lin = gpu_lib.QuantizedLinear(*dev_triple(*tri))
    dt = torch.float32 if case["f32"] else torch.bfloat16
    tok, val, logits = lin.forward_greedy(dev_x(x), softcap=cap, out_dtype=dt, return_logits=True)
    torch.cuda.synchronize()
    lin.close()
    sc = A.softcap_ops(C.qmm_f64(x, *tri).astype(np.float32), cap, bf16=not case["f32"])
    lg = host_bits(logits)
    if case["f32"]:
        ok, worst = A.check_f32_output(lg, sc, F32_REL)
        lgf = lg
    else:
        ok, worst = A.check_bf16_output(lg, sc, BF16_REL)
        lgf = A.bf16_bits_to_f32(lg)
    assert ok, f"{what}: logits worst error / RMS = {worst:.3e}"
    tok, val = tok.cpu().numpy(), val.cpu().numpy()
    assert np.array_equal(val, lgf[np.arange(m), tok]), what  # the value is the logit at the token
    assert np.all(lgf <= val[:, None]), what                  # and the row's maximum
    _check_token(tok, sc, bf16=not case["f32"])
