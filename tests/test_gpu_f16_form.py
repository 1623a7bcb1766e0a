"""GPU parity of the GEMM's fp16 form against the oracle, beside the bf16 form.

The fp16 form (256-row tiles of handles whose scales allow it) scales each row of x by
a power of two into fp16, exact for every x within 2^32 of the row's largest, and
expands the weights as s 2^p (q - 8), exact in fp16 when every nonzero scale lies
within 2^26 of the largest; the matrix cores then sum exact products with no
per-group scale step.  gemma4_qmm_set_gemm_form(1) pins the bf16 form, so both run on
the same inputs.  Checks (bars of test_gpu_parity.py's prefill tests: bf16 outputs
within 1e-2 RMS + ulp/2 of the float64 oracle, fp32 within GEMM_REL = 5e-4 RMS):
  * the plan takes the form where it should: the workspace grows by the fp16 copy of x
    and the row exponents exactly when the handle's scales allow it;
  * gate at 2048 rows, ragged rows and row blocks (15000 x 3840 at 1000 rows), a
    last octet of one group (K = 2112) and the gate|up pair, bf16 and fp32, sampled
    rows against the oracle in both forms, and the two forms' fp32 outputs within
    GEMM_REL * RMS of each other;
  * scales far from 1 (all near 2^-30: the power p moves them into range) stay in the
    fp16 form; scales spanning more than 2^26, or holding inf, fall back to the bf16
    form; both correct;
  * rows of x with extreme ranges, each against its own oracle row: an outlier of 2^100
    beside values near 1, values near 2^-100, a row of zeros, values spread over 2^-40
    to 2^40, and a row holding inf (its outputs not finite, every other row's finite
    and correct);
  * an 8-bit handle (two 4-bit planes, 16 s in the high one) against the bf16 form
    (the plan may take the fp16 form or the one-pass 8-bit form of
    test_gpu_q8_one_pass.py);
  * graph replays of the fp16 form equal the eager call.
"""

import numpy as np
import pytest

from oracle import affine as A
from oracle import c_oracle as C

from test_gpu_parity import assert_close, dev_triple, dev_x, host_bits, random_triple

pytestmark = pytest.mark.gpu

# the GEMM's fp32 accumulation bar (test_gpu_parity.py's prefill tests): exact products
# summed in fp32 over K, the bf16 form through one scale step per group
GEMM_REL = 5e-4


def _round256(b):
    return (b + 255) // 256 * 256


def _forms(lin, x, m, dtype):
    """Outputs of the fp16 form (the default) and the pinned bf16 form."""
    import torch

    from helios_amd import qmm as Q

    y16 = lin.forward(x, out_dtype=dtype)
    with Q.gemm_form(1):
        ybf = lin.forward(x, out_dtype=dtype)
    torch.cuda.synchronize()
    return y16, ybf


def _takes_f16(lin, m, kx):
    from helios_amd import qmm as Q

    auto = lin.scratch_bytes(m)
    with Q.gemm_form(1):
        bf = lin.scratch_bytes(m)
    if auto == bf:
        return False
    assert auto - bf == _round256(m * kx * 2) + _round256(m * 4), (auto, bf)
    return True


def _check_rows(y16, ybf, want, rt, what):
    import torch

    if y16.dtype == torch.bfloat16:
        assert_close(y16[rt], want, what + " fp16 form")
        assert_close(ybf[rt], want, what + " bf16 form")
    else:
        assert assert_close(y16[rt], want, what + " fp16 form") < GEMM_REL
        assert assert_close(ybf[rt], want, what + " bf16 form") < GEMM_REL
        rms = float(np.sqrt(np.mean(np.asarray(want, np.float64) ** 2)))
        diff = float((y16[rt] - ybf[rt]).abs().max())
        assert diff <= GEMM_REL * rms, f"{what}: forms differ by {diff / rms:.3e} x RMS"


@pytest.mark.parametrize("name,n,k,m", [("gate", 15360, 3840, 2048), ("ragged rows and row blocks", 15000, 3840, 1000),
                                        ("a last octet of one group", 12288, 2112, 1000)])
def test_fp16_form_projections(gpu_lib, name, n, k, m):
    import torch

    tri = random_triple(n, k, seed=6100 + n)
    lin = gpu_lib.QuantizedLinear(*dev_triple(*tri))
    assert _takes_f16(lin, m, k), f"{name}: the fp16 form was not planned at {m} rows"
    x = A.make_activations(m, k, seed=6200 + n, outliers=True)
    xd = dev_x(x)
    rows = np.unique(np.linspace(0, m - 1, 8).astype(np.int64))
    rt = torch.from_numpy(rows).cuda()
    want = C.qmm_f64(np.ascontiguousarray(x[rows]), *tri)
    for dtype in (torch.bfloat16, torch.float32):
        y16, ybf = _forms(lin, xd, m, dtype)
        _check_rows(y16, ybf, want, rt, f"{name} {dtype}")
    lin.close()


def test_fp16_form_gate_up_pair(gpu_lib):
    import torch

    from test_gpu_geglu import _check, _exact_gu

    f, k, m = 15360, 3840, 2048
    gate, up = random_triple(f, k, 6300), random_triple(f, k, 6301)
    pair = gpu_lib.QuantizedGeGLU(dev_triple(*gate), dev_triple(*up))
    assert _takes_f16(pair, m, k)
    x = A.make_activations(m, k, seed=6302, outliers=True)
    xd = dev_x(x)
    rows = np.unique(np.linspace(0, m - 1, 6).astype(np.int64))
    rt = torch.from_numpy(rows).cuda()
    h16, hbf = _forms(pair, xd, m, torch.bfloat16)
    g_exact, u_exact = _exact_gu(x, gate, up, rows)
    _check(h16[rt], g_exact, u_exact, "pair fp16 form")
    _check(hbf[rt], g_exact, u_exact, "pair bf16 form")
    pair.close()


def test_fp16_form_scale_ranges(gpu_lib):
    import torch

    n, k, m = 15360, 3840, 2048
    wq, s, b = random_triple(n, k, seed=6400)
    x = A.make_activations(m, k, seed=6401, outliers=True)
    xd = dev_x(x)
    rows = np.array([0, 1, 777, 2047])
    rt = torch.from_numpy(rows).cuda()
    sf = A.bf16_bits_to_f32(s)
    bf = A.bf16_bits_to_f32(b)
    cases = {
        # every scale and bias times 2^-30: p moves the scales back into range
        "small": (A.f32_to_bf16_bits(sf * 2.0 ** -30), A.f32_to_bf16_bits(bf * 2.0 ** -30), True),
        # one group's scale 2^-40 of the others: more than 2^26 apart
        "wide": (s.copy(), b, False),
        # one scale inf
        "inf": (s.copy(), b, False),
        # every scale a bf16 subnormal (exponent field 0) and no biases: the fp16 form
        # would flush them, so the handle keeps the bf16 form
        "subnormal": (A.f32_to_bf16_bits(sf * 2.0 ** -123), np.zeros_like(b), False),
        # every scale zero: the products are the biases' alone, in either form
        "zero": (np.zeros_like(s), b, True),
    }
    cases["wide"][0][5, 7] = A.f32_to_bf16_bits(np.array([sf[5, 7] * 2.0 ** -40], np.float32))[0]
    cases["inf"][0][9, 3] = 0x7F80
    sub = cases["subnormal"][0]
    assert ((sub & 0x7F80) == 0).all() and (sub & 0x7F).any()  # subnormal or zero, some nonzero
    for what, (s2, b2, f16) in cases.items():
        tri = (wq, s2, b2)
        lin = gpu_lib.QuantizedLinear(*dev_triple(*tri))
        assert _takes_f16(lin, m, k) == f16, what
        if what == "inf":
            y = lin.forward(xd)
            torch.cuda.synchronize()
            yf = A.bf16_bits_to_f32(host_bits(y))
            assert not np.isfinite(yf[:, 9]).all() and np.isfinite(np.delete(yf, 9, axis=1)).all(), what
            lin.close()
            continue
        want = C.qmm_f64(np.ascontiguousarray(x[rows]), *tri)
        for dtype in (torch.bfloat16, torch.float32):
            y16, ybf = _forms(lin, xd, m, dtype)
            _check_rows(y16, ybf, want, rt, f"scales {what} {dtype}")
        lin.close()


def test_fp16_form_extreme_rows(gpu_lib):
    import torch

    n, k, m = 15360, 3840, 2048
    tri = random_triple(n, k, seed=6500)
    lin = gpu_lib.QuantizedLinear(*dev_triple(*tri))
    assert _takes_f16(lin, m, k)
    rng = np.random.default_rng(6501)
    xf = A.bf16_bits_to_f32(A.make_activations(m, k, seed=6502)).copy()
    xf[0, 17] = 2.0 ** 100                                    # an outlier beside values near 1
    xf[1] = rng.standard_normal(k) * 2.0 ** -100              # values near 2^-100
    xf[2] = 0.0                                               # zeros
    xf[3] = rng.standard_normal(k) * 2.0 ** rng.integers(-40, 41, k)  # spread over 2^-40..2^40
    xf[5, 100] = np.inf                                       # inf: this row's outputs not finite
    xf[6] = rng.standard_normal(k) * 2.0 ** -130              # bf16 subnormals only (exponent 0)
    x = A.f32_to_bf16_bits(xf.astype(np.float32))
    xd = dev_x(x)
    checked = [0, 1, 3, 4, 6, 2047]
    for dtype in (torch.bfloat16, torch.float32):
        y16, ybf = _forms(lin, xd, m, dtype)
        for r in checked:
            want = C.qmm_f64(np.ascontiguousarray(x[r:r + 1]), *tri)
            _check_rows(y16, ybf, want, torch.tensor([r], device="cuda"), f"row {r} {dtype}")
        z16 = host_bits(y16[2:3]) if dtype == torch.float32 else A.bf16_bits_to_f32(host_bits(y16[2:3]))
        assert not np.any(z16), f"zero row {dtype}: nonzero outputs"
        for y in (y16, ybf):
            yf = host_bits(y) if dtype == torch.float32 else A.bf16_bits_to_f32(host_bits(y))
            assert not np.isfinite(yf[5]).all(), f"inf row {dtype}"
            assert np.isfinite(np.delete(yf, 5, axis=0)).all(), f"rows other than the inf row {dtype}"
    lin.close()


def test_fp16_form_eight_bit(gpu_lib):
    import torch

    n, k, m = 15360, 3840, 2048
    rng = np.random.default_rng(6600)
    w = A.round_to_bf16((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    tri = C.quantize(w, bits=8)
    lin = gpu_lib.QuantizedLinear(*dev_triple(*tri), bits=8)
    x = A.make_activations(m, k, seed=6601, outliers=True)
    xd = dev_x(x)
    rows = np.array([0, 255, 256, 1500, 2047])
    rt = torch.from_numpy(rows).cuda()
    want = C.qmm_f64(np.ascontiguousarray(x[rows]), *tri, bits=8)
    for dtype in (torch.bfloat16, torch.float32):
        y16, ybf = _forms(lin, xd, m, dtype)
        _check_rows(y16, ybf, want, rt, f"8-bit {dtype}")
    lin.close()


def test_fp16_form_graph_replays(gpu_lib):
    """Three gate calls at 2048 rows captured in a graph, replayed four times with new
    inputs written between replays: every replay equals the eager result."""
    import torch

    n, k, m = 15360, 3840, 2048
    lin = gpu_lib.QuantizedLinear(*dev_triple(*random_triple(n, k, seed=6700)))
    assert _takes_f16(lin, m, k)
    xs = [dev_x(A.make_activations(m, k, seed=6710 + i)) for i in range(3)]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for x in xs:
            lin.forward(x)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        outs = [lin.forward(x) for x in xs]
    torch.cuda.synchronize()
    for rep in range(4):
        for i, x in enumerate(xs):
            x.copy_(dev_x(A.make_activations(m, k, seed=6720 + 10 * rep + i, outliers=True)))
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize()
        for i, x in enumerate(xs):
            y = lin.forward(x)
            torch.cuda.synchronize()
            assert torch.equal(outs[i], y), f"replay {rep} call {i} differs from eager"
    del g
    lin.close()
