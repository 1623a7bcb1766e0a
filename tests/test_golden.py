"""Golden vectors (tests/golden/q4_golden.npz, written by tests/golden/make_golden.py).

Expected values there come from exact rational arithmetic rounded once (RNE) to
fp32 / bf16, not from the oracle, so they pin:
  * the oracle (CPU): numpy and C dequantize bit-exact; float64 qmm rounded once
    gives exactly the correctly rounded fp32 and bf16 outputs;
  * the rounding helper itself, against numpy's own float64 -> float32 conversion;
  * the HIP path (GPU, through the C ABI): dequantize bit-exact; forward within the
    bars (fp32 output max|err| <= 2e-3 * RMS, bf16 output <= 1e-2 * RMS + half an
    ulp) on the decode path (M = 3) and on the GEMM path (the rows repeated to M = 40).
"""

import os
import sys
from fractions import Fraction

import numpy as np
import pytest

from oracle import affine as A
from oracle import c_oracle as C

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_golden as G  # noqa: E402

GOLDEN = np.load(os.path.join(HERE, "golden", "q4_golden.npz"))
CASES = ("mm", "ed")


def test_rounding_helper_matches_ieee_conversion():
    rng = np.random.default_rng(5)
    vals = np.concatenate([rng.standard_normal(2000) * 10.0 ** rng.integers(-45, 38, 2000),
                           [1.0 + 2.0 ** -24, 1.0 + 3 * 2.0 ** -24, 2.0 ** -149 * 1.5, 2.0 ** -149 * 2.5,
                            3.4028235677973366e38, -0.0, 2.0 ** -150]])
    with np.errstate(over="ignore"):  # values beyond the fp32 range round to inf on both sides
        for v in vals:
            assert G.round_fraction(Fraction(float(v)), 24) == float(np.float32(v)), v
    f = (rng.standard_normal(2000) * 10.0 ** rng.integers(-30, 30, 2000)).astype(np.float32)
    want = A.f32_to_bf16_bits(f)
    got = np.array([G.f32_bits(G.round_fraction(Fraction(float(v)), 8)) >> 16 for v in f], dtype=np.uint16)
    assert np.array_equal(got, want)


def test_fixture_matches_generator():
    # the committed file is what the committed script writes
    data = {}
    for fn in (G.dequant_case, G.matmul_case, G.edge_case):
        data.update(fn())
    assert sorted(data) == sorted(GOLDEN.files)
    for k, v in data.items():
        assert np.array_equal(np.asarray(v), GOLDEN[k]), k


def test_oracle_dequantize_bit_exact():
    want = GOLDEN["dq_w_f32"].view(np.uint32)
    args = (GOLDEN["dq_wq"], GOLDEN["dq_scales"], GOLDEN["dq_biases"])
    assert np.array_equal(A.dequantize(*args).view(np.uint32), want)
    assert np.array_equal(C.dequantize(*args).view(np.uint32), want)


@pytest.mark.parametrize("case", CASES)
def test_oracle_qmm_correctly_rounded(case):
    g = {k: GOLDEN[f"{case}_{k}"] for k in ("x", "wq", "scales", "biases", "y_exact", "y_f32", "y_bf16")}
    for y in (A.qmm_f64(g["x"], g["wq"], g["scales"], g["biases"]),
              C.qmm_f64(g["x"], g["wq"], g["scales"], g["biases"])):
        y = np.asarray(y)
        assert np.array_equal(y.astype(np.float32).view(np.uint32), g["y_f32"].view(np.uint32))
        assert np.array_equal(A.f32_to_bf16_bits(y.astype(np.float32)), g["y_bf16"])
        assert np.allclose(y, g["y_exact"], rtol=1e-15, atol=0)


@pytest.mark.gpu
def test_gpu_dequantize_golden(gpu_lib):
    from test_gpu_parity import dev_triple

    lin = gpu_lib.QuantizedLinear(*dev_triple(GOLDEN["dq_wq"], GOLDEN["dq_scales"], GOLDEN["dq_biases"]))
    got = lin.dequantize().cpu().numpy()
    lin.close()
    assert np.array_equal(got.view(np.uint32), GOLDEN["dq_w_f32"].view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("rows", [3, 40])
@pytest.mark.parametrize("out_dtype", ["bf16", "f32"])
def test_gpu_forward_golden(gpu_lib, gemm_from_32, case, rows, out_dtype):
    import torch

    from test_gpu_parity import BF16_REL, F32_REL, dev_triple, dev_x, host_bits

    g = {k: GOLDEN[f"{case}_{k}"] for k in ("x", "wq", "scales", "biases", "y_exact", "y_f32")}
    reps = -(-rows // g["x"].shape[0])
    x = np.tile(g["x"], (reps, 1))[:rows]
    y_exact = np.tile(g["y_exact"], (reps, 1))[:rows]
    lin = gpu_lib.QuantizedLinear(*dev_triple(g["wq"], g["scales"], g["biases"]))
    dt = torch.bfloat16 if out_dtype == "bf16" else torch.float32
    y = lin.forward(dev_x(x), out_dtype=dt)
    torch.cuda.synchronize()
    lin.close()
    if out_dtype == "bf16":
        ok, worst = A.check_bf16_output(host_bits(y), y_exact, BF16_REL)
    else:
        ok, worst = A.check_f32_output(host_bits(y), y_exact, F32_REL)
        # all-zero activation rows give exactly zero
        zero_rows = ~np.any(A.bf16_bits_to_f32(x) != 0, axis=1)
        assert np.all(host_bits(y)[zero_rows] == 0)
    assert ok, f"{case} rows={rows} {out_dtype}: worst error / RMS = {worst:.3e}"
