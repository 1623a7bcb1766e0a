"""GPU parity of the int8-limb decode kernels (q4_limbs.hip: one row of x, and 2-8 rows).

The kernel splits every 64-column group of x into three int8 limbs relative to the
group's largest magnitude (exact for every x within 2^12 of it, rounded at 2^-21 of
it otherwise) and sums on the int8 matrix cores.  Bars, as in test_gpu_parity.py:
fp32 output within 2e-3 * RMS of the float64 oracle (and, the kernel's actual
accuracy, within ACC_REL = 1e-4 * RMS); bf16 output one rounding of such a value.
Cases: every Gemma projection and the fused q|k|v at full size under both kernel
families (gemma4_qmm_set_decode_kernel 1 and 2), each of the three launch shapes
(long K with at most one row block per CU, up to four row blocks per CU, more),
ragged N and odd group counts, groups whose values span the whole bf16 exponent
range (subnormals, zeros, the largest finite values), inf/NaN inputs, and run-to-run
determinism."""

import numpy as np
import pytest

from oracle import affine as A
from oracle import c_oracle as C

from test_gpu_parity import ACC_REL, F32_REL, PROJ, assert_close, assert_rounded, dev_triple, dev_x, host_bits, random_triple

pytestmark = pytest.mark.gpu


def run(lin, x_bits, f32, variant, gpu_lib):
    import torch

    with gpu_lib.decode_kernel(variant):
        y = lin.forward(dev_x(x_bits), out_dtype=torch.float32 if f32 else torch.bfloat16)
    torch.cuda.synchronize()
    return y


@pytest.mark.parametrize("proj", sorted(PROJ) + ["qkv_proj"])
def test_projections_both_kernels(gpu_lib, proj):
    """Full-size projections at one row: the int8 kernel and the bf16 kernels each
    against the oracle, bf16 and fp32 outputs."""
    if proj == "qkv_proj":
        parts = [A.make_weights(*PROJ[p], seed=4000 + i) for i, p in enumerate(("q_proj", "k_proj", "v_proj"))]
        wq, s, b = (np.concatenate([p[j] for p in parts]) for j in range(3))
        k = 3840
    else:
        n, k = PROJ[proj]
        wq, s, b = A.make_weights(n, k, seed=4100 + sorted(PROJ).index(proj))
    x = A.make_activations(1, k, seed=4200, outliers=True)
    lin = gpu_lib.QuantizedLinear(*dev_triple(wq, s, b))
    y_exact = C.qmm_f64(x, wq, s, b)
    for variant in (1, 2):
        y_f = run(lin, x, True, variant, gpu_lib)
        assert assert_close(y_f, y_exact, f"{proj} kernel {variant} f32") < ACC_REL
        y_b = run(lin, x, False, variant, gpu_lib)
        assert_rounded(y_b, y_exact, f"{proj} kernel {variant} bf16")
    lin.close()


# (N, K): one row block per CU or fewer with long K (16-wave workgroups); up to four
# per CU; more (three workgroups per CU, blocks dealt round the grid); odd group
# counts (the last chunk holds one record), K of one group, ragged N
SHAPES = [(3840, 15360), (256, 8192), (40, 320), (1000, 192), (16, 64), (33, 640), (4096 + 8, 3840),
          (15360, 3840), (20000, 576), (70000 + 40, 384), (131072, 128)]


@pytest.mark.parametrize("n,k", SHAPES)
def test_launch_shapes(gpu_lib, n, k):
    wq, s, b = random_triple(n, k, seed=n + 3 * k)
    x = A.make_activations(1, k, seed=n, outliers=True)
    lin = gpu_lib.QuantizedLinear(*dev_triple(wq, s, b))
    y_exact = C.qmm_f64(x, wq, s, b)
    y_f = run(lin, x, True, 1, gpu_lib)
    assert assert_close(y_f, y_exact, f"{n}x{k} f32") < ACC_REL
    y_b = run(lin, x, False, 1, gpu_lib)
    assert_close(y_b, y_exact, f"{n}x{k} bf16")
    lin.close()


def _wide_range_x(k, seed, group_spread):
    """bf16 bits of x [1, k] whose 64-column groups each sit in a random binade within
    2^+-group_spread and whose values spread over 2^-40..2^0 of it, with zeros,
    bf16 subnormals and an all-zero group."""
    rng = np.random.default_rng(seed)
    g = k // 64
    base = rng.integers(-group_spread, group_spread + 1, size=g)
    spread = rng.integers(-40, 1, size=(g, 64))
    mant = rng.uniform(1.0, 2.0, size=(g, 64)) * rng.choice([-1.0, 1.0], size=(g, 64))
    x = (mant * np.exp2((base[:, None] + spread).astype(np.float64))).astype(np.float32)
    x[rng.random((g, 64)) < 0.05] = 0.0
    x[0, :8] = np.float32(1e-39) * np.arange(1, 9)  # bf16 subnormals
    x[2 % g] = 0.0                                   # an all-zero group
    return A.f32_to_bf16_bits(x.reshape(1, k))


@pytest.mark.parametrize("n,k", [(64, 640), (15360, 3840)])
@pytest.mark.parametrize("group_spread", [0, 100])
def test_wide_dynamic_range(gpu_lib, n, k, group_spread):
    """Values far below their group's maximum are where the limb split rounds: the
    fp32 output must still sit within the accumulation bar of the exact sum.  With
    group_spread 0 every group's maximum is near 1 (the bar sees every group); with
    100 the groups' scales differ by up to 2^200 (the exponent handling)."""
    wq, s, b = random_triple(n, k, seed=77)
    x = _wide_range_x(k, seed=k, group_spread=group_spread)
    y_exact = C.qmm_f64(x, wq, s, b)
    assert np.isfinite(y_exact).all()
    lin = gpu_lib.QuantizedLinear(*dev_triple(wq, s, b))
    y_f = run(lin, x, True, 1, gpu_lib)
    assert assert_close(y_f, y_exact, "wide range f32") < ACC_REL
    lin.close()


def test_largest_finite_x(gpu_lib):
    """Entries near the largest finite bf16 (group exponent 254) among N(0, 1) values."""
    n, k = 64, 384
    wq, s, b = random_triple(n, k, seed=78)
    x = A.bf16_bits_to_f32(A.make_activations(1, k, seed=79)).copy()
    x[0, [3, 100, 200]] = np.float32([3.0e38, -2.5e38, 1.0e38])
    x = A.f32_to_bf16_bits(x)
    y_exact = C.qmm_f64(x, wq, s, b)
    lin = gpu_lib.QuantizedLinear(*dev_triple(wq, s, b))
    y_f = run(lin, x, True, 1, gpu_lib)
    fin = np.isfinite(y_exact) & (np.abs(y_exact) < 3.0e38)
    got = host_bits(y_f).astype(np.float64)
    rms = float(np.sqrt(np.mean(y_exact[fin] ** 2)))
    assert np.max(np.abs(got[fin] - y_exact[fin])) <= ACC_REL * rms
    lin.close()


def test_exact_when_x_is_representable(gpu_lib):
    """Small integer x is split without rounding and the int8 sums are exact, so the
    only rounding left is the fp32 scale step: the fp32 output is within a few fp32
    ulps of the float64 oracle (1e-6 * RMS)."""
    n, k = 48, 256
    rng = np.random.default_rng(5)
    wq, s, b = random_triple(n, k, seed=6)
    x = A.f32_to_bf16_bits(rng.integers(-8, 9, size=(1, k)).astype(np.float32))
    y_exact = C.qmm_f64(x, wq, s, b)
    lin = gpu_lib.QuantizedLinear(*dev_triple(wq, s, b))
    y_f = host_bits(run(lin, x, True, 1, gpu_lib))
    rms = float(np.sqrt(np.mean(y_exact ** 2)))
    assert np.max(np.abs(y_f.astype(np.float64) - y_exact)) <= 1e-6 * rms
    lin.close()


@pytest.mark.parametrize("value", [np.inf, -np.inf, np.nan])
def test_non_finite_x_reaches_y(gpu_lib, value):
    """inf or NaN in x gives non-finite outputs (the reference's sum of products would
    hold inf or NaN), never finite garbage."""
    n, k = 64, 384
    wq, s, b = random_triple(n, k, seed=9)
    x = A.make_activations(1, k, seed=10)
    x = A.f32_to_bf16_bits(np.where(np.arange(k) == 70, np.float32(value), A.bf16_bits_to_f32(x)).reshape(1, k))
    lin = gpu_lib.QuantizedLinear(*dev_triple(wq, s, b))
    y = host_bits(run(lin, x, True, 1, gpu_lib))
    assert not np.isfinite(y).any()
    lin.close()


@pytest.mark.parametrize("m", [1, 2, 4, 8])
@pytest.mark.parametrize("n,k", [(4096 + 8, 3840), (3840, 15360)])
def test_rows_of_tiny_values(gpu_lib, n, k, m):
    """Rows whose every value is tiny: normal values near 2^-115 (below the 2^-108 where
    the int8 kernels' split exponent is clamped), bf16 subnormals only (group exponent 0),
    and groups of each mixed within a row, fp32 output, each row against the oracle.
    The bf16 kernels meet the accumulation bar on every row.  The int8 kernels clamp the
    split exponent at 19, i.e. they round x to a multiple of 2^-127 in a group whose
    largest |x| lies below 2^-108 (a group of bf16 subnormals only reads as zeros), so
    their error is held to that rounding's bound, 2^-128 sum_k |W[n, k]| on top of the
    accumulation bar, and on the normal rows that is still below 2e-3 of the row's RMS."""
    wq, s, b = random_triple(n, k, seed=n + k + 11 * m)
    rng = np.random.default_rng(900 + m)
    lin = gpu_lib.QuantizedLinear(*dev_triple(wq, s, b))
    w_abs = np.abs(C.dequantize(wq, s, b).astype(np.float64)).sum(axis=1)
    scales = [2.0 ** -115, 2.0 ** -130]
    for case in ("normal", "subnormal", "mixed"):
        xf = rng.standard_normal((m, k))
        if case == "mixed":
            xf = xf * np.where((np.arange(k) // 64) % 2 == 0, scales[0], scales[1])
        else:
            xf = xf * scales[case == "subnormal"]
        x = A.f32_to_bf16_bits(xf.astype(np.float32))
        if case == "subnormal":
            assert ((x & 0x7F80) == 0).all() and (x & 0x7F).any()
        y_exact = C.qmm_f64(x, wq, s, b)
        for variant in (1, 2):
            y = host_bits(run(lin, x, True, variant, gpu_lib)).astype(np.float64)
            for r in range(m):
                rms = float(np.sqrt(np.mean(y_exact[r] ** 2)))
                what = f"{case} rows {n}x{k} m={m} kernel {variant} row {r}"
                err = np.abs(y[r] - y_exact[r])
                if variant == 2:
                    assert float(err.max()) < ACC_REL * rms, f"{what}: {err.max() / rms:.3e} x RMS"
                else:
                    bound = ACC_REL * rms + 2.0 ** -128 * w_abs
                    assert (err <= bound).all(), f"{what}: {float(np.max(err / bound)):.3f} x the bound"
                    if case != "subnormal":
                        assert float(err.max()) < F32_REL * rms, f"{what}: {err.max() / rms:.3e} x RMS"
    lin.close()


def test_deterministic_and_agrees_with_bf16_kernels(gpu_lib):
    """Repeated calls are bit-identical; the two kernel families agree within twice
    the accumulation bar (they sum in different orders)."""
    import torch

    n, k = 15360, 3840
    wq, s, b = A.make_weights(n, k, seed=12)
    x = A.make_activations(1, k, seed=13)
    lin = gpu_lib.QuantizedLinear(*dev_triple(wq, s, b))
    a = run(lin, x, True, 1, gpu_lib)
    for _ in range(3):
        assert torch.equal(a, run(lin, x, True, 1, gpu_lib))
    c = run(lin, x, True, 2, gpu_lib)
    rms = c.pow(2).mean().sqrt().item()
    assert (a - c).abs().max().item() <= 2 * ACC_REL * rms
    lin.close()


# ---- 2-8 rows (decode_limb_rows_kernel, pinned with gemma4_qmm_set_decode_kernel(1)) ----
# Rows pad to 2, 4 or 8; where the limbs of x and the slots do not fit a CU's LDS (down
# at more than 2 rows) the pinned family falls back to the bf16 kernels, so every case
# still holds the bars.

@pytest.mark.parametrize("m", [2, 3, 4, 5, 8])
@pytest.mark.parametrize("proj", sorted(PROJ) + ["qkv_proj"])
def test_rows_projections(gpu_lib, proj, m):
    if proj == "qkv_proj":
        parts = [A.make_weights(*PROJ[p], seed=4300 + i) for i, p in enumerate(("q_proj", "k_proj", "v_proj"))]
        wq, s, b = (np.concatenate([p[j] for p in parts]) for j in range(3))
        k = 3840
    else:
        n, k = PROJ[proj]
        wq, s, b = A.make_weights(n, k, seed=4400 + sorted(PROJ).index(proj))
    x = A.make_activations(m, k, seed=4500 + m, outliers=True)
    lin = gpu_lib.QuantizedLinear(*dev_triple(wq, s, b))
    y_exact = C.qmm_f64(x, wq, s, b)
    y_f = run(lin, x, True, 1, gpu_lib)
    assert assert_close(y_f, y_exact, f"{proj} m={m} f32") < ACC_REL
    y_b = run(lin, x, False, 1, gpu_lib)
    assert_rounded(y_b, y_exact, f"{proj} m={m} bf16")
    lin.close()


@pytest.mark.parametrize("m", [2, 3, 6, 7])
@pytest.mark.parametrize("n,k", [(40, 320), (1000, 192), (16, 64), (33, 640), (4096 + 8, 3840), (20000, 576),
                                 (70000 + 40, 384), (3840, 15360)])
def test_rows_launch_shapes(gpu_lib, n, k, m):
    wq, s, b = random_triple(n, k, seed=n + 5 * k + m)
    x = A.make_activations(m, k, seed=n + m, outliers=True)
    lin = gpu_lib.QuantizedLinear(*dev_triple(wq, s, b))
    y_exact = C.qmm_f64(x, wq, s, b)
    y_f = run(lin, x, True, 1, gpu_lib)
    assert assert_close(y_f, y_exact, f"{n}x{k} m={m} f32") < ACC_REL
    lin.close()


@pytest.mark.parametrize("m", [2, 4, 8])
def test_rows_wide_dynamic_range_and_non_finite(gpu_lib, m):
    """Rows whose groups span the bf16 exponent range (each row its own exponents), and
    a row holding inf: that row's outputs are non-finite, the others unaffected."""
    import torch

    n, k = 15360, 3840
    wq, s, b = random_triple(n, k, seed=80 + m)
    x = np.concatenate([_wide_range_x(k, seed=k + r, group_spread=100 * (r % 2)) for r in range(m)])
    y_exact = C.qmm_f64(x, wq, s, b)
    lin = gpu_lib.QuantizedLinear(*dev_triple(wq, s, b))
    y_f = run(lin, x, True, 1, gpu_lib)
    assert assert_close(y_f, y_exact, f"wide range m={m} f32") < ACC_REL
    xi = A.bf16_bits_to_f32(x).copy()
    xi[m - 1, 77] = np.inf
    y_i = host_bits(run(lin, A.f32_to_bf16_bits(xi), True, 1, gpu_lib))
    assert not np.isfinite(y_i[m - 1]).any() and np.isfinite(y_i[: m - 1]).all()
    lin.close()
    del torch


@pytest.mark.parametrize("m", [2, 4, 8])
def test_rows_gate_up_pair(gpu_lib, m):
    from test_gpu_geglu import _check, _exact_gu

    gate = A.make_weights(15360, 3840, seed=4600)
    up = A.make_weights(15360, 3840, seed=4601)
    x = A.make_activations(m, 3840, seed=4700 + m, outliers=True)
    pair = gpu_lib.QuantizedGeGLU(dev_triple(*gate), dev_triple(*up))
    import torch

    with gpu_lib.decode_kernel(1):
        h = pair.forward(dev_x(x))
        hf = pair.forward(dev_x(x), out_dtype=torch.float32)
    torch.cuda.synchronize()
    g_exact, u_exact = _exact_gu(x, gate, up)
    _check(h, g_exact, u_exact, f"pair m={m} bf16")
    _check(hf, g_exact, u_exact, f"pair m={m} f32")
    pair.close()


@pytest.mark.parametrize("m", [2, 4, 8])
def test_rows_lm_head_and_greedy(gpu_lib, m):
    """The lm_head at 2, 4 and 8 rows (every output against the oracle; at 4 and 8 rows
    the phased launch, one workgroup per CU) and its greedy head under the int8
    kernels."""
    import torch

    from test_gpu_greedy import _check_token, _oracle
    from test_gpu_parity import lm_head_triple

    wq, s, b = lm_head_triple()
    x = A.make_activations(m, 3840, seed=4800 + m)
    lin = gpu_lib.QuantizedLinear(*dev_triple(wq, s, b))
    y_exact = C.qmm_f64(x, wq, s, b)
    y_f = run(lin, x, True, 1, gpu_lib)
    assert assert_close(y_f, y_exact, f"lm_head m={m} f32") < ACC_REL
    with gpu_lib.decode_kernel(1):
        tok, val, logits = lin.forward_greedy(dev_x(x), softcap=30.0, return_logits=True)
    torch.cuda.synchronize()
    sc = A.softcap_ops(y_exact.astype(np.float32), 30.0, bf16=True)
    _check_token(tok.cpu().numpy(), sc, True)
    lg = host_bits(logits)
    assert np.array_equal(A.bf16_bits_to_f32(lg[np.arange(m), tok.cpu().numpy()]), val.cpu().numpy())
    lin.close()
    del _oracle
