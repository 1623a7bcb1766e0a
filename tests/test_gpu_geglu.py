"""GPU parity of the fused gate|up projection with the GeGLU epilogue
(gemma4_qgeglu_forward) against the oracle, through the C ABI.

The reference computes gate and up with quantized_linear, rounds each to the bf16
model dtype, then applies geglu op by op in bf16 (native_model.cc:934-949,
:378-386).  The oracle's h is geglu_ops on the correctly rounded exact products
(bf16 or fp32, per the output dtype).  Bars:
  * bf16 h: at most 3% of elements differ from h_ref at all, and each that does is
    what geglu_ops gives for gate and up each moved by one bf16 ulp (within one ulp
    of h), or is within 1.2*|up|*dG + |gate|*dU + 2 ulp(h_ref) of h_ref, with
    dG = 2e-4 * RMS(gate) and dU = 2e-4 * RMS(up): the GeGLU of gate and up values
    within the kernel's fp32 accumulation error (~1e-5 * RMS measured) of the exact
    ones.  A difference needs that error to carry gate or up across a bf16 rounding
    boundary (about 1% of elements at K = 640 with outliers).  A plain RMS bar does
    not fit: the bf16 op sequence turns one ulp of gate into several percent of
    RMS(h) where 1 + tanh cancels.  The device GeGLU itself equals geglu_ops bit for
    bit on bf16 inputs (tanh's last fp32 ulp aside);
  * fp32 h: max |h - h_ref| <= 2e-3 * RMS(h_ref);
  * the pair's dequantize is bit-exact for both halves;
  * against the unfused path at decode (two gemma4_qlinear_forward calls, then
    geglu_ops on their bf16 outputs) at most 0.5% of elements differ.
"""

import numpy as np
import pytest

from oracle import affine as A
from oracle import c_oracle as C
from test_gpu_parity import BF16_REL, F32_REL, dev_triple, dev_x, host_bits, random_triple

pytestmark = pytest.mark.gpu

MISMATCH_FRAC = 3e-2   # against the oracle
UNFUSED_FRAC = 5e-3    # against the unfused path (same accumulation: only tanh can differ)


def _pair(f, k, seed):
    return random_triple(f, k, seed), random_triple(f, k, seed + 1)


def _exact_gu(x, gate, up, rows=None):
    xs = x if rows is None else np.ascontiguousarray(x[rows])
    return C.qmm_f64(xs, *gate).astype(np.float32), C.qmm_f64(xs, *up).astype(np.float32)


def _check(h_dev, g, u, what):
    """h against geglu_ops(g, u) (g, u the correctly rounded exact products)."""
    import torch

    h = host_bits(h_dev)
    if h_dev.dtype != torch.bfloat16:
        ref = A.geglu_ops(g, u, bf16=False).astype(np.float64)
        rms = float(np.sqrt(np.mean(ref ** 2))) or 1.0
        worst = float(np.max(np.abs(h.astype(np.float64) - ref))) / rms
        assert worst <= F32_REL, f"{what}: worst error / RMS = {worst:.3e}"
        return
    ref_bits = A.f32_to_bf16_bits(A.geglu_ops(g, u, bf16=True))
    bad = np.nonzero(ref_bits != h)
    frac = bad[0].size / h.size
    assert frac <= MISMATCH_FRAC, f"{what}: {frac:.4%} of elements differ from the oracle"
    if bad[0].size == 0:
        return
    got = A.bf16_bits_to_f32(h[bad]).astype(np.float64)
    gb = A.f32_to_bf16_bits(g[bad]).astype(np.int32)
    ub = A.f32_to_bf16_bits(u[bad]).astype(np.int32)
    best = np.full(got.shape, np.inf)
    for dg in (-1, 0, 1):
        for du in (-1, 0, 1):
            cand = A.geglu_ops(A.bf16_bits_to_f32((gb + dg).astype(np.uint16)),
                               A.bf16_bits_to_f32((ub + du).astype(np.uint16)), bf16=True).astype(np.float64)
            best = np.minimum(best, np.abs(got - cand) / A.bf16_ulp(cand))
    ref = A.bf16_bits_to_f32(ref_bits[bad]).astype(np.float64)
    dg = 2e-4 * float(np.sqrt(np.mean(g.astype(np.float64) ** 2)))
    du = 2e-4 * float(np.sqrt(np.mean(u.astype(np.float64) ** 2)))
    slack = 1.2 * np.abs(u[bad]) * dg + np.abs(g[bad]) * du + 2 * A.bf16_ulp(ref)
    ok = (best <= 1.0) | (np.abs(got - ref) <= slack)
    assert np.all(ok), f"{what}: {int(np.sum(~ok))} differences beyond the accumulation error of gate/up"


@pytest.mark.parametrize("f,k,m", [(40, 192, 1), (40, 192, 3), (13, 64, 2), (300, 640, 17), (72, 128, 8),
                                   (13, 64, 33), (300, 640, 40), (136, 1088, 300)])
@pytest.mark.parametrize("f32", [False, True])
def test_geglu_small_shapes(gpu_lib, gemm_from_32, f, k, m, f32):
    import torch

    gate, up = _pair(f, k, 500 + f + k)
    x = A.make_activations(m, k, seed=m + k, outliers=True)
    pair = gpu_lib.QuantizedGeGLU(dev_triple(*gate), dev_triple(*up))
    h = pair.forward(dev_x(x), out_dtype=torch.float32 if f32 else torch.bfloat16)
    torch.cuda.synchronize()
    assert tuple(h.shape) == (m, f)
    _check(h, *_exact_gu(x, gate, up), f"F={f} K={k} M={m} f32={f32}")
    info = pair.info()
    assert info["out_features"] == f and info["flags"] == gpu_lib.GEGLU_PAIR
    pair.close()


@pytest.mark.parametrize("m", [1, 2, 4, 8])
def test_geglu_decode_gate_up(gpu_lib, m):
    """The Gemma 4 12B MLP front half at decode (gate and up 15360 x 3840)."""
    import torch

    gate, up = _pair(15360, 3840, 20260630 + 2004)
    x = A.make_activations(m, 3840, seed=9000 + m)
    pair = gpu_lib.QuantizedGeGLU(dev_triple(*gate), dev_triple(*up))
    xd = dev_x(x)
    h = pair.forward(xd)
    hf = pair.forward(xd, out_dtype=torch.float32)
    torch.cuda.synchronize()
    g_exact, u_exact = _exact_gu(x, gate, up)
    _check(h, g_exact, u_exact, f"decode M={m} bf16")
    _check(hf, g_exact, u_exact, f"decode M={m} f32")
    # the unfused path: two projections, then the GeGLU ops on their bf16 outputs
    lg = gpu_lib.QuantizedLinear(*dev_triple(*gate))
    lu = gpu_lib.QuantizedLinear(*dev_triple(*up))
    g, u = lg.forward(xd), lu.forward(xd)
    torch.cuda.synchronize()
    unfused = A.f32_to_bf16_bits(A.geglu_ops(A.bf16_bits_to_f32(host_bits(g)), A.bf16_bits_to_f32(host_bits(u)),
                                             bf16=True))
    frac = float(np.mean(unfused != host_bits(h)))
    assert frac <= UNFUSED_FRAC, f"{frac:.4%} differ from the unfused path"
    for obj in (pair, lg, lu):
        obj.close()


@pytest.mark.parametrize("m", [33, 64, 512, 2048])
def test_geglu_prefill_gate_up(gpu_lib, m):
    """Chunked prefill: the fused pair at M=512 and 2048 (and short prompts of 33 and 64
    rows, the 64-row tile), sampled rows against the oracle, then the chain into
    down_proj (the prefill MLP's GeGLU -> down)."""
    import torch

    gate, up = _pair(15360, 3840, 20260630 + 2004)
    down = random_triple(3840, 15360, 20260630 + 2006)
    x = A.make_activations(m, 3840, seed=m, outliers=True)
    pair = gpu_lib.QuantizedGeGLU(dev_triple(*gate), dev_triple(*up))
    xd = dev_x(x)
    h = pair.forward(xd)
    hf = pair.forward(xd, out_dtype=torch.float32)
    torch.cuda.synchronize()
    rows = np.sort(np.random.default_rng(m).choice(m, min(m, 12), replace=False))
    rt = torch.from_numpy(rows).cuda()
    g_exact, u_exact = _exact_gu(x, gate, up, rows)
    _check(h[rt], g_exact, u_exact, f"prefill M={m} bf16")
    _check(hf[rt], g_exact, u_exact, f"prefill M={m} f32")
    # down_proj consumes h directly (identical bf16 bytes on both sides)
    ld = gpu_lib.QuantizedLinear(*dev_triple(*down))
    d = ld.forward(h)
    torch.cuda.synchronize()
    hb = host_bits(h)
    d_exact = C.qmm_f64(np.ascontiguousarray(hb[rows]), *down)
    ok, worst = A.check_bf16_output(host_bits(d[rt]), d_exact, BF16_REL)
    assert ok, f"down after GeGLU M={m}: worst error / RMS = {worst:.3e}"
    pair.close()
    ld.close()


def test_geglu_pair_dequantize_bit_exact_and_handle_kinds(gpu_lib):
    import torch

    f, k = 37, 192
    gate, up = _pair(f, k, 77)
    pair = gpu_lib.QuantizedGeGLU(dev_triple(*gate), dev_triple(*up))
    w = pair.dequantize().cpu().numpy()
    assert w.shape == (2, f, k)
    assert np.array_equal(w[0].view(np.uint32), A.dequantize(*gate).view(np.uint32))
    assert np.array_equal(w[1].view(np.uint32), A.dequantize(*up).view(np.uint32))
    # host-array create gives the same pair
    pair_h = gpu_lib.QuantizedGeGLU(gate, up)
    assert np.array_equal(pair_h.dequantize().cpu().numpy().view(np.uint32), w.view(np.uint32))
    # a pair is not a projection and a projection is not a pair
    lin = gpu_lib.QuantizedLinear(*dev_triple(*gate))
    x = dev_x(A.make_activations(2, k, seed=1))
    y = torch.empty((2, f), dtype=torch.bfloat16, device="cuda")
    lib = gpu_lib.load_library()
    st = lib.gemma4_qlinear_forward(pair._handle, None, gpu_lib._dev_ptr(x), 2, gpu_lib._dev_ptr(y), 0)
    assert st == gpu_lib.Status.INVALID_ARGUMENT and "gate|up pair" in gpu_lib.last_error()
    st = lib.gemma4_qgeglu_forward(lin._handle, None, gpu_lib._dev_ptr(x), 2, gpu_lib._dev_ptr(y), 0)
    assert st == gpu_lib.Status.INVALID_ARGUMENT and "not a gate|up pair" in gpu_lib.last_error()
    assert lin.info()["flags"] == 0
    for obj in (pair, pair_h, lin):
        obj.close()
