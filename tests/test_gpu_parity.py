"""GPU parity: the gfx950 HIP path, called through the C ABI, against the CPU oracle.

Bars (written here, applied in every test below):
  * dequantize: bit-exact fp32 (w = s*q + b is unique in fp32);
  * fp32 output: max |y - y_exact| <= 2e-3 * RMS(y_exact);
  * bf16 output: max |y - y_exact| <= 1e-2 * RMS(y_exact) + ulp_bf16(y_exact)/2
    (the half ulp is the rounding any bf16 output makes);
  where y_exact is the oracle's float64 accumulation of exact products.
The kernel's own error is far below these bars (fp32 accumulation of exact
products), so the decode and prefill projection tests also assert the tighter
property the kernels have:
  * bf16 output: each output is the round-to-nearest-even of a value within
    ACC_REL * RMS(y_exact) of y_exact (A.check_bf16_rounding), and at least
    RNE_FRAC of the outputs equal RNE(y_exact) exactly (a truncating or otherwise
    wrong rounding would match about half);
  * where the correctly rounded outputs themselves meet the literal bar
    max |y - y_exact| <= 1e-2 * RMS (no half-ulp allowance), the kernel's do too
    (decode inputs without outliers: bf16 rounding alone can exceed the literal bar
    only when the largest output sits in a binade whose half ulp is > 1e-2 * RMS).
"""

import functools

import numpy as np
import pytest

from oracle import affine as A
from oracle import c_oracle as C

pytestmark = pytest.mark.gpu

BF16_REL = 1e-2
F32_REL = 2e-3
ACC_REL = 1e-4   # fp32 accumulation of exact products (measured up to ~7e-5 with outliers)
# outputs equal to the correctly rounded exact value: the rest are those within the
# accumulation error of a rounding boundary (measured 98.4-100%; with 1% outliers x20
# the group sums carry more of the error).  A wrong rounding mode gives about 50%.
RNE_FRAC = 0.95

# (N, K) of the reference's projections at the benchmark configurations
PROJ = {
    "q_proj": (4096, 3840),
    "k_proj": (2048, 3840),
    "v_proj": (2048, 3840),
    "o_proj": (3840, 4096),
    "gate_proj": (15360, 3840),
    "up_proj": (15360, 3840),
    "down_proj": (3840, 15360),
}


def dev_triple(wq, s, b):
    import torch

    return (torch.from_numpy(np.ascontiguousarray(wq).view(np.int32)).cuda(),
            torch.from_numpy(np.ascontiguousarray(s).view(np.int16)).view(torch.bfloat16).cuda(),
            torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16).cuda())


def dev_x(x_bits):
    import torch

    return torch.from_numpy(np.ascontiguousarray(x_bits).view(np.int16)).view(torch.bfloat16).cuda()


def host_bits(t):
    import torch

    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def random_triple(n, k, seed, std=0.02):
    rng = np.random.default_rng(seed)
    w = A.round_to_bf16((rng.standard_normal((n, k)) * std).astype(np.float32))
    return C.quantize(w)


def assert_close(y_dev, y_exact, what=""):
    import torch

    if y_dev.dtype == torch.bfloat16:
        ok, worst = A.check_bf16_output(host_bits(y_dev), y_exact, BF16_REL)
    else:
        ok, worst = A.check_f32_output(host_bits(y_dev), y_exact, F32_REL)
    assert ok, f"{what}: worst error / RMS = {worst:.3e}"
    return worst


def assert_rounded(y_dev, y_exact, what="", literal=False):
    """bf16 output: one rounding of a value within ACC_REL * RMS of the exact result,
    RNE(exact) on at least RNE_FRAC of the outputs; with `literal`, the literal bar
    max |err| <= 1e-2 * RMS wherever RNE(exact) itself meets it."""
    y = host_bits(y_dev)
    ok, worst, equal = A.check_bf16_rounding(y, y_exact, ACC_REL)
    assert ok, f"{what}: error beyond ulp/2 = {worst:.3e} x RMS"
    assert equal >= RNE_FRAC, f"{what}: only {equal:.4%} of outputs equal RNE(exact)"
    if literal:
        y_exact = np.asarray(y_exact, np.float64)
        rms = float(np.sqrt(np.mean(y_exact ** 2)))
        rne_err = float(np.max(np.abs(A.bf16_bits_to_f32(A.f64_to_bf16_bits(y_exact)) - y_exact)))
        err = float(np.max(np.abs(A.bf16_bits_to_f32(y).astype(np.float64) - y_exact)))
        if rne_err <= BF16_REL * rms:
            assert err <= BF16_REL * rms, f"{what}: literal bar: max |err| = {err / rms:.3e} x RMS"
    return equal


@functools.lru_cache(maxsize=1)
def lm_head_triple():
    """The lm_head weight triple (262144 x 3840, W ~ N(0, 0.02) quantized), built once
    per test process."""
    return A.make_weights(262144, 3840, seed=20260630 + 3000)


@pytest.mark.parametrize("n,k", [(16, 64), (48, 128), (40, 192), (33, 640), (4096, 3840)])
def test_dequantize_bit_exact(gpu_lib, n, k):
    wq, s, b = random_triple(n, k, seed=n * 7 + k)
    lin = gpu_lib.QuantizedLinear(*dev_triple(wq, s, b))
    got = lin.dequantize().cpu().numpy()
    want = C.dequantize(wq, s, b)
    assert got.shape == (n, k)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    lin.close()


def test_dequantize_host_create_edge_groups(gpu_lib):
    """Host-pointer create path, with negative scales, eps scales, zero groups and
    a group spanning every code."""
    k = 256
    w = np.zeros((20, k), np.float32)
    w[0] = np.arange(k) / 4.0
    w[1] = -np.arange(k) / 4.0
    w[2] = 0.5
    w[3, :64] = 1e-6 * np.arange(64)
    w[4] = np.where(np.arange(k) % 2 == 0, 3.0, -5.0)
    rng = np.random.default_rng(3)
    w[5:] = rng.standard_normal((15, k)) * 0.05
    wq, s, b = C.quantize(A.round_to_bf16(w))
    lin = gpu_lib.QuantizedLinear(wq, s, b)  # numpy -> gemma4_qlinear_create
    got = lin.dequantize().cpu().numpy()
    assert np.array_equal(got.view(np.uint32), C.dequantize(wq, s, b).view(np.uint32))


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 12, 16, 17, 40])
@pytest.mark.parametrize("f32", [False, True])
def test_forward_small_shapes(gpu_lib, gemm_from_32, m, f32):
    import torch

    n, k = 40, 384  # N not a multiple of 16, 6 groups
    wq, s, b = random_triple(n, k, seed=100 + m)
    x = A.make_activations(m, k, seed=200 + m, outliers=True)
    lin = gpu_lib.QuantizedLinear(*dev_triple(wq, s, b))
    y = lin.forward(dev_x(x), out_dtype=torch.float32 if f32 else torch.bfloat16)
    torch.cuda.synchronize()
    assert tuple(y.shape) == (m, n)
    assert_close(y, C.qmm_f64(x, wq, s, b), f"m={m}")


def test_forward_odd_group_count_and_3d_input(gpu_lib):
    import torch

    n, k = 64, 320  # 5 groups: the last group pair is half padding
    wq, s, b = random_triple(n, k, seed=7)
    x = A.make_activations(6, k, seed=8)
    lin = gpu_lib.QuantizedLinear(*dev_triple(wq, s, b))
    y = lin.forward(dev_x(x).reshape(1, 6, k), out_dtype=torch.float32)
    assert tuple(y.shape) == (1, 6, n)
    assert_close(y.reshape(6, n), C.qmm_f64(x, wq, s, b))


@pytest.mark.parametrize("proj", sorted(PROJ))
@pytest.mark.parametrize("m", [1, 2, 4, 8])
def test_forward_decode_projections(gpu_lib, proj, m):
    """Config shapes at full size: decoder projections at decode batch M."""
    import torch

    n, k = PROJ[proj]
    wq, s, b = A.make_weights(n, k, seed=20260630 + 1000 + sorted(PROJ).index(proj))
    x = A.make_activations(m, k, seed=777 + m)
    lin = gpu_lib.QuantizedLinear(*dev_triple(wq, s, b))
    xd = dev_x(x)
    y_bf = lin.forward(xd)
    y_f32 = lin.forward(xd, out_dtype=torch.float32)
    torch.cuda.synchronize()
    y_exact = C.qmm_f64(x, wq, s, b)
    assert_close(y_bf, y_exact, f"{proj} m={m} bf16")
    assert_rounded(y_bf, y_exact, f"{proj} m={m} bf16", literal=True)
    worst = assert_close(y_f32, y_exact, f"{proj} m={m} f32")
    assert worst < ACC_REL  # exact products + fp32 accumulation: far inside the bar
    lin.close()


@pytest.mark.parametrize("m", [1, 2, 8, 16])
def test_lm_head_decode_and_verify(gpu_lib, m):
    """The lm_head (262144 x 3840) at decode M = 1 and at the verify blocks M = 8 and
    16 (native_model.cc:1782-1795, called at :2006 with the block of
    gemma4_mlx.h:77-79), bf16 and fp32 logits against the oracle on every output.
    At M = 8 and 16 one workgroup fits a CU and each walks 64 row blocks: the
    decode kernel with four chunks per wave in flight."""
    import torch

    wq, s, b = lm_head_triple()
    x = A.make_activations(m, 3840, seed=31 + m)
    lin = gpu_lib.QuantizedLinear(*dev_triple(wq, s, b))
    xd = dev_x(x)
    y_bf = lin.forward(xd)
    y_f = lin.forward(xd, out_dtype=torch.float32)
    torch.cuda.synchronize()
    y_exact = C.qmm_f64(x, wq, s, b)
    assert_close(y_bf, y_exact, f"lm_head m={m} bf16")
    assert_rounded(y_bf, y_exact, f"lm_head m={m} bf16", literal=True)
    assert assert_close(y_f, y_exact, f"lm_head m={m} f32") < ACC_REL
    lin.close()


@pytest.mark.parametrize("m,n", [(9, 70000), (16, 70000), (14, 76800), (8, 76800 + 40)])
def test_forward_decode_four_chunks_in_flight(gpu_lib, m, n):
    """Mid-size N at K = 3840 and M = 8-16: LDS admits one workgroup per CU and each
    walks 17-19 row blocks, so the decode kernel keeps four chunks in flight and its
    tail runs 1, 2 or 3 chunks after the last full round of four (4375 blocks over
    244 workgroups of 18 or 17; 4800 over 253 of 19 or 18; a ragged last block)."""
    import torch

    k = 3840
    wq, s, b = random_triple(n, k, seed=5150 + m)
    x = A.make_activations(m, k, seed=5151 + m, outliers=True)
    lin = gpu_lib.QuantizedLinear(*dev_triple(wq, s, b))
    y = lin.forward(dev_x(x), out_dtype=torch.float32)
    y_bf = lin.forward(dev_x(x))
    torch.cuda.synchronize()
    y_exact = C.qmm_f64(x, wq, s, b)
    assert assert_close(y, y_exact, f"m={m} n={n} f32") < ACC_REL
    assert_rounded(y_bf, y_exact, f"m={m} n={n} bf16")
    lin.close()


def test_host_and_device_create_agree_and_properties(gpu_lib):
    """Same bytes through both create paths give identical outputs; linearity in x
    and zero input hold at the gate_proj size."""
    import torch

    n, k = PROJ["gate_proj"]
    wq, s, b = A.make_weights(n, k, seed=5)
    lin_h = gpu_lib.QuantizedLinear(wq, s, b)
    lin_d = gpu_lib.QuantizedLinear(*dev_triple(wq, s, b))
    x1 = dev_x(A.make_activations(4, k, seed=1))
    x2 = dev_x(A.make_activations(4, k, seed=2))
    ya = lin_h.forward(x1, out_dtype=torch.float32)
    yb = lin_d.forward(x1, out_dtype=torch.float32)
    assert torch.equal(ya, yb)
    # linearity: y(x1) + y(x2) vs y(x1 + x2) (x1 + x2 rounded to bf16 -> compare to oracle)
    x12 = (x1.float() + x2.float()).bfloat16()
    y12 = lin_d.forward(x12, out_dtype=torch.float32)
    y2 = lin_d.forward(x2, out_dtype=torch.float32)
    resid = (y12 - ya - y2).abs().max().item()
    rms = y12.pow(2).mean().sqrt().item()
    assert resid <= 2e-2 * rms  # bf16 rounding of x1 + x2 dominates
    z = lin_d.forward(torch.zeros_like(x1), out_dtype=torch.float32)
    assert torch.count_nonzero(z).item() == 0
    # deterministic: same call twice gives identical bits
    assert torch.equal(lin_d.forward(x1), lin_d.forward(x1))


def test_forward_rejects_misaligned_x(gpu_lib):
    import torch

    wq, s, b = random_triple(16, 128, seed=9)
    lin = gpu_lib.QuantizedLinear(*dev_triple(wq, s, b))
    buf = torch.zeros(2 * 128 + 8, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(gpu_lib.Gemma4Error) as e:
        lin.forward_raw(buf.data_ptr() + 2, 1, buf.data_ptr())
    assert e.value.status == gpu_lib.Status.INVALID_ARGUMENT and "aligned" in e.value.message


@pytest.mark.parametrize("m", [0, 1, 4, 33])
@pytest.mark.parametrize("n,k", [(1, 64), (15, 192), (17, 64)])
def test_forward_empty_rows_and_partial_row_blocks(gpu_lib, gemm_from_32, m, n, k):
    """M = 0 returns an empty result without a launch; N of 1, 15 and 17 leave a row
    block mostly or partly empty, on the decode (M = 1, 4) and GEMM (M = 33) paths."""
    import torch

    wq, s, b = random_triple(n, k, seed=71 + n + k)
    x = A.make_activations(m, k, seed=72 + m, outliers=True)
    lin = gpu_lib.QuantizedLinear(*dev_triple(wq, s, b))
    for f32 in (False, True):
        y = lin.forward(dev_x(x), out_dtype=torch.float32 if f32 else torch.bfloat16)
        torch.cuda.synchronize()
        assert tuple(y.shape) == (m, n)
        if m:
            assert_close(y, C.qmm_f64(x, wq, s, b), f"m={m} n={n} k={k} f32={f32}")
    lin.close()


@pytest.mark.parametrize("m", [1, 3, 4])
@pytest.mark.parametrize("n,k", [(131072 + 48, 128), (32768 + 40, 256)])
def test_forward_many_row_blocks_per_workgroup(gpu_lib, m, n, k):
    """Tall, narrow weights: more 16-row blocks than resident waves, so the persistent
    decode kernels walk several row blocks per workgroup (8195 blocks: the streaming
    kernel) or per wave (2051 blocks at M = 1: the row-block-per-wave kernel), with a
    ragged last block."""
    import torch

    wq, s, b = random_triple(n, k, seed=41 + m)
    x = A.make_activations(m, k, seed=42 + m, outliers=True)
    lin = gpu_lib.QuantizedLinear(*dev_triple(wq, s, b))
    y = lin.forward(dev_x(x), out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert_close(y, C.qmm_f64(x, wq, s, b), f"tall m={m}")


@pytest.mark.parametrize("f32", [False, True])
@pytest.mark.parametrize("m,n,k", [(3, 48, 15360), (4, 40, 15360), (5, 48, 15360), (8, 3840, 15360),
                                   (13, 40, 14976), (16, 3840, 15360),
                                   (16, 48, 4096), (16, 33 * 16, 14976)])
def test_forward_decode_x_beyond_lds(gpu_lib, m, n, k, f32):
    """Decode launches that read x from global memory: x too long for LDS (down_proj's
    K = 15360 from M = 5, o_proj's 4096 at M = 16, 117 pairs) and down_proj-like K at
    M = 3-4 (one pass of 8 pairs per wave); ragged row counts and a last slab of fewer
    than 16 rows."""
    import torch

    wq, s, b = random_triple(n, k, seed=61 + m + n)
    x = A.make_activations(m, k, seed=62 + m, outliers=True)
    lin = gpu_lib.QuantizedLinear(*dev_triple(wq, s, b))
    y = lin.forward(dev_x(x), out_dtype=torch.float32 if f32 else torch.bfloat16)
    y2 = lin.forward(dev_x(x), out_dtype=torch.float32 if f32 else torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)  # deterministic
    assert_close(y, C.qmm_f64(x, wq, s, b), f"x beyond LDS m={m} n={n} k={k}")
    lin.close()


# ---------------------------------------------------------------- prefill (GEMM path)

# K = 64, 576, 1088: one group, and a last octet of one group (9, 17 groups)
@pytest.mark.parametrize("n,k,m", [(40, 384, 33), (256, 640, 300), (130, 320, 257), (512, 3840, 64), (16, 64, 33),
                                   (48, 576, 40), (130, 1088, 300)])
@pytest.mark.parametrize("f32", [False, True])
def test_gemm_small_shapes(gpu_lib, gemm_from_32, n, k, m, f32):
    """GEMM path (M >= 32): ragged M and N, odd group counts, outlier activations."""
    import torch

    wq, s, b = random_triple(n, k, seed=n + k + m)
    x = A.make_activations(m, k, seed=m, outliers=True)
    lin = gpu_lib.QuantizedLinear(*dev_triple(wq, s, b))
    y = lin.forward(dev_x(x), out_dtype=torch.float32 if f32 else torch.bfloat16)
    torch.cuda.synchronize()
    worst = assert_close(y, C.qmm_f64(x, wq, s, b), f"gemm n={n} k={k} m={m}")
    if f32:
        # exact products and fp32 accumulation; the group sums X_g enter the bias term
        # as two bf16 parts (about 16 bits), which outlier rows make the largest term
        assert worst < 5e-4


@pytest.mark.parametrize("proj", sorted(PROJ))
@pytest.mark.parametrize("m", [512, 2048])
def test_gemm_prefill_projections(gpu_lib, proj, m):
    """The seven projections at the prefill chunks M = 512 and 2048, activations
    with 1% outliers x20."""
    import torch

    n, k = PROJ[proj]
    triple = A.make_weights(n, k, seed=20260630 + 2000 + sorted(PROJ).index(proj))
    x = A.make_activations(m, k, seed=m, outliers=True)
    lin = gpu_lib.QuantizedLinear(*dev_triple(*triple))
    xd = dev_x(x)
    y_bf = lin.forward(xd)
    y_f = lin.forward(xd, out_dtype=torch.float32)
    torch.cuda.synchronize()
    # full-size prefill is too large for the float64 CPU oracle in full: sample rows
    rows = np.random.default_rng(1).choice(m, 24, replace=False)
    rows.sort()
    y_exact = C.qmm_f64(np.ascontiguousarray(x[rows]), *triple)
    rt = torch.from_numpy(rows).cuda()
    assert_close(y_bf[rt], y_exact, f"{proj} m={m} bf16")
    assert_rounded(y_bf[rt], y_exact, f"{proj} m={m} bf16")
    worst = assert_close(y_f[rt], y_exact, f"{proj} m={m} f32")
    assert worst < 5e-4
    # every row block of the output is written (no stale tiles): compare the f32 and
    # bf16 results everywhere, which agree to bf16 rounding
    diff = (y_bf.float() - y_f).abs()
    assert torch.all(diff <= y_f.abs() * 2**-8 + 1e-6).item()


# the real Gemma 4 12B's full-attention layers (native_model.cc:795-798, :820-827): q
# 3840 -> 8192, k 3840 -> 512 (k doubles as v, no v_proj), o 8192 -> 3840
FULL_ATTENTION = {"full_q_proj": (8192, 3840), "full_k_proj": (512, 3840), "full_o_proj": (3840, 8192)}


@pytest.mark.parametrize("proj", sorted(FULL_ATTENTION))
@pytest.mark.parametrize("m", [1, 3, 4, 8, 256, 2048])
def test_full_attention_projections(gpu_lib, proj, m):
    """The full-attention shapes at decode (every output against the oracle) and at the
    long-context chunk M = 256 and the prefill chunk M = 2048 (sampled rows)."""
    import torch

    n, k = FULL_ATTENTION[proj]
    triple = A.make_weights(n, k, seed=20260630 + 6000 + sorted(FULL_ATTENTION).index(proj))
    x = A.make_activations(m, k, seed=6100 + m, outliers=m > 8)
    lin = gpu_lib.QuantizedLinear(*dev_triple(*triple))
    xd = dev_x(x)
    y_bf = lin.forward(xd)
    y_f = lin.forward(xd, out_dtype=torch.float32)
    torch.cuda.synchronize()
    rows = np.arange(m) if m <= 8 else np.sort(np.random.default_rng(m).choice(m, 24, replace=False))
    rt = torch.from_numpy(rows).cuda()
    y_exact = C.qmm_f64(np.ascontiguousarray(x[rows]), *triple)
    assert_close(y_bf[rt], y_exact, f"{proj} m={m} bf16")
    assert_rounded(y_bf[rt], y_exact, f"{proj} m={m} bf16", literal=m <= 8)
    assert assert_close(y_f[rt], y_exact, f"{proj} m={m} f32") < (ACC_REL if m <= 8 else 5e-4)
    lin.close()


# (projection, rows) the automatic path choice runs on the decode kernels past 32 rows
# (16-row slabs x N x K <= 5.5e7): 16-row slabs with one workgroup per row block and
# slab, the ragged last slab included; 9 and 15 rows are single slabs of the same
# kernel, and so are 10 rows of the 8192-row full-attention q (two row blocks per
# workgroup).
SLAB_CASES = [("q_proj", 9), ("q_proj", 15), ("q_proj", 41), ("q_proj", 48), ("k_proj", 33), ("k_proj", 93),
              ("o_proj", 45), ("full_q_proj", 10), ("full_q_proj", 31), ("full_k_proj", 256), ("full_k_proj", 420)]


@pytest.mark.parametrize("proj,m", SLAB_CASES)
def test_forward_decode_slabs_past_32_rows(gpu_lib, proj, m):
    """Sampled rows of every slab against the oracle, bf16 and fp32 outputs, with the
    tighter accumulation bars of the decode path; the same rows through the GEMM
    (pinned from 32 rows on) meet the same bars."""
    import torch

    shapes = {**PROJ, **FULL_ATTENTION}
    n, k = shapes[proj]
    seed = (20260630 + 1000 + sorted(PROJ).index(proj) if proj in PROJ
            else 20260630 + 6000 + sorted(FULL_ATTENTION).index(proj))
    triple = A.make_weights(n, k, seed=seed)
    x = A.make_activations(m, k, seed=6300 + m, outliers=True)
    lin = gpu_lib.QuantizedLinear(*dev_triple(*triple))
    xd = dev_x(x)
    y_bf = lin.forward(xd)
    y_f = lin.forward(xd, out_dtype=torch.float32)
    with gpu_lib.gemm_min_rows(32):
        y_gemm = lin.forward(xd, out_dtype=torch.float32)
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([np.linspace(0, m - 1, 24).astype(np.int64), [m - 1]]))
    rt = torch.from_numpy(rows).cuda()
    y_exact = C.qmm_f64(np.ascontiguousarray(x[rows]), *triple)
    assert_close(y_bf[rt], y_exact, f"{proj} m={m} bf16")
    assert_rounded(y_bf[rt], y_exact, f"{proj} m={m} bf16")
    assert assert_close(y_f[rt], y_exact, f"{proj} m={m} f32") < ACC_REL
    assert assert_close(y_gemm[rt], y_exact, f"{proj} m={m} f32 (GEMM)") < 5e-4
    lin.close()


@pytest.mark.parametrize("m", [33, 64])
def test_gemm_short_prompt_mlp(gpu_lib, gemm_from_32, m):
    """Short prompts and prefill tails on the MLP shapes (the 64-row tile): gate and
    down on sampled rows against the oracle (the gate|up pair: test_gpu_geglu.py)."""
    import torch

    rows = np.unique(np.concatenate([np.linspace(0, m - 1, 8).astype(np.int64), [m - 1]]))
    rt = torch.from_numpy(rows).cuda()
    for proj in ("gate_proj", "down_proj"):
        n, k = PROJ[proj]
        tri = A.make_weights(n, k, seed=20260630 + 1000 + sorted(PROJ).index(proj))
        x = A.make_activations(m, k, seed=6500 + m, outliers=True)
        lin = gpu_lib.QuantizedLinear(*dev_triple(*tri))
        y = lin.forward(dev_x(x))
        yf = lin.forward(dev_x(x), out_dtype=torch.float32)
        torch.cuda.synchronize()
        lin.close()
        want = C.qmm_f64(np.ascontiguousarray(x[rows]), *tri)
        assert_close(y[rt], want, f"{proj} m={m} bf16")
        assert assert_close(yf[rt], want, f"{proj} m={m} f32") < 5e-4


@pytest.mark.parametrize("proj,m", [("q_proj", 80), ("o_proj", 113), ("q_proj", 128), ("full_q_proj", 128),
                                    ("full_o_proj", 128)])
def test_gemm_64_row_tile_two_row_tiles(gpu_lib, gemm_from_32, proj, m):
    """The 64-row tile past 64 rows (two row tiles, the second ragged at 80 and 113):
    the attention projections at 65-128 rows; sampled rows of both tiles against the
    oracle."""
    import torch

    shapes = {**PROJ, **FULL_ATTENTION}
    n, k = shapes[proj]
    seed = (20260630 + 1000 + sorted(PROJ).index(proj) if proj in PROJ
            else 20260630 + 6000 + sorted(FULL_ATTENTION).index(proj))
    tri = A.make_weights(n, k, seed=seed)
    x = A.make_activations(m, k, seed=6600 + m, outliers=True)
    lin = gpu_lib.QuantizedLinear(*dev_triple(*tri))
    y = lin.forward(dev_x(x))
    yf = lin.forward(dev_x(x), out_dtype=torch.float32)
    torch.cuda.synchronize()
    lin.close()
    rows = np.unique(np.concatenate([np.linspace(0, m - 1, 16).astype(np.int64), [63, 64, m - 1]]))
    rt = torch.from_numpy(rows).cuda()
    want = C.qmm_f64(np.ascontiguousarray(x[rows]), *tri)
    assert_close(y[rt], want, f"{proj} m={m} bf16")
    assert assert_close(yf[rt], want, f"{proj} m={m} f32") < 5e-4


# (N, M) whose plans (64-row tile, 8 splits; 64-row, 4 splits; 128-row, 4 splits;
# 256-row, 3 splits) end a K split of two or more octets on the last octet
@pytest.mark.parametrize("n,m", [(1000, 40), (1000, 700), (1000, 1500), (3000, 1500)])
def test_gemm_last_octet_of_one_group(gpu_lib, gemm_from_32, n, m):
    """K of 57 groups: seven whole octets and a last octet of one group.  Where a K
    split ends on it with two or more octets, that octet's one step also applies the
    previous octet's bias term, so the 64- and 128-row tiles write its group sums of x
    after the loop and the 256-row tile loads them there from the pre-pass; with eight
    splits the octet is a split of its own.  Sampled rows against the oracle, bf16 and
    fp32."""
    import torch

    k = 57 * 64
    tri = random_triple(n, k, 5700 + n)
    x = A.make_activations(m, k, seed=5800 + m, outliers=True)
    lin = gpu_lib.QuantizedLinear(*dev_triple(*tri))
    y = lin.forward(dev_x(x))
    yf = lin.forward(dev_x(x), out_dtype=torch.float32)
    torch.cuda.synchronize()
    lin.close()
    rows = np.unique(np.concatenate([np.linspace(0, m - 1, 24).astype(np.int64), [m - 1]]))
    rt = torch.from_numpy(rows).cuda()
    want = C.qmm_f64(np.ascontiguousarray(x[rows]), *tri)
    assert_close(y[rt], want, f"N={n} K={k} M={m} bf16")
    assert assert_close(yf[rt], want, f"N={n} K={k} M={m} f32") < 5e-4


def test_gemm_prefill_chain_m2048_geglu(gpu_lib):
    """Chunked-prefill chain at M=2048: gate and up, GeGLU on the host (identical bf16
    bytes to both sides), then down_proj; sampled rows against the oracle."""
    import torch

    m = 2048
    tri = {p: A.make_weights(*PROJ[p], seed=20260630 + 2000 + sorted(PROJ).index(p)) for p in
           ("gate_proj", "up_proj", "down_proj")}
    x = A.make_activations(m, 3840, seed=2048, outliers=True)
    lins = {p: gpu_lib.QuantizedLinear(*dev_triple(*t)) for p, t in tri.items()}
    xd = dev_x(x)
    g = lins["gate_proj"].forward(xd)
    u = lins["up_proj"].forward(xd)
    torch.cuda.synchronize()
    rows = np.sort(np.random.default_rng(2).choice(m, 16, replace=False))
    rt = torch.from_numpy(rows).cuda()
    assert_close(g[rt], C.qmm_f64(np.ascontiguousarray(x[rows]), *tri["gate_proj"]), "gate m=2048")
    assert_close(u[rt], C.qmm_f64(np.ascontiguousarray(x[rows]), *tri["up_proj"]), "up m=2048")
    h = A.gelu_tanh_times(host_bits(g), host_bits(u))
    d = lins["down_proj"].forward(dev_x(h))
    torch.cuda.synchronize()
    assert_close(d[rt], C.qmm_f64(np.ascontiguousarray(h[rows]), *tri["down_proj"]), "down m=2048")


@pytest.mark.parametrize("f32", [False, True])
def test_gemm_split_k_deterministic_and_unaligned_y(gpu_lib, f32):
    """k_proj at M=512 runs with K split over workgroups (fp32 partial planes summed in
    a fixed order): repeated calls give identical bits, and an output that is only
    element-aligned (not 16-byte aligned) gets the same values."""
    import torch

    n, k = PROJ["k_proj"]
    m = 512
    wq, s, b = A.make_weights(n, k, seed=21)
    x_bits = A.make_activations(m, k, seed=22, outliers=True)
    lin = gpu_lib.QuantizedLinear(*dev_triple(wq, s, b))
    x = dev_x(x_bits)
    dt = torch.float32 if f32 else torch.bfloat16
    y1 = lin.forward(x, out_dtype=dt)
    y2 = lin.forward(x, out_dtype=dt)
    assert torch.equal(y1, y2)
    buf = torch.zeros(m * n + 8, dtype=dt, device="cuda")
    lin.forward_raw(x.data_ptr(), m, buf.data_ptr() + buf.element_size(), f32=f32,
                    stream_ptr=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    y3 = buf[1:1 + m * n].view(m, n)
    assert torch.equal(y1, y3)
    assert buf[0].item() == 0 and torch.count_nonzero(buf[1 + m * n:]).item() == 0
    rows = np.arange(0, m, 37)
    assert_close(y1[rows], C.qmm_f64(x_bits[rows], wq, s, b), "k_proj m=512 split-K")
    lin.close()
