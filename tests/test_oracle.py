"""Pins for the CPU oracle (oracle/affine.py, oracle/q4_oracle.c).

The reference holds no quantized-matmul vectors (its only parity checks are
whole-model ones that need the absent 6.7 GB artifact), so each oracle function
is pinned here by hand-derived known answers, exact rational arithmetic, brute
force on tiny inputs, textbook special cases and invariants.  Each check is
chosen so that a plausible slip (wrong nibble order, dropped bias, flipped scale
sign, transposed operand, wrong rounding) fails at least one of them.
"""

from fractions import Fraction

import numpy as np
import pytest

from oracle import affine as A
from oracle import c_oracle as C


# ---------------------------------------------------------------- bf16 helpers

def test_bf16_round_to_nearest_even_known_answers():
    vals = np.array([1.0, 1.0 + 2**-8, 1.0 + 3 * 2**-8, 1.0 + 2**-9, -2.5, 0.0, 65504.0], np.float32)
    # 1+2^-8 is a tie -> even (1.0); 1+3*2^-8 is a tie -> even (1+2^-6)
    want = np.array([0x3F80, 0x3F80, 0x3F82, 0x3F80, 0xC020, 0x0000, 0x4780], np.uint16)
    assert np.array_equal(A.f32_to_bf16_bits(vals), want)
    lib = C.load()
    import ctypes
    lib.oracle_f32_to_bf16.argtypes = [ctypes.c_float]
    lib.oracle_f32_to_bf16.restype = ctypes.c_uint16
    assert [lib.oracle_f32_to_bf16(float(v)) for v in vals] == want.tolist()
    assert np.array_equal(A.bf16_bits_to_f32(want)[:2], np.array([1.0, 1.0], np.float32))


def test_bf16_matches_torch_rounding():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(7)
    v = (rng.standard_normal(100000) * np.exp2(rng.integers(-30, 30, 100000))).astype(np.float32)
    ours = A.f32_to_bf16_bits(v)
    theirs = torch.from_numpy(v).bfloat16().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)


# ---------------------------------------------------------------- packing

def test_pack_hand_vector_lsb_first():
    q = np.array([[0, 1, 2, 3, 4, 5, 6, 7, 15, 14, 13, 12, 11, 10, 9, 8]], np.uint8)
    wq = A.pack(q)
    assert wq.tolist() == [[0x76543210, 0x89ABCDEF]]
    assert np.array_equal(A.unpack(wq), q)


def test_pack_unpack_identity_and_bit_positions():
    rng = np.random.default_rng(0)
    for bits in (2, 4, 8):
        q = rng.integers(0, 1 << bits, size=(5, 128), dtype=np.uint32)
        wq = A.pack(q, bits)
        assert wq.shape == (5, 128 * bits // 32)
        assert np.array_equal(A.unpack(wq, bits), q.astype(np.uint8))
        per = 32 // bits
        for r in range(5):
            for c in range(0, 128, 7):  # brute-force bit positions
                word = int(wq[r, c // per])
                assert (word >> (bits * (c % per))) & ((1 << bits) - 1) == q[r, c]


# ---------------------------------------------------------------- dequantize

def test_dequantize_exact_over_all_q_and_sampled_scales():
    """s*q+b evaluated exactly in rationals, rounded once to fp32, equals the oracle."""
    rng = np.random.default_rng(1)
    n = 256
    s = A.f32_to_bf16_bits((rng.standard_normal(n) * 0.01).astype(np.float32))
    s[:8] = A.f32_to_bf16_bits(np.array([-1.05, 1.05, 1e-7, -1e-7, 3.0e-3, -7.5, 0.0, 2.0**-20], np.float32))
    b = A.f32_to_bf16_bits((rng.standard_normal(n) * 0.05).astype(np.float32))
    q = np.tile(np.arange(16, dtype=np.uint32), (n, 4))  # every q in every row, K = 64
    wq = A.pack(q)
    deq = A.dequantize(wq, s[:, None], b[:, None])
    deq_c = C.dequantize(wq, s[:, None], b[:, None])
    assert np.array_equal(deq.view(np.uint32), deq_c.view(np.uint32))
    sf = A.bf16_bits_to_f32(s)
    bf = A.bf16_bits_to_f32(b)
    for r in range(n):
        for c in range(16):
            exact = Fraction(float(sf[r])) * c + Fraction(float(bf[r]))
            want = np.float32(float(exact))  # one rounding of the exact value
            # float(Fraction) is correctly rounded to double; double->float32 could
            # double-round only at exact fp32 ties, which the assertion would expose.
            assert deq[r, c] == want, (r, c)


# ---------------------------------------------------------------- quantize

def _frac_quantize_group(vals):
    """Independent restatement with exact rationals where MLX uses fp32; returns
    (q list, scale fp32, bias fp32).  fp32 divisions are reproduced by rounding the
    exact quotient to fp32, which is what IEEE division does."""
    f32 = np.float32
    w = [f32(v) for v in vals]
    w_max, w_min = max(w), min(w)
    mask = abs(w_min) > abs(w_max)
    scale = max(f32(float(Fraction(float(w_max - w_min)) / 15)), f32(1e-7))
    scale = scale if mask else -scale
    edge = w_min if mask else w_max
    q0 = np.rint(f32(float(Fraction(float(edge)) / Fraction(float(scale)))))
    bias = f32(0)
    if q0 != 0:
        scale = f32(float(Fraction(float(edge)) / Fraction(float(q0))))
        bias = edge
    q = []
    for v in w:
        t = f32(float(Fraction(float(f32(v - bias))) / Fraction(float(scale))))
        q.append(int(min(max(np.rint(t), 0), 15)))
    return q, f32(scale), f32(bias)


KNOWN_GROUPS = {
    "ramp_up": [j / 4 for j in range(64)],          # |max| wins -> negative scale, bias = max
    "ramp_down": [-j / 4 for j in range(64)],       # |min| wins -> positive scale, bias = min
    "constant": [0.5] * 64,                          # eps scale, exact reconstruction
    "zeros": [0.0] * 64,                             # q0 == 0 -> bias 0
    "straddle": [(j - 16) / 8 for j in range(64)],  # refined scale edge/q0 with q0 = -11
}


@pytest.mark.parametrize("name", sorted(KNOWN_GROUPS))
def test_quantize_known_answer_groups(name):
    vals = KNOWN_GROUPS[name]
    w = np.array([vals], np.float32)
    wq, s, b = A.quantize(w)
    q, scale, bias = _frac_quantize_group(vals)
    assert A.unpack(wq)[0].tolist() == q
    assert s[0, 0] == A.f32_to_bf16_bits(np.array([scale]))[0]
    assert b[0, 0] == A.f32_to_bf16_bits(np.array([bias]))[0]
    cq = C.quantize(w)
    assert all(np.array_equal(x, y) for x, y in zip((wq, s, b), cq))


def test_quantize_hand_values():
    # ramp_up: scale = -(15.75/15) = -1.05 -> bf16 0xBF86 (-1.046875), bias 15.75 = 0x417C,
    # q_j = rint((63 - j) / 4.2): j=0 -> 15, j=21 -> 10, j=63 -> 0.
    wq, s, b = A.quantize(np.array([KNOWN_GROUPS["ramp_up"]], np.float32))
    q = A.unpack(wq)[0]
    assert (s[0, 0], b[0, 0]) == (0xBF86, 0x417C)
    assert (q[0], q[21], q[63]) == (15, 10, 0)
    wq, s, b = A.quantize(np.array([KNOWN_GROUPS["ramp_down"]], np.float32))
    assert (s[0, 0], b[0, 0]) == (0x3F86, 0xC17C)
    # constant group: q == 0, bias == the constant, so dequantize is exact
    wq, s, b = A.quantize(np.array([KNOWN_GROUPS["constant"]], np.float32))
    assert A.unpack(wq).max() == 0 and A.dequantize(wq, s, b).tolist() == [[0.5] * 64]
    wq, s, b = A.quantize(np.zeros((1, 64), np.float32))
    assert b[0, 0] == 0 and A.dequantize(wq, s, b).max() == 0


def test_quantize_invariants_random_groups():
    rng = np.random.default_rng(3)
    w = A.round_to_bf16((rng.standard_normal((32, 1024)) * 0.02).astype(np.float32))
    w[0, :64] *= 50  # an outlier group
    wq, s, b = A.quantize(w)
    q = A.unpack(wq).astype(np.float64).reshape(32, 16, 64)
    assert q.min() >= 0 and q.max() <= 15
    sf = A.bf16_bits_to_f32(s).astype(np.float64)[..., None]
    bf = A.bf16_bits_to_f32(b).astype(np.float64)[..., None]
    wg = w.astype(np.float64).reshape(32, 16, 64)
    # reconstruction error <= |s|/2 (plus what bf16 rounding of s and b moves) for
    # interior codes; the end codes may clip, because the refined scale edge/q0
    # pins the edge element exactly and can leave the far end outside the grid
    err = np.abs(wg - (sf * q + bf))
    slack = np.abs(sf) * 2**-8 * 15 + np.abs(bf) * 2**-8
    interior = (q > 0) & (q < 15)
    assert np.all((err <= np.abs(sf) / 2 + slack + 1e-12)[interior])
    # chosen q is the nearest grid point (with the unrounded fp32 scale/bias this is
    # exact; against the bf16-stored ones allow the same slack)
    grid = sf[..., None] * np.arange(16)[None, None, None, :] + bf[..., None]
    best = np.abs(wg[..., None] - grid).min(-1)
    assert np.all(err <= best + slack + 1e-12)
    # the edge element (the larger-magnitude end) is the bias and is coded q = 0
    w_max, w_min = wg.max(-1), wg.min(-1)
    min_edge = np.abs(w_min) > np.abs(w_max)
    edge = np.where(min_edge, w_min, w_max)
    assert np.array_equal(b, A.f32_to_bf16_bits(edge.astype(np.float32)))
    edge_pos = np.where(min_edge, wg.argmin(-1), wg.argmax(-1))
    assert np.all(np.take_along_axis(q, edge_pos[..., None], -1) == 0)
    # negative scale exactly when the max is the edge
    assert np.array_equal(sf[..., 0] < 0, ~min_edge)


def test_quantize_c_matches_numpy_large():
    rng = np.random.default_rng(4)
    w = A.round_to_bf16((rng.standard_normal((256, 3840)) * 0.02).astype(np.float32))
    a = A.quantize(w)
    c = C.quantize(w)
    assert all(np.array_equal(x, y) for x, y in zip(a, c))


# ---------------------------------------------------------------- quantized matmul

def _brute_qmm(x_bits, wq, s, b):
    """Pure-Python triple loop over the packed bytes (tiny shapes only)."""
    m, k = x_bits.shape
    n = wq.shape[0]
    xs = [[float(A.bf16_bits_to_f32(np.array([x_bits[i, c]]))[0]) for c in range(k)] for i in range(m)]
    y = np.zeros((m, n))
    for r in range(n):
        for i in range(m):
            acc = Fraction(0)
            for c in range(k):
                q = (int(wq[r, c // 8]) >> (4 * (c % 8))) & 0xF
                sc = Fraction(float(A.bf16_bits_to_f32(np.array([s[r, c // 64]]))[0]))
                bi = Fraction(float(A.bf16_bits_to_f32(np.array([b[r, c // 64]]))[0]))
                acc += Fraction(xs[i][c]) * (sc * q + bi)
            y[i, r] = float(acc)
    return y


def test_qmm_brute_force_tiny():
    rng = np.random.default_rng(5)
    w = A.round_to_bf16((rng.standard_normal((3, 128)) * 0.02).astype(np.float32))
    wq, s, b = A.quantize(w)
    x = A.make_activations(2, 128, 11, outliers=True)
    want = _brute_qmm(x, wq, s, b)
    assert np.allclose(A.qmm_f64(x, wq, s, b), want, rtol=0, atol=1e-12)
    assert np.allclose(C.qmm_f64(x, wq, s, b), want, rtol=0, atol=1e-12)


def test_qmm_matches_float64_matmul_and_transpose_convention():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(6)
    n, k, m = 48, 384, 5
    w = A.round_to_bf16((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    wq, s, b = A.quantize(w)
    x = A.make_activations(m, k, 12)
    wd = torch.from_numpy(A.dequantize(wq, s, b)).double()
    xd = torch.from_numpy(A.bf16_bits_to_f32(x)).double()
    want = (xd @ wd.T).numpy()  # y = x . W^T  (transpose=true)
    got = A.qmm_f64(x, wq, s, b)
    assert got.shape == (m, n)
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)
    assert np.allclose(C.qmm_f64(x, wq, s, b), want, rtol=1e-12, atol=1e-12)


def test_qmm_closed_forms():
    k = 256
    # all q = 0 with bias beta per group: y = sum_g beta_g * sum_{k in g} x_k
    wq = np.zeros((2, k // 8), np.uint32)
    s = A.f32_to_bf16_bits(np.full((2, 4), 0.37, np.float32))
    beta = np.array([[0.5, -1.0, 2.0, 0.25], [1.0, 1.0, 1.0, 1.0]], np.float32)
    b = A.f32_to_bf16_bits(beta)
    x = A.make_activations(3, k, 13)
    xf = A.bf16_bits_to_f32(x).astype(np.float64).reshape(3, 4, 64).sum(-1)
    want = xf @ beta.astype(np.float64).T
    assert np.allclose(A.qmm_f64(x, wq, s, b), want, atol=1e-12)
    assert np.allclose(C.qmm_f64(x, wq, s, b), want, atol=1e-12)
    # zero activations -> zero output
    assert np.all(C.qmm_f64(np.zeros((2, k), np.uint16), wq, s, b) == 0)
    # all q = 15, bias 0, scale 1: y = 15 * sum x
    wq15 = A.pack(np.full((1, k), 15, np.uint32))
    one = A.f32_to_bf16_bits(np.ones((1, 4), np.float32))
    zero = np.zeros((1, 4), np.uint16)
    y = C.qmm_f64(x, wq15, one, zero)
    assert np.allclose(y[:, 0], 15 * A.bf16_bits_to_f32(x).astype(np.float64).sum(1), atol=1e-9)


def test_qmm_f32_baseline_close_to_f64():
    rng = np.random.default_rng(8)
    w = A.round_to_bf16((rng.standard_normal((64, 3840)) * 0.02).astype(np.float32))
    wq, s, b = A.quantize(w)
    x = A.make_activations(4, 3840, 14)
    y64 = C.qmm_f64(x, wq, s, b)
    y32 = C.qmm_f32(x, wq, s, b)
    ok, worst = A.check_f32_output(y32, y64)
    assert ok, worst


# ---------------------------------------------------------------- tolerance helpers

def test_tolerance_helpers_accept_exact_and_reject_planted_error():
    rng = np.random.default_rng(9)
    y = rng.standard_normal((4, 1000)) * 1.3
    assert A.check_f32_output(y.astype(np.float32), y)[0]
    assert A.check_bf16_output(A.f32_to_bf16_bits(y.astype(np.float32)), y)[0]
    bad = y.copy()
    bad[1, 7] += 0.05 * np.sqrt(np.mean(y ** 2))
    assert not A.check_f32_output(bad.astype(np.float32), y)[0]
    assert not A.check_bf16_output(A.f32_to_bf16_bits(bad.astype(np.float32)), y)[0]


def test_f64_to_bf16_rounds_once():
    """Agrees with the float32 conversion where float32 holds the value exactly, and
    rounds a value just past a bf16 midpoint away from it (float32 first would tie
    to even): 1 + 2^-8 + 2^-40 -> 1 + 2^-7, 1 + 2^-8 -> 1 (tie to even),
    1 + 3 * 2^-8 -> 1 + 2^-6 (tie to even, upwards), negative values alike."""
    v = A.bf16_bits_to_f32(np.arange(0x0080, 0x7F00, 7, dtype=np.uint16)).astype(np.float64)
    v = np.concatenate([v, -v, v * (1 + 2.0 ** -9), v * (1 + 2.0 ** -8)])
    assert np.array_equal(A.f64_to_bf16_bits(v), A.f32_to_bf16_bits(v.astype(np.float32)))
    cases = {1 + 2.0 ** -8 + 2.0 ** -40: 1 + 2.0 ** -7, 1 + 2.0 ** -8: 1.0, 1 + 3 * 2.0 ** -8: 1 + 2.0 ** -6,
             -(1 + 2.0 ** -8 + 2.0 ** -40): -(1 + 2.0 ** -7), 1 + 2.0 ** -8 - 2.0 ** -40: 1.0}
    got = A.bf16_bits_to_f32(A.f64_to_bf16_bits(np.array(list(cases)))).astype(np.float64)
    assert np.array_equal(got, np.array(list(cases.values())))
    assert A.f32_to_bf16_bits(np.float32(1 + 2.0 ** -8 + 2.0 ** -40)) == 0x3F80  # the double rounding


def test_bf16_rounding_helper_pins_one_rounding_of_a_near_exact_value():
    """check_bf16_rounding accepts RNE(exact) and RNE(exact + small accumulation
    error), and rejects a value rounded the wrong way on a large output (one ulp off
    where the accumulation error cannot reach the boundary), a truncation, and an
    error beyond acc_rel * RMS on a tiny output."""
    rng = np.random.default_rng(19)
    y = rng.standard_normal((4, 2000)) * 1.3
    rms = float(np.sqrt(np.mean(y ** 2)))
    rne = A.f64_to_bf16_bits(y)
    ok, worst, equal = A.check_bf16_rounding(rne, y)
    assert ok and equal == 1.0 and worst <= 0.0
    # an accumulation error of 1e-5 RMS before the rounding: still one rounding of a
    # near-exact value, and nearly every output equals RNE(exact)
    noisy = A.f32_to_bf16_bits((y + rng.uniform(-1e-5, 1e-5, y.shape) * rms).astype(np.float32))
    ok, _, equal = A.check_bf16_rounding(noisy, y)
    assert ok and 0.99 < equal <= 1.0
    # largest output moved one ulp: the exact value sits ~half an ulp (>> 1e-4 RMS)
    # from where that rounding would need it
    i = np.unravel_index(np.argmax(np.abs(y)), y.shape)
    off = rne.copy()
    off[i] = off[i] + 1
    assert not A.check_bf16_rounding(off, y)[0]
    # truncation instead of rounding: wrong on about half the outputs
    trunc = (y.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    assert not A.check_bf16_rounding(trunc, y)[0]
    # a tiny output carrying an error of 1e-3 RMS (far above its half ulp)
    j = np.unravel_index(np.argmin(np.abs(y)), y.shape)
    tiny = rne.copy()
    tiny[j] = A.f32_to_bf16_bits(np.float32(y[j] + 1e-3 * rms))[0]
    assert not A.check_bf16_rounding(tiny, y)[0]


# ---------------------------------------------------------------- GeGLU

def test_geglu_matches_library_gelu_tanh():
    torch = pytest.importorskip("torch")
    g = A.make_activations(4, 512, 21)
    u = A.make_activations(4, 512, 22)
    got = A.bf16_bits_to_f32(A.gelu_tanh_times(g, u))
    gt = torch.from_numpy(A.bf16_bits_to_f32(g)).double()
    ut = torch.from_numpy(A.bf16_bits_to_f32(u)).double()
    want = (torch.nn.functional.gelu(gt, approximate="tanh") * ut).numpy()
    # bf16 ops, each rounded (the bf16 model dtype): the error bound of
    # tests/test_geglu_oracle.py, scaled by |up|
    gu = np.abs(A.bf16_bits_to_f32(g).astype(np.float64) * A.bf16_bits_to_f32(u))
    assert np.all(np.abs(got - want) <= 2.0 ** -6 * (np.abs(want) + 0.5 * gu) + 1e-30)
