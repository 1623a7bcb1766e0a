"""Writes tests/golden/q4_golden.npz: small affine-Q4 vectors whose expected outputs
come from exact rational arithmetic, independent of the oracle and of the kernels.

The reference holds no quantization vectors (its parity checks are whole-model
token dumps that need a 6.7 GB checkpoint), so these fixtures are built here from
the definition of the op (native/gemma4_mlx/src/native_model.cc:349-362, :281-287):

    q[n, k] = (W[n, k // 8] >> 4 * (k % 8)) & 0xF          (LSB-first nibbles)
    w[n, k] = s[n, k // 64] * q[n, k] + b[n, k // 64]        (bf16 s, b)
    y[m, n] = sum_k x[m, k] * w[n, k]                        (transpose=true)

Every value is a ``fractions.Fraction``; dequantized weights and outputs are
rounded once, round-to-nearest-even, to fp32 and bf16 by ``round_fraction`` below
(a direct statement of IEEE-754 rounding, subnormals included).  Dequantized
weights are also rounded from the exact s*q + b, so they pin the fp32 dequant
contract bit for bit.

Cases
  dq_*   dequantize: 6 rows x 128 (2 groups), every nibble value in every group,
         scales/biases chosen to hit sign changes, exact cancellation, results
         below the fp32 normal range, huge/tiny exponent gaps, zero scale.
  mm_*   matmul: M=3, N=8, K=192 (3 groups: odd group count, N not a multiple of
         16), seeded N(0,1) bf16 activations with one x20 outlier, seeded codes and
         bf16 scales/biases of the size a N(0, 0.02) weight quantizes to, packed
         by the nibble rule above.
  ed_*   matmul edges: M=3, N=5, K=64; an all-zero activation row, a row of
         powers of two, zero scales (bias only), negative scales, all-15 codes.

Run from the repository root:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import os
from fractions import Fraction

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "q4_golden.npz")
GROUP = 64


def round_fraction(v: Fraction, mant_bits: int, emin: int = -126, emax: int = 127) -> float:
    """Rounds an exact rational to the nearest binary float with `mant_bits`
    significand bits (24: fp32, 8: bf16) and exponent range [emin, emax], ties to
    even; below 2**emin the spacing stays 2**(emin - mant_bits + 1) (subnormals)."""
    if v == 0:
        return 0.0
    neg = v < 0
    a = -v if neg else v
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    if Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, emin)
    quantum = Fraction(2) ** (e - mant_bits + 1)
    q = a // quantum
    r = a - q * quantum
    half = quantum / 2
    if r > half or (r == half and q % 2 == 1):
        q += 1
    val = q * quantum
    if val >= Fraction(2) ** (emax + 1):
        out = float("inf")
    else:
        out = float(val)
    return -out if neg else out


def f32_bits(v: float) -> int:
    return int(np.array([v], dtype=np.float32).view(np.uint32)[0])


def bf16_bits_exact(v: float) -> int:
    """bf16 bit pattern of a value that is exactly representable in bf16."""
    u = f32_bits(v)
    assert u & 0xFFFF == 0, v
    return u >> 16


def bf16_value(bits: int) -> Fraction:
    return Fraction(float(np.array([bits << 16], dtype=np.uint32).view(np.float32)[0]))


def bf16_of(x: float) -> int:
    """bf16 bits nearest to a float (via the exact rounding above)."""
    return bf16_bits_exact(round_fraction(Fraction(x), 8))


def pack_rows(q: np.ndarray) -> np.ndarray:
    """Nibble rule: element k of a row -> word k // 8, bits 4*(k % 8) .. +3."""
    n, k = q.shape
    w = np.zeros((n, k // 8), dtype=np.uint32)
    for r in range(n):
        for c in range(k):
            w[r, c // 8] |= np.uint32(int(q[r, c]) << (4 * (c % 8)))
    return w


def exact_weights(q, s_bits, b_bits):
    n, k = q.shape
    return [[bf16_value(int(s_bits[r, c // GROUP])) * int(q[r, c]) + bf16_value(int(b_bits[r, c // GROUP]))
             for c in range(k)] for r in range(n)]


def dequant_case():
    n, k = 6, 128
    rng = np.random.Generator(np.random.PCG64(7001))
    q = np.zeros((n, k), dtype=np.uint32)
    for r in range(n):
        for g in range(k // GROUP):
            q[r, g * GROUP:(g + 1) * GROUP] = rng.permutation(np.tile(np.arange(16), GROUP // 16))
    # (scale, bias) per (row, group) as floats, each exactly a bf16
    pairs = [
        [(0.0078125, -0.05859375), (-0.01171875, 0.1015625)],   # ordinary, both signs
        [(0.25, -1.875), (-0.125, 0.9375)],                      # s*q + b hits exact zero
        [(1e-20, 1.0), (3.0e8, -2.5e9)],                         # exponent gaps
        [(2.0 ** -130, 2.0 ** -128), (2.0 ** -126, -(2.0 ** -123))],  # fp32 subnormal results
        [(0.0, 0.5), (0.0, -0.0)],                               # zero scale: bias only, signed zero
        [(1.0e30, -7.5e30), (-3.0e-5, 1.2e-3)],                  # large magnitude, small magnitude
    ]
    s_bits = np.array([[bf16_of(p[0]) for p in row] for row in pairs], dtype=np.uint16)
    b_bits = np.array([[bf16_of(p[1]) for p in row] for row in pairs], dtype=np.uint16)
    b_bits[4, 1] = 0x8000  # -0: (+0)*q + (-0) is +0 under round-to-nearest, as the exact sum says
    exact = exact_weights(q, s_bits, b_bits)
    w_f32 = np.array([[round_fraction(v, 24) for v in row] for row in exact], dtype=np.float32)
    return {"dq_wq": pack_rows(q), "dq_scales": s_bits, "dq_biases": b_bits, "dq_w_f32": w_f32}


def matmul_expected(x_bits, q, s_bits, b_bits):
    m, k = x_bits.shape
    n = q.shape[0]
    w = exact_weights(q, s_bits, b_bits)
    xs = [[bf16_value(int(x_bits[i, c])) for c in range(k)] for i in range(m)]
    y_exact = np.zeros((m, n), dtype=np.float64)
    y_f32 = np.zeros((m, n), dtype=np.float32)
    y_bf16 = np.zeros((m, n), dtype=np.uint16)
    for i in range(m):
        for j in range(n):
            acc = sum((xs[i][c] * w[j][c] for c in range(k)), Fraction(0))
            y_exact[i, j] = float(acc)
            y_f32[i, j] = round_fraction(acc, 24)
            y_bf16[i, j] = bf16_bits_exact(round_fraction(acc, 8))
    return y_exact, y_f32, y_bf16


def matmul_case():
    m, n, k = 3, 8, 192
    rng = np.random.Generator(np.random.PCG64(7002))
    xf = rng.standard_normal((m, k))
    xf[1, 37] *= 20.0
    x_bits = np.array([[bf16_of(v) for v in row] for row in xf], dtype=np.uint16)
    # weights: integer codes and bf16 scale/bias drawn directly (the op is defined on
    # the stored triple; how it was quantized does not enter the product)
    q = rng.integers(0, 16, size=(n, k), dtype=np.uint32)
    s = rng.uniform(0.002, 0.008, size=(n, k // GROUP)) * rng.choice([-1.0, 1.0], size=(n, k // GROUP))
    b = -7.5 * s + rng.normal(0.0, 0.002, size=(n, k // GROUP))
    s_bits = np.array([[bf16_of(v) for v in row] for row in s], dtype=np.uint16)
    b_bits = np.array([[bf16_of(v) for v in row] for row in b], dtype=np.uint16)
    y_exact, y_f32, y_bf16 = matmul_expected(x_bits, q, s_bits, b_bits)
    return {"mm_x": x_bits, "mm_wq": pack_rows(q), "mm_scales": s_bits, "mm_biases": b_bits,
            "mm_y_exact": y_exact, "mm_y_f32": y_f32, "mm_y_bf16": y_bf16}


def edge_case():
    m, n, k = 3, 5, 64
    x = np.zeros((m, k))
    x[1] = [2.0 ** ((c % 7) - 3) * (-1) ** c for c in range(k)]
    x[2] = np.linspace(-4.0, 4.0, k)
    x_bits = np.array([[bf16_of(v) for v in row] for row in x], dtype=np.uint16)
    q = np.zeros((n, k), dtype=np.uint32)
    q[0] = np.arange(k) % 16
    q[1] = 15
    q[2] = (np.arange(k) * 7) % 16
    q[3] = np.arange(k) % 16
    q[4] = 0
    s = np.array([[0.03125], [-0.015625], [0.0], [-0.5], [1.0]])
    b = np.array([[-0.25], [0.125], [0.75], [3.75], [-0.0078125]])
    s_bits = np.array([[bf16_of(v) for v in row] for row in s], dtype=np.uint16)
    b_bits = np.array([[bf16_of(v) for v in row] for row in b], dtype=np.uint16)
    y_exact, y_f32, y_bf16 = matmul_expected(x_bits, q, s_bits, b_bits)
    return {"ed_x": x_bits, "ed_wq": pack_rows(q), "ed_scales": s_bits, "ed_biases": b_bits,
            "ed_y_exact": y_exact, "ed_y_f32": y_f32, "ed_y_bf16": y_bf16}


def main():
    data = {}
    data.update(dequant_case())
    data.update(matmul_case())
    data.update(edge_case())
    np.savez(OUT, **data)
    print(f"wrote {OUT}: " + ", ".join(f"{k}{list(v.shape)}" for k, v in data.items()))


if __name__ == "__main__":
    main()
