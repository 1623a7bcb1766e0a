"""Pins for the oracle at bits = 8 (the QAT override the reference's loader allows,
model_manifest.cc:148; MLX packs four 8-bit codes per uint32, lowest byte first):

* pack/unpack: hand vector, lowest byte first;
* dequantize: every code 0..255 against exact rationals rounded once (s*q is exact
  in fp32: 8 + 8 significant bits);
* quantize: known-answer groups against an independent restatement with 255 bins;
* qmm: brute force with exact rationals on a tiny shape, and the two-plane identity
  the kernels use (q = 16*qh + ql, w = (16s)*qh + b + s*ql) reproduces the 8-bit
  product exactly.
"""

from fractions import Fraction

import numpy as np

from oracle import affine as A
from oracle import c_oracle as C


def test_pack_hand_vector_lowest_byte_first():
    q = np.array([[0x01, 0x23, 0x45, 0x67, 0xFF, 0x80, 0x00, 0x7F]], np.uint32)
    wq = A.pack(q, 8)
    assert wq.tolist() == [[0x67452301, 0x7F0080FF]]
    assert np.array_equal(A.unpack(wq, 8), q.astype(np.uint8))


def test_dequantize_all_codes_exact():
    rng = np.random.default_rng(21)
    n = 64
    s = A.f32_to_bf16_bits((rng.standard_normal(n) * 0.001).astype(np.float32))
    s[:4] = A.f32_to_bf16_bits(np.array([-1.05, 3.0e-3, 0.0, 2.0 ** -30], np.float32))
    b = A.f32_to_bf16_bits((rng.standard_normal(n) * 0.05).astype(np.float32))
    q = np.tile(np.arange(256, dtype=np.uint32)[None, :64], (n, 1))
    q = np.concatenate([q + 0, q + 64, q + 128, q + 192], axis=1)  # every code, K = 256
    wq = A.pack(q, 8)
    s4, b4 = np.repeat(s[:, None], 4, 1), np.repeat(b[:, None], 4, 1)
    deq = A.dequantize(wq, s4, b4, bits=8)
    assert np.array_equal(deq.view(np.uint32), C.dequantize(wq, s4, b4, bits=8).view(np.uint32))
    sf, bf = A.bf16_bits_to_f32(s), A.bf16_bits_to_f32(b)
    for r in range(0, n, 3):
        for c in range(256):
            exact = Fraction(float(sf[r])) * int(q[r, c]) + Fraction(float(bf[r]))
            assert deq[r, c] == np.float32(float(exact)), (r, c)


def _frac_quantize_group8(vals):
    f32 = np.float32
    w = [f32(v) for v in vals]
    w_max, w_min = max(w), min(w)
    mask = abs(w_min) > abs(w_max)
    scale = max(f32(float(Fraction(float(w_max - w_min)) / 255)), f32(1e-7))
    scale = scale if mask else -scale
    edge = w_min if mask else w_max
    q0 = np.rint(f32(float(Fraction(float(edge)) / Fraction(float(scale)))))
    bias = f32(0)
    if q0 != 0:
        scale = f32(float(Fraction(float(edge)) / Fraction(float(q0))))
        bias = edge
    q = [int(min(max(np.rint(f32(float(Fraction(float(f32(v - bias))) / Fraction(float(scale))))), 0), 255))
         for v in w]
    return q, f32(scale), f32(bias)


def test_quantize_known_answer_groups():
    groups = {"ramp": [j / 8 for j in range(64)], "down": [-j / 16 for j in range(64)],
              "straddle": [(j - 16) / 32 for j in range(64)], "constant": [0.25] * 64}
    for name, vals in groups.items():
        wq, s, b = A.quantize(np.array([vals], np.float32), bits=8)
        q, scale, bias = _frac_quantize_group8(vals)
        assert A.unpack(wq, 8)[0].tolist() == q, name
        assert s[0, 0] == A.f32_to_bf16_bits(np.array([scale]))[0], name
        assert b[0, 0] == A.f32_to_bf16_bits(np.array([bias]))[0], name
        assert all(np.array_equal(x, y) for x, y in zip((wq, s, b), C.quantize(np.array([vals], np.float32), bits=8)))


def test_qmm_brute_force_and_two_plane_identity():
    rng = np.random.default_rng(22)
    w = A.round_to_bf16((rng.standard_normal((3, 128)) * 0.02).astype(np.float32))
    wq, s, b = A.quantize(w, bits=8)
    x = A.make_activations(2, 128, 23, outliers=True)
    q = A.unpack(wq, 8).astype(int)
    xs = A.bf16_bits_to_f32(x)
    sf, bf = A.bf16_bits_to_f32(s), A.bf16_bits_to_f32(b)
    want = np.zeros((2, 3))
    for i in range(2):
        for r in range(3):
            acc = Fraction(0)
            for c in range(128):
                acc += Fraction(float(xs[i, c])) * (Fraction(float(sf[r, c // 64])) * q[r, c] + Fraction(float(bf[r, c // 64])))
            want[i, r] = float(acc)
    assert np.allclose(A.qmm_f64(x, wq, s, b, bits=8), want, rtol=0, atol=1e-12)
    assert np.allclose(C.qmm_f64(x, wq, s, b, bits=8), want, rtol=0, atol=1e-12)
    # two planes over K' = 2K with x' = [x | x]: high nibbles (scale 16s, bias b),
    # low nibbles (scale s, bias 0)
    hi = A.pack(q >> 4, 4)
    lo = A.pack(q & 15, 4)
    wq2 = np.concatenate([hi, lo], axis=1)
    s2 = np.concatenate([A.f32_to_bf16_bits(sf * 16), s], axis=1)
    b2 = np.concatenate([b, np.zeros_like(b)], axis=1)
    x2 = np.concatenate([x, x], axis=1)
    assert np.allclose(A.qmm_f64(x2, wq2, s2, b2), want, rtol=0, atol=1e-12)
