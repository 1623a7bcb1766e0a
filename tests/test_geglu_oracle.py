"""The oracle's GeGLU (oracle/affine.py geglu_ops), the epilogue of the fused gate|up
projection (native_model.cc:378-386), pinned without the reference:

* the constants are the bf16 values nearest the reference's fp32 constants
  (model_scalar makes them bf16 in the bf16 model dtype, native_model.cc:342-347);
* in fp32 the op sequence agrees with torch's tanh-approximation GELU (a library
  routine of the same formula) evaluated in float64, times up;
* in bf16, every one of the 65536 bf16 gate values stays within the error the
  per-op bf16 roundings allow of the float64 formula (a dropped or altered term
  fails somewhere over that range), and a hand-derived value pins the op order and
  the round-half-to-even inside it;
* the prefill epilogue's compact gelu table (q4_common.h kGeluTable: entries only
  for biased exponents 118..128, closed forms elsewhere) reproduces the op sequence
  for every bf16 pattern, infinities and NaN included.
"""

import numpy as np
import torch

from oracle import affine as A


def exact_gelu64(g):
    g = np.asarray(g, dtype=np.float64)
    return 0.5 * g * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (g + 0.044715 * g ** 3)))


def test_constants_are_the_nearest_bf16_values():
    for c, want in ((A.GEGLU_C_TANH, 0.796875), (A.GEGLU_C_CUBIC, 0.044677734375)):
        got = float(A.round_to_bf16(np.float32(c))[0])
        assert got == want
        # the bf16 neighbours of `want` are farther from the fp32 constant
        bits = int(A.f32_to_bf16_bits(np.float32(want))[0])
        for nb in (bits - 1, bits + 1):
            assert abs(float(A.bf16_bits_to_f32(np.uint16(nb))[0]) - c) > abs(want - c)
    assert np.float32(A.GEGLU_C_TANH) == np.float32(np.sqrt(2.0 / np.pi))


def test_f32_matches_torch_gelu_tanh():
    rng = np.random.default_rng(11)
    g = np.concatenate([rng.standard_normal(20000) * 3, rng.standard_normal(2000) * 30,
                        [0.0, -0.0, 1e-30, -1e-30, 5.0, -5.0, 80.0, -80.0]]).astype(np.float32)
    u = rng.standard_normal(g.size).astype(np.float32)
    got = A.geglu_ops(g, u, bf16=False).astype(np.float64)
    ref = torch.nn.functional.gelu(torch.from_numpy(g.astype(np.float64)), approximate="tanh").numpy() * u
    # float32 ops: a few ulps relative, plus cancellation in 1 + tanh for negative g
    # (absolute error ~ 0.5*|g|*|u| * 2^-23 per op)
    tol = 8 * 2.0 ** -24 * (np.abs(ref) + 0.5 * np.abs(g * u)) + 1e-37
    assert np.all(np.abs(got - ref) <= tol), np.max(np.abs(got - ref) / tol)


def test_bf16_all_gate_values_within_rounding_error():
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    g = A.bf16_bits_to_f32(bits)
    g = g[np.isfinite(g)]
    h = A.geglu_ops(g, np.ones_like(g), bf16=True).astype(np.float64)
    assert np.all(np.isfinite(h))
    ref = exact_gelu64(g)
    # each of the ~9 roundings contributes at most 2^-9 relative to its own result;
    # the sum 1 + t and the product carry that into 0.5*|g| absolute at most
    tol = 2.0 ** -6 * (0.5 * np.abs(g) + np.abs(ref)) + 1e-38
    assert np.all(np.abs(h - ref) <= tol), np.max(np.abs(h - ref) / tol)
    assert np.all(h[g == 0] == 0)
    assert np.all(h[(g > 0) & (g < 3e38) & (g > 4)] == g[(g > 0) & (g < 3e38) & (g > 4)])  # tanh -> 1, exact


def test_bf16_hand_derived_value():
    # g = 1, up = 1 in bf16 ops:
    #   g^3 = 1;  c2*g^3 = 0.044677734375 (bf16 constant, exact);
    #   a = bf16(1.044677734375) = 1.046875 (ulp 2^-7: 133.72 -> 134);
    #   c1*a = 0.796875 * 1.046875 = 0.834228515625 -> bf16 0.8359375 (ulp 2^-8: 213.56 -> 214);
    #   tanh(0.8359375) = 0.68366... -> bf16 0.68359375 (175.02 -> 175);
    #   1 + t = 1.68359375 -> bf16: 215.5 ulps of 2^-7, a tie, to even 216 -> 1.6875;
    #   0.5*g = 0.5;  gelu = bf16(0.5 * 1.6875) = 0.84375;  h = 0.84375 * 1 = 0.84375
    assert float(A.geglu_ops(np.float32(1.0), np.float32(1.0), bf16=True).reshape(-1)[0]) == 0.84375
    assert abs(np.tanh(0.8359375) - 0.68366) < 1e-5
    # g = 1.5, up = 1:
    #   g^3 = 3.375;  c2*g^3 = 0.150787353515625 -> 0.150390625 (ulp 2^-10: 154.41 -> 154);
    #   a = 1.650390625 -> 1.6484375 (211.25 -> 211);
    #   c1*a = (51/64)*(211/128) = 1.3135986328125 -> 1.3125 (168.14 -> 168);
    #   tanh(1.3125) = 0.864907 -> 0.86328125 (221.42 -> 221);
    #   1 + t = 1.86328125: 238.5 ulps of 2^-7, a tie, to even 238 -> 1.859375;
    #   gelu = 0.75 * 1.859375 = 1.39453125: 178.5 ulps, a tie, to even 178 -> 1.390625
    #   (without rounding 1 + t first it would be 1.3984375)
    assert float(A.geglu_ops(np.float32(1.5), np.float32(1.0), bf16=True).reshape(-1)[0]) == 1.390625
    assert abs(np.tanh(1.3125) - 0.864907) < 1e-6


def test_compact_gelu_table_covers_every_pattern():
    import warnings

    bits = np.arange(1 << 16, dtype=np.uint32)
    g = A.bf16_bits_to_f32(bits.astype(np.uint16))
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        want = A.f32_to_bf16_bits(A.geglu_ops(g, np.ones_like(g), bf16=True))
        e, neg, man = (bits >> 7) & 0xFF, bits >> 15, bits & 0x7F
        lo, n_exp = 118, 11
        idx = np.arange(2 * n_exp * 128)
        pat = ((idx // (n_exp * 128)) << 15) | ((lo + (idx // 128) % n_exp) << 7) | (idx % 128)
        table = A.f32_to_bf16_bits(A.geglu_ops(A.bf16_bits_to_f32(pat.astype(np.uint16)), np.ones(idx.size, np.float32),
                                               bf16=True))
        got = np.empty_like(want)
        tab = (e >= lo) & (e < lo + n_exp)
        got[tab] = table[((neg * n_exp + (e - lo)) * 128 + man)[tab]]
        small = e < lo
        got[small] = A.f32_to_bf16_bits(A.round_to_bf16(np.float32(0.5) * g[small]))
        big = (e >= lo + n_exp) & (e < 255)
        got[big & (neg == 0)] = bits[big & (neg == 0)]
        got[big & (neg == 1)] = 0x8000
        spec = e == 255
        got[spec] = np.where((man[spec] == 0) & (neg[spec] == 0), bits[spec], 0xFFC0)
    nan = np.isnan(A.bf16_bits_to_f32(want))
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all(np.isnan(A.bf16_bits_to_f32(got[nan])))
