"""The oracle's lm_head softcap and greedy pick (oracle/affine.py softcap_ops, greedy),
pinned without the reference (native_model.cc:1782-1795 softcap, :3734 argmax):

* fp32: softcap_ops agrees with the float64 closed form 30*tanh(x/30) to a few ulps;
* bf16: over all 65536 bf16 logits it stays within what its per-op roundings allow of
  the float64 closed form, is odd-symmetric and monotone (non-decreasing), and a
  hand-derived value pins the op order;
* greedy returns the first maximum (np.argmax's documented rule) and its value.
"""

import numpy as np

from oracle import affine as A


def test_f32_matches_closed_form():
    rng = np.random.default_rng(2)
    x = np.concatenate([rng.standard_normal(50000) * 20, rng.standard_normal(5000) * 300,
                        [0.0, -0.0, 1e-30, 29.9, -29.9, 1e4, -1e4]]).astype(np.float32)
    got = A.softcap_ops(x, 30.0, bf16=False).astype(np.float64)
    ref = 30.0 * np.tanh(x.astype(np.float64) / 30.0)
    assert np.all(np.abs(got - ref) <= 4 * 2.0 ** -24 * np.abs(ref) + 1e-37), np.max(np.abs(got - ref))
    assert np.array_equal(A.softcap_ops(x, 0.0, bf16=False), x)


def test_bf16_all_logits():
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    x = A.bf16_bits_to_f32(bits)
    x = x[np.isfinite(x)]
    got = A.softcap_ops(x, 30.0, bf16=True).astype(np.float64)
    ref = 30.0 * np.tanh(x.astype(np.float64) / 30.0)
    # the quotient, tanh and product roundings (2^-9 relative each, carried through
    # tanh' <= 1) plus the rounding of 30 * tanh where bf16's spacing is coarsest
    assert np.all(np.abs(got - ref) <= 5 * 2.0 ** -9 * np.abs(ref) + 1e-38)
    assert np.array_equal(A.softcap_ops(-x, 30.0, True), -A.softcap_ops(x, 30.0, True))
    order = np.argsort(x, kind="stable")
    assert np.all(np.diff(got[order]) >= 0)
    assert np.max(got) == 30.0  # saturates at the cap exactly
    assert np.array_equal(A.softcap_ops(x, 0.0, True), x)


def test_bf16_hand_derived_value():
    # logits = 10: 10/30 = 0.33333... -> bf16 0.333984375 (ulp 2^-9 in [0.25, 0.5): 170.67 -> 171);
    # tanh(0.333984375) = 0.3220964... -> bf16 0.322265625 (164.91 -> 165);
    # 0.322265625 * 30 = 9.66796875 -> bf16 (ulp 2^-4 in [8, 16)): 154.69 -> 155 -> 9.6875
    assert float(A.softcap_ops(np.float32(10.0), 30.0, True).reshape(-1)[0]) == 9.6875
    assert abs(np.tanh(0.333984375) - 0.3220964) < 1e-6
    # logits = 8: 8/30 -> 0.267578125 (136.53 ulps of 2^-9 -> 137); tanh = 0.2613698 ->
    # 0.26171875 (133.82 -> 134); * 30 = 7.8515625 -> 7.84375 (251.25 ulps of 2^-5 -> 251).
    # (Without rounding the quotient first: 7.78125.)
    assert float(A.softcap_ops(np.float32(8.0), 30.0, True).reshape(-1)[0]) == 7.84375
    assert abs(np.tanh(0.267578125) - 0.2613698) < 1e-6
    # logits = 5: 5/30 -> 0.1669921875 (170.67 ulps of 2^-10 -> 171); tanh = 0.1654575 ->
    # 0.1650390625 (169.43 -> 169); * 30 = 4.951171875 -> 4.9375 (158.44 -> 158).
    # (Without rounding tanh first: 4.96875.)
    assert float(A.softcap_ops(np.float32(5.0), 30.0, True).reshape(-1)[0]) == 4.9375
    assert abs(np.tanh(0.1669921875) - 0.1654575) < 1e-6


def test_greedy_first_maximum():
    v = np.array([[1.0, 3.0, 2.0, 3.0], [-1.0, -1.0, -2.0, -5.0], [0.0, 0.0, 0.0, 0.0]], np.float32)
    idx, val = A.greedy(v)
    assert idx.tolist() == [1, 0, 0] and val.tolist() == [3.0, -1.0, 0.0]
    rng = np.random.default_rng(4)
    w = rng.integers(0, 5, (50, 300)).astype(np.float32)  # many ties
    idx, val = A.greedy(w)
    for r in range(50):
        first = int(np.nonzero(w[r] == w[r].max())[0][0])
        assert idx[r] == first and val[r] == w[r].max()
