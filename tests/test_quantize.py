"""helios_amd.quantize (the package's MLX-format affine quantizer, torch) against the
oracle's C quantizer: identical codes, scales and biases, 4 and 8 bits, on random
weights and on groups that exercise each branch (min edge, max edge, q0 = 0, a
constant group at the 1e-7 floor, all zeros)."""

import numpy as np
import pytest
import torch

from helios_amd.quantize import quantize
from oracle import affine as A
from oracle import c_oracle as C


def special_rows(k):
    rows = [
        np.full(k, 0.0),                                 # all zero: scale floor, bias 0
        np.full(k, 0.0123),                              # constant: q0 != 0 path
        np.linspace(-0.5, 0.1, k),                       # min is the edge
        np.linspace(-0.1, 0.5, k),                       # max is the edge
        np.linspace(-1e-9, 1e-9, k),                     # tiny range: scale at the floor
        np.where(np.arange(k) % 2 == 0, -3.0, 2.0),      # two values
    ]
    return np.stack(rows).astype(np.float32)


@pytest.mark.parametrize("bits", [4, 8])
def test_quantize_matches_oracle(bits):
    rng = np.random.default_rng(17 + bits)
    k = 512
    w = np.concatenate([rng.standard_normal((58, k)).astype(np.float32) * np.float32(0.02), special_rows(k)])
    w = A.round_to_bf16(w)
    wq, s, b = quantize(torch.from_numpy(w), bits=bits)
    want_q, want_s, want_b = C.quantize(w, bits=bits)
    assert np.array_equal(wq.numpy().view(np.uint32), want_q)
    assert np.array_equal(s.view(torch.int16).numpy().view(np.uint16), want_s)
    assert np.array_equal(b.view(torch.int16).numpy().view(np.uint16), want_b)


def test_quantize_rejects_bad_shapes():
    with pytest.raises(ValueError):
        quantize(torch.zeros(4, 100))
    with pytest.raises(ValueError):
        quantize(torch.zeros(4, 128), bits=3)
