"""The oracle's LoRA delta (oracle/affine.py lora_ops, native_model.cc:316-328) and the
adapter-loading rules (helios_amd/loader.py: PEFT prefix mapping and target-module
matching of native_model.cc:237-279), on the CPU:

* rank 1 with A = a unit vector e_j and B = ones gives delta = scale * x_j in every
  column (closed form); scale 0 leaves the (rounded) base;
* fp32 agrees with a float64 x A^T B^T scale to fp32 rounding; bf16 rounds base,
  delta and the sum (hand-checked value);
* prefixes and target modules map as the reference maps them.
"""

import numpy as np

from helios_amd import loader as L
from oracle import affine as A


def test_closed_forms():
    k, n = 128, 6
    x = A.make_activations(3, k, seed=1)
    xf = A.bf16_bits_to_f32(x).astype(np.float64)
    base = np.zeros((3, n), np.float32)
    a = np.zeros((1, k), np.float32)
    a[0, 17] = 1.0
    b = np.ones((n, 1), np.float32)
    got = A.lora_ops(x, a, b, 0.5, base, bf16=False)
    assert np.array_equal(got, np.repeat((0.5 * xf[:, 17:18]).astype(np.float32), n, 1))
    got = A.lora_ops(x, a, b, 0.0, base + 1.25, bf16=True)
    assert np.all(got == 1.25)


def test_f32_matches_float64_and_bf16_rounding():
    rng = np.random.default_rng(2)
    k, n, r = 256, 40, 8
    x = A.make_activations(4, k, seed=3)
    a = (rng.standard_normal((r, k)) * 0.05).astype(np.float32)
    b = (rng.standard_normal((n, r)) * 0.05).astype(np.float32)
    base = rng.standard_normal((4, n)).astype(np.float32)
    xf = A.bf16_bits_to_f32(x).astype(np.float64)
    ref = base.astype(np.float64) + (xf @ a.T.astype(np.float64)) @ b.T.astype(np.float64) * 2.0
    got = A.lora_ops(x, a, b, 2.0, base, bf16=False).astype(np.float64)
    assert np.allclose(got, ref, rtol=1e-6, atol=1e-6)
    gb = A.lora_ops(x, a, b, 2.0, base, bf16=True)
    assert np.array_equal(gb, A.round_to_bf16(gb))  # bf16 values
    # hand value: base 1.0, delta 0.0107421875 (exact in bf16) -> 1.0107421875 -> bf16 1.0078125
    one = np.ones((1, 1), np.float32)
    xa = A.f32_to_bf16_bits(np.array([[1.0]], np.float32))
    assert float(A.lora_ops(xa, np.array([[0.0107421875]], np.float32), one, 1.0, one, bf16=True)[0, 0]) == 1.0078125


def test_prefix_mapping_and_targets():
    assert L.canonical_lora_prefix("base_model.model.model.layers.0.mlp.up_proj") == \
        "language_model.model.layers.0.mlp.up_proj"
    assert L.canonical_lora_prefix("base_model.model.layers.1.self_attn.q_proj") == \
        "language_model.model.layers.1.self_attn.q_proj"
    assert L.canonical_lora_prefix("model.layers.2.mlp.down_proj") == "language_model.model.layers.2.mlp.down_proj"
    assert L.canonical_lora_prefix("language_model.model.x") == "language_model.model.x"
    p = "language_model.model.layers.0.self_attn.q_proj"
    assert L.target_module_allowed(p, ["q_proj"]) and L.target_module_allowed(p, [" self_attn.q_proj "])
    assert L.target_module_allowed(p, [p]) and not L.target_module_allowed(p, ["k_proj", "", "proj"])
