"""Loading a synthetic MLX-format checkpoint (config.json quantization block with an
8-bit override, one safetensors file) into resident handles and running them: the
results match the oracle on the triples written, with the bars of test_gpu_parity.py."""

import json

import numpy as np
import pytest

from helios_amd import loader as L
from oracle import affine as A
from oracle import c_oracle as C
from test_gpu_parity import BF16_REL, assert_close, dev_x, host_bits

pytestmark = pytest.mark.gpu


def test_checkpoint_to_handles(gpu_lib, tmp_path):
    import torch

    rng = np.random.default_rng(5)
    k, f = 384, 320
    base = "language_model.model.layers.0"
    specs = {f"{base}.self_attn.q_proj": (256, 4), f"{base}.mlp.gate_proj": (f, 4), f"{base}.mlp.up_proj": (f, 4),
             f"{base}.mlp.down_proj": (k, 8)}
    tris, tensors = {}, {}
    for prefix, (n, bits) in specs.items():
        kk = f if prefix.endswith("down_proj") else k
        w = A.round_to_bf16((rng.standard_normal((n, kk)) * 0.02).astype(np.float32))
        tris[prefix] = C.quantize(w, bits=bits)
        tensors[prefix + ".weight"] = tris[prefix][0]
        tensors[prefix + ".scales"] = ("BF16", tris[prefix][1])
        tensors[prefix + ".biases"] = ("BF16", tris[prefix][2])
    L.write_safetensors(str(tmp_path / "model.safetensors"), tensors)
    (tmp_path / "config.json").write_text(json.dumps(
        {"quantization": {"group_size": 64, "bits": 4, f"{base}.mlp.down_proj": {"group_size": 64, "bits": 8}}}))
    ck = L.Checkpoint(str(tmp_path))
    cfg = L.parse_quantization(str(tmp_path / "config.json"))
    assert ck.quantized_prefixes() == sorted(specs)

    x = A.make_activations(2, k, seed=6)
    q = L.load_linear(ck, cfg, f"{base}.self_attn.q_proj")
    y = q.forward(dev_x(x))
    pair = L.load_geglu_pair(ck, cfg, f"{base}.mlp")
    h = pair.forward(dev_x(x))
    down = L.load_linear(ck, cfg, f"{base}.mlp.down_proj")
    assert down.info()["bits"] == 8 and down.in_features == f
    d = down.forward(h)
    torch.cuda.synchronize()
    assert_close(y, C.qmm_f64(x, *tris[f"{base}.self_attn.q_proj"]), "q_proj")
    hb = host_bits(h)
    g = C.qmm_f64(x, *tris[f"{base}.mlp.gate_proj"]).astype(np.float32)
    u = C.qmm_f64(x, *tris[f"{base}.mlp.up_proj"]).astype(np.float32)
    ref = A.f32_to_bf16_bits(A.geglu_ops(g, u, bf16=True))
    assert np.mean(ref != hb) <= 0.03  # the GeGLU bar of test_gpu_geglu.py (bit-level agreement)
    ok, worst = A.check_bf16_output(host_bits(d), C.qmm_f64(hb, *tris[f"{base}.mlp.down_proj"], bits=8), BF16_REL)
    assert ok, f"down (8-bit) after the pair: worst error / RMS = {worst:.3e}"
    for o in (q, pair, down):
        o.close()
