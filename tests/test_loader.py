"""The MLX-checkpoint loader (helios_amd/loader.py) on the CPU: the quantization block
of config.json as model_manifest.cc:101-162 reads it (default, language_model.model.*
overrides limited to group 64 with 4 or 8 bits, quantization_config first), the
per-prefix lookup of native_model.cc:208-215, and the safetensors reader against the
`safetensors` library's own writer (uint32, fp32 and bf16 tensors)."""

import json

import numpy as np
import pytest

from helios_amd import loader as L
from helios_amd import qmm
from oracle import affine as A


def test_parse_quantization_defaults_and_overrides(tmp_path):
    cfg = {"quantization": {"group_size": 64, "bits": 4,
                            "language_model.model.layers.0.mlp.down_proj": {"group_size": 64, "bits": 8},
                            "language_model.model.layers.1.mlp.down_proj": {"bits": 8},
                            "vision_tower.x": {"bits": 3, "group_size": 32}}}
    p = tmp_path / "config.json"
    p.write_text(json.dumps(cfg))
    q = L.parse_quantization(str(p))
    assert q.default == L.QuantizationSpec(4, 64)
    assert L.quantization_for(q, "language_model.model.layers.0.mlp.down_proj") == L.QuantizationSpec(8, 64)
    assert L.quantization_for(q, "language_model.model.layers.1.mlp.down_proj") == L.QuantizationSpec(8, 64)
    assert L.quantization_for(q, "language_model.model.layers.0.mlp.up_proj") == L.QuantizationSpec(4, 64)
    assert "vision_tower.x" not in q.overrides  # only language_model.model.* keys count
    # quantization_config wins over quantization
    q2 = L.parse_quantization({"quantization_config": {"bits": 8, "group_size": 64}, "quantization": {"bits": 4, "group_size": 64}})
    assert q2.default.bits == 8
    for bad in ({"bits": 3, "group_size": 64}, {"bits": 8, "group_size": 32}):
        with pytest.raises(qmm.Gemma4Error):
            L.parse_quantization({"quantization": {"bits": 4, "group_size": 64, "language_model.model.a": bad}})
    with pytest.raises(qmm.Gemma4Error):
        L.parse_quantization({"text_config": {}})


def test_reader_matches_safetensors_library(tmp_path):
    torch = pytest.importorskip("torch")
    from safetensors.torch import save_file

    rng = np.random.default_rng(0)
    w = rng.integers(0, 2**32, (8, 16), dtype=np.uint64).astype(np.uint32)
    f = rng.standard_normal((3, 5)).astype(np.float32)
    bf = torch.randn(4, 6).bfloat16()
    path = tmp_path / "lib.safetensors"
    save_file({"a.weight": torch.from_numpy(w.view(np.int32)), "a.f": torch.from_numpy(f), "a.scales": bf},
              str(path), metadata={"format": "mlx"})
    ck = L.Checkpoint(str(path))
    assert ck.keys() == ["a.f", "a.scales", "a.weight"]
    assert np.array_equal(ck.get("a.weight").view(np.int32), w.view(np.int32))
    assert np.array_equal(ck.get("a.f"), f)
    assert ck.dtype("a.scales") == "BF16"
    assert np.array_equal(ck.get("a.scales"), bf.view(torch.int16).numpy().view(np.uint16))


def test_writer_roundtrip_and_triples(tmp_path):
    from safetensors.torch import load_file

    tri4 = A.quantize(A.round_to_bf16(np.random.default_rng(1).standard_normal((32, 128)).astype(np.float32) * 0.02))
    tri8 = A.quantize(A.round_to_bf16(np.random.default_rng(2).standard_normal((16, 192)).astype(np.float32) * 0.02), bits=8)
    t = {}
    for prefix, (wq, s, b) in (("language_model.model.p4", tri4), ("language_model.model.p8", tri8)):
        t[prefix + ".weight"] = wq
        t[prefix + ".scales"] = ("BF16", s)
        t[prefix + ".biases"] = ("BF16", b)
    t["language_model.model.norm.weight"] = ("BF16", np.zeros(4, np.uint16))
    path = tmp_path / "model.safetensors"
    L.write_safetensors(str(path), t)
    assert sorted(load_file(str(path))) == sorted(t)  # the library reads our file
    ck = L.Checkpoint(str(tmp_path))
    assert ck.quantized_prefixes() == ["language_model.model.p4", "language_model.model.p8"]
    cfg = L.parse_quantization({"quantization": {"bits": 4, "group_size": 64,
                                                 "language_model.model.p8": {"bits": 8, "group_size": 64}}})
    (w, s, b), k = ck.triple("language_model.model.p8", L.quantization_for(cfg, "language_model.model.p8"))
    assert k == 192 and np.array_equal(w, tri8[0]) and np.array_equal(s, tri8[1])
    (w, s, b), k = ck.triple("language_model.model.p4", cfg.default)
    assert k == 128 and np.array_equal(b, tri4[2])
    with pytest.raises(qmm.Gemma4Error):  # wrong spec: scales no longer match
        ck.triple("language_model.model.p8", cfg.default)
