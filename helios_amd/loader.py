"""Loading MLX-format quantized checkpoints into resident handles.

The reference reads a model directory's ``config.json`` and every ``*.safetensors``
file in it (sorted, ``native/gemma4_mlx/src/native_model.cc:118-130``, ``:3550-3566``)
and keeps each quantized projection as the triple ``<prefix>.weight`` (uint32 packed
codes), ``<prefix>.scales`` and ``<prefix>.biases`` (bf16).  The quantization spec of
a prefix is the config's per-prefix override when there is one, else the default
(``native_model.cc:208-215``); the config's ``quantization`` (or
``quantization_config``) object carries the default ``bits``/``group_size`` and
overrides keyed by ``language_model.model.*`` prefixes, which may only be group 64
with 4 or 8 bits (``model_manifest.cc:101-162``, ``:188-192``).  K follows from the
packed width, ``K = weight.shape[1] * 32 / bits`` (``native_model.cc:281-287``).

This module mirrors that: :func:`parse_quantization`, :func:`quantization_for`,
:class:`Checkpoint` (a safetensors reader that maps the files and executes nothing
from them), :func:`load_linear` / :func:`load_geglu_pair` (handles on the current
device), :func:`load_lora_adapter` (the LoRA modules of an adapter directory,
``native_model.cc:3300-3440``) and :func:`write_safetensors` (for fixtures).
"""

from __future__ import annotations

import dataclasses
import glob
import json
import os
import struct

import numpy as np

from . import qmm

# safetensors dtype -> numpy dtype of the raw elements (bf16 / f16 stay 16-bit patterns)
_DTYPES = {
    "U8": np.uint8, "I8": np.int8, "U16": np.uint16, "I16": np.int16, "U32": np.uint32, "I32": np.int32,
    "U64": np.uint64, "I64": np.int64, "F32": np.float32, "F64": np.float64, "BF16": np.uint16, "F16": np.uint16,
    "BOOL": np.bool_,
}
_NAMES = {np.dtype(np.uint32): "U32", np.dtype(np.int32): "I32", np.dtype(np.float32): "F32",
          np.dtype(np.uint8): "U8", np.dtype(np.int64): "I64", np.dtype(np.float64): "F64"}


@dataclasses.dataclass(frozen=True)
class QuantizationSpec:
    """bits and group size of one quantized projection (model_manifest.h:10-13)."""

    bits: int
    group_size: int


@dataclasses.dataclass
class QuantizationConfig:
    default: QuantizationSpec
    overrides: dict


def parse_quantization(config) -> QuantizationConfig:
    """The quantization block of a config.json (a dict, or a path to the file)."""
    if isinstance(config, (str, os.PathLike)):
        with open(config) as f:
            config = json.load(f)
    block = config.get("quantization_config", config.get("quantization"))
    if not isinstance(block, dict) or "bits" not in block or "group_size" not in block:
        raise qmm.Gemma4Error(qmm.Status.MODEL_LOAD, "config.json is missing quantization bits/group_size")
    default = QuantizationSpec(int(block["bits"]), int(block["group_size"]))
    overrides = {}
    for key, value in block.items():
        if not key.startswith("language_model.model.") or not isinstance(value, dict) or "bits" not in value:
            continue
        spec = QuantizationSpec(int(value["bits"]), int(value.get("group_size", default.group_size)))
        if spec.group_size != 64 or spec.bits not in (4, 8):
            raise qmm.Gemma4Error(qmm.Status.MODEL_LOAD, f"unsupported quantization override for {key}")
        overrides[key] = spec
    return QuantizationConfig(default, overrides)


def quantization_for(config: QuantizationConfig, prefix: str) -> QuantizationSpec:
    return config.overrides.get(prefix, config.default)


class Checkpoint:
    """The tensors of one or more safetensors files (a model directory's files in
    sorted order, or explicit paths).  Arrays are memory-mapped read-only and copied
    on access; bf16 comes back as uint16 bit patterns."""

    def __init__(self, paths):
        if isinstance(paths, (str, os.PathLike)) and os.path.isdir(paths):
            paths = sorted(glob.glob(os.path.join(paths, "*.safetensors")))
        elif isinstance(paths, (str, os.PathLike)):
            paths = [paths]
        self.index = {}  # name -> (path, dtype string, shape, begin, end)
        for path in paths:
            with open(path, "rb") as f:
                (hlen,) = struct.unpack("<Q", f.read(8))
                if hlen > 100 << 20:
                    raise qmm.Gemma4Error(qmm.Status.MODEL_LOAD, f"{path}: implausible safetensors header")
                header = json.loads(f.read(hlen))
            base = 8 + hlen
            for name, meta in header.items():
                if name == "__metadata__":
                    continue
                if meta["dtype"] not in _DTYPES:
                    raise qmm.Gemma4Error(qmm.Status.MODEL_LOAD, f"{path}: {name} has unsupported dtype {meta['dtype']}")
                begin, end = meta["data_offsets"]
                self.index[name] = (str(path), meta["dtype"], tuple(meta["shape"]), base + begin, base + end)

    def keys(self):
        return sorted(self.index)

    def dtype(self, name: str) -> str:
        return self.index[name][1]

    def get(self, name: str) -> np.ndarray:
        if name not in self.index:
            raise qmm.Gemma4Error(qmm.Status.MODEL_LOAD, f"missing loaded tensor {name}")
        path, dt, shape, begin, end = self.index[name]
        np_dt = np.dtype(_DTYPES[dt])
        count = int(np.prod(shape)) if shape else 1
        if end - begin != count * np_dt.itemsize:
            raise qmm.Gemma4Error(qmm.Status.MODEL_LOAD, f"{path}: {name} byte range does not match its shape")
        mm = np.memmap(path, dtype=np_dt, mode="r", offset=begin, shape=(count,))
        return np.array(mm).reshape(shape)

    def quantized_prefixes(self):
        """Prefixes with a weight, scales and biases triple (the quantized linears)."""
        names = set(self.index)
        return sorted(n[: -len(".weight")] for n in names
                      if n.endswith(".weight") and n[: -len(".weight")] + ".scales" in names
                      and n[: -len(".weight")] + ".biases" in names)

    def triple(self, prefix: str, spec: QuantizationSpec):
        """(weight uint32 [N, K*bits/32], scales, biases bf16 bits [N, K/g]) with the
        shapes checked against the spec; returns the triple and K."""
        w = self.get(prefix + ".weight")
        s = self.get(prefix + ".scales")
        b = self.get(prefix + ".biases")
        if self.dtype(prefix + ".weight") != "U32" or self.dtype(prefix + ".scales") != "BF16" or \
                self.dtype(prefix + ".biases") != "BF16":
            raise qmm.Gemma4Error(qmm.Status.MODEL_LOAD, f"{prefix}: expected uint32 weight and bf16 scales/biases")
        if w.ndim != 2 or s.ndim != 2:
            raise qmm.Gemma4Error(qmm.Status.MODEL_LOAD, f"{prefix}: expected 2-d tensors")
        k = w.shape[1] * 32 // spec.bits
        if s.shape != (w.shape[0], k // spec.group_size) or b.shape != s.shape:
            raise qmm.Gemma4Error(qmm.Status.MODEL_LOAD,
                                  f"{prefix}: scales/biases {s.shape} do not match weight {w.shape} at "
                                  f"bits={spec.bits} group_size={spec.group_size}")
        return (w, s, b), k


def load_linear(ckpt: Checkpoint, config: QuantizationConfig, prefix: str) -> qmm.QuantizedLinear:
    """The projection `prefix` as a resident handle on the current device."""
    spec = quantization_for(config, prefix)
    tri, _ = ckpt.triple(prefix, spec)
    return qmm.QuantizedLinear(*tri, group_size=spec.group_size, bits=spec.bits)


def load_geglu_pair(ckpt: Checkpoint, config: QuantizationConfig, mlp_prefix: str) -> qmm.QuantizedGeGLU:
    """`<mlp_prefix>.gate_proj` and `.up_proj` as one GeGLU pair (both must share a spec)."""
    gp, up = mlp_prefix + ".gate_proj", mlp_prefix + ".up_proj"
    sg, su = quantization_for(config, gp), quantization_for(config, up)
    if sg != su:
        raise qmm.Gemma4Error(qmm.Status.UNSUPPORTED_CONFIG, f"{mlp_prefix}: gate and up are quantized differently")
    tg, _ = ckpt.triple(gp, sg)
    tu, _ = ckpt.triple(up, su)
    return qmm.QuantizedGeGLU(tg, tu, group_size=sg.group_size, bits=sg.bits)


def write_safetensors(path: str, tensors: dict, metadata: dict | None = None) -> None:
    """Writes tensors {name: array or ("BF16", uint16 array)} as one safetensors file."""
    header, blobs, off = {}, [], 0
    for name in sorted(tensors):
        v = tensors[name]
        dt, arr = (v[0], np.ascontiguousarray(v[1])) if isinstance(v, tuple) else (None, np.ascontiguousarray(v))
        dt = dt or _NAMES[arr.dtype]
        raw = arr.tobytes()
        header[name] = {"dtype": dt, "shape": list(arr.shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    if metadata:
        header["__metadata__"] = {str(k): str(v) for k, v in metadata.items()}
    h = json.dumps(header, separators=(",", ":")).encode()
    h += b" " * ((8 - len(h) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for raw in blobs:
            f.write(raw)


# ---------------------------------------------------------------------------
# LoRA adapters (native_model.cc:225-288, :3300-3440)
# ---------------------------------------------------------------------------

def canonical_lora_prefix(prefix: str) -> str:
    """PEFT names -> the base model's tensor prefixes (native_model.cc:237-248)."""
    for head in ("base_model.model.model.", "base_model.model.", "model."):
        if prefix.startswith(head):
            return "language_model.model." + prefix[len(head):]
    return prefix


def target_module_allowed(prefix: str, target_modules) -> bool:
    """The leaf name, the whole prefix or a dotted suffix matches (native_model.cc:267-279)."""
    leaf = prefix.rsplit(".", 1)[-1]
    for module in target_modules:
        t = module.strip()
        if t and (leaf == t or prefix == t or prefix.endswith("." + t)):
            return True
    return False


def load_lora_adapter(adapter_path: str, rank: int, alpha: float, target_modules, ckpt: Checkpoint,
                      config: QuantizationConfig) -> dict:
    """{prefix: LoraAdapter} from <adapter_path>/adapter_model.safetensors, checked
    against the base checkpoint the way the reference checks them: lora_A [rank, K]
    and lora_B [N, rank] for a quantized projection that exists, K from its packed
    width; scale = alpha / rank."""
    if rank <= 0:
        raise qmm.Gemma4Error(qmm.Status.ADAPTER, "LoRA rank must be greater than zero")
    if not (alpha > 0 and np.isfinite(alpha)):
        raise qmm.Gemma4Error(qmm.Status.ADAPTER, "LoRA alpha must be finite and positive")
    if not target_modules:
        raise qmm.Gemma4Error(qmm.Status.ADAPTER, "LoRA target_modules must not be empty")
    path = os.path.join(adapter_path, "adapter_model.safetensors")
    if not os.path.exists(path):
        raise qmm.Gemma4Error(qmm.Status.ADAPTER, f"adapter_model.safetensors not found at {path}")
    ad = Checkpoint(path)
    lora_a, lora_b = {}, {}
    for name in ad.keys():
        for suffix, dst in ((".lora_A.weight", lora_a), (".lora_B.weight", lora_b)):
            if name.endswith(suffix):
                prefix = canonical_lora_prefix(name[: -len(suffix)])
                if target_module_allowed(prefix, target_modules):
                    dst[prefix] = name
    scale = np.float32(alpha) / np.float32(rank)
    out = {}
    for prefix, a_name in sorted(lora_a.items()):
        if prefix not in lora_b:
            raise qmm.Gemma4Error(qmm.Status.ADAPTER, f"missing lora_B tensor for {prefix}")
        if prefix + ".weight" not in ckpt.index:
            raise qmm.Gemma4Error(qmm.Status.ADAPTER, f"adapter target module does not exist in native model: {prefix}")
        a = _as_float32(ad, a_name)
        b = _as_float32(ad, lora_b[prefix])
        spec = quantization_for(config, prefix)
        w_shape = ckpt.index[prefix + ".weight"][2]
        k = w_shape[1] * (32 // spec.bits)
        if a.shape != (rank, k) or b.shape != (w_shape[0], rank):
            raise qmm.Gemma4Error(qmm.Status.ADAPTER,
                                  f"LoRA shape mismatch for {prefix}: A={list(a.shape)} B={list(b.shape)} "
                                  f"expected A=[{rank},{k}] B=[{w_shape[0]},{rank}]")
        out[prefix] = qmm.LoraAdapter(a, b, float(scale))
    if not out:
        raise qmm.Gemma4Error(qmm.Status.ADAPTER, "adapter contains no supported LoRA tensor pairs for requested "
                                                  "target_modules")
    return out


def _as_float32(ck: Checkpoint, name: str) -> np.ndarray:
    dt = ck.dtype(name)
    v = ck.get(name)
    if dt == "BF16":
        return (v.astype(np.uint32) << 16).view(np.float32)
    if dt == "F16":
        return v.view(np.float16).astype(np.float32)
    if dt in ("F32", "F64"):
        return v.astype(np.float32)
    raise qmm.Gemma4Error(qmm.Status.ADAPTER, f"{name}: unsupported LoRA dtype {dt}")
