"""CPU oracle for MLX-format affine quantized matmul — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
import this module, and only to check results.  The product path
(``helios_amd``) never does.

numpy restatement of what the reference reaches through
``mlx::core::quantize`` / ``dequantize`` / ``quantized_matmul(mode="affine")``:

* ``native/gemma4_mlx/src/native_model.cc:349-362`` — every linear layer is
  ``quantized_matmul(x, w, scales, biases, transpose=true, group_size, bits, "affine")``;
* ``native/gemma4_mlx/src/native_model.cc:1782-1795`` — the lm_head uses the same op;
* ``native/gemma4_mlx/src/native_model.cc:281-287`` — ``K = packed_cols * 32 / bits``;
* ``native/gemma4_mlx/src/native_model.cc:364-376`` — ``dequantize`` of the same triple;
* ``native/gemma4_mlx/src/model_manifest.cc:148`` — group 64 with bits 4 or 8;
* ``scripts/xr54_dequant_assistant.py:103-126`` — ``dequantize(..., dtype=float32)``
  with float32 scales/biases, i.e. ``w = s*q + b`` in fp32;
* ``native/gemma4_mlx/src/native_model.cc:378-386`` — GeGLU (tanh form) feeding down_proj.

The arithmetic itself is MLX 0.31.2's (not vendored in the reference); the
quantize steps restate MLX's published CPU quantize loop.  What pins each
function is listed in ``oracle/q4_oracle.h``; exact MLX bf16 bits for quantize
scales/biases and MLX's own accumulation order stay unpinned (no MLX here).
"""

from __future__ import annotations

import numpy as np

GROUP_SIZE = 64
BITS = 4


# ---------------------------------------------------------------------------
# bf16 helpers (round to nearest even, as the hardware and torch do)
# ---------------------------------------------------------------------------

def f32_to_bf16_bits(a) -> np.ndarray:
    """fp32 -> bf16 bit patterns (uint16), round-to-nearest-even, NaN kept quiet.

    In uint32: u + 0x7FFF + lsb cannot wrap for a finite or infinite u (at most
    0xFF800000 + 0x8000); NaNs, which could, are replaced afterwards."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    r = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    if nan.any():
        r[nan] = ((u[nan] >> np.uint32(16)) | np.uint32(0x40)).astype(np.uint16)
    return r


def f64_to_bf16_bits(a) -> np.ndarray:
    """float64 -> bf16 bit patterns with ONE round-to-nearest-even (going through
    float32 first would round twice: a value just above a bf16 midpoint can land on
    the midpoint in float32 and then tie to even the other way).  Finite values in
    the normal bf16 range."""
    u = np.ascontiguousarray(a, dtype=np.float64).view(np.uint64)
    drop = np.uint64(45)  # 52 - 7 fraction bits
    lsb = (u >> drop) & np.uint64(1)
    r = (u + np.uint64((1 << 44) - 1) + lsb) & ~np.uint64((1 << 45) - 1)
    return (r.view(np.float64).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)


def bf16_bits_to_f32(b) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_to_bf16(a) -> np.ndarray:
    """fp32 values rounded to the nearest bf16, returned as fp32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(a, dtype=np.float32)))


def bf16_ulp(a) -> np.ndarray:
    """Spacing of bf16 numbers at |a| (8 significant bits)."""
    a = np.abs(np.asarray(a, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(a, np.finfo(np.float32).tiny)))
    return np.exp2(e - 7)


# ---------------------------------------------------------------------------
# packing (element c of a row in word c // (32/bits), low bits first)
# ---------------------------------------------------------------------------

def pack(q: np.ndarray, bits: int = BITS) -> np.ndarray:
    """q uint [N, K] with values < 2**bits -> uint32 [N, K*bits/32]."""
    q = np.asarray(q, dtype=np.uint32)
    n, k = q.shape
    per = 32 // bits
    assert k % per == 0
    q = q.reshape(n, k // per, per)
    shifts = (np.arange(per, dtype=np.uint32) * bits).astype(np.uint32)
    return np.bitwise_or.reduce(q << shifts, axis=2).astype(np.uint32)


def unpack(wq: np.ndarray, bits: int = BITS) -> np.ndarray:
    """uint32 [N, W] -> uint8 [N, W*32/bits]."""
    wq = np.asarray(wq, dtype=np.uint32)
    n, w = wq.shape
    per = 32 // bits
    shifts = (np.arange(per, dtype=np.uint32) * bits).astype(np.uint32)
    q = (wq[:, :, None] >> shifts) & np.uint32((1 << bits) - 1)
    return q.reshape(n, w * per).astype(np.uint8)


# ---------------------------------------------------------------------------
# quantize / dequantize / qmm
# ---------------------------------------------------------------------------

def quantize(w: np.ndarray, group_size: int = GROUP_SIZE, bits: int = BITS):
    """MLX affine quantize of fp32 W [N, K] -> (wq uint32, scales bf16 bits, biases bf16 bits).

    Per group (all in fp32): scale = max((max-min)/n_bins, 1e-7); if |min| > |max|
    the edge is min and the scale positive, else the edge is max and the scale
    negative; q0 = rint(edge/scale); when q0 != 0 the scale becomes edge/q0 and the
    bias the edge, else the bias is 0; q = clip(rint((w-bias)/scale), 0, n_bins)
    with the unrounded scale and bias; scale and bias are stored as bf16.
    """
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    assert k % group_size == 0
    n_bins = np.float32((1 << bits) - 1)
    eps = np.float32(1e-7)
    wg = w.reshape(n, k // group_size, group_size)
    w_max = wg.max(axis=-1)
    w_min = wg.min(axis=-1)
    min_is_edge = np.abs(w_min) > np.abs(w_max)
    scale = np.maximum((w_max - w_min) / n_bins, eps).astype(np.float32)
    scale = np.where(min_is_edge, scale, -scale).astype(np.float32)
    edge = np.where(min_is_edge, w_min, w_max).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        q0 = np.rint(edge / scale).astype(np.float32)
        refined = (edge / np.where(q0 != 0, q0, np.float32(1))).astype(np.float32)
    scale = np.where(q0 != 0, refined, scale).astype(np.float32)
    bias = np.where(q0 != 0, edge, np.float32(0)).astype(np.float32)
    q = np.rint((wg - bias[..., None]) / scale[..., None]).astype(np.float32)
    q = np.clip(q, np.float32(0), n_bins).astype(np.uint32).reshape(n, k)
    return pack(q, bits), f32_to_bf16_bits(scale), f32_to_bf16_bits(bias)


def dequantize(wq, scales, biases, group_size: int = GROUP_SIZE, bits: int = BITS) -> np.ndarray:
    """fp32 W [N, K] = s*q + b.  s*q is exact in fp32 (8-bit significand times a
    value < 2**bits), so the single rounding of the add makes this unique."""
    q = unpack(wq, bits).astype(np.float32)
    n, k = q.shape
    s = bf16_bits_to_f32(scales).reshape(n, k // group_size, 1)
    b = bf16_bits_to_f32(biases).reshape(n, k // group_size, 1)
    return (s * q.reshape(n, k // group_size, group_size) + b).astype(np.float32).reshape(n, k)


def dequantize_f64(wq, scales, biases, group_size: int = GROUP_SIZE, bits: int = BITS) -> np.ndarray:
    """Exact affine weights s*q + b in float64."""
    q = unpack(wq, bits).astype(np.float64)
    n, k = q.shape
    s = bf16_bits_to_f32(scales).astype(np.float64).reshape(n, k // group_size, 1)
    b = bf16_bits_to_f32(biases).astype(np.float64).reshape(n, k // group_size, 1)
    return (s * q.reshape(n, k // group_size, group_size) + b).reshape(n, k)


def qmm_f64(x_bits, wq, scales, biases, group_size: int = GROUP_SIZE, bits: int = BITS) -> np.ndarray:
    """y = x · Wᵀ (transpose=true) with x bf16 bits [M, K]; float64 accumulation of
    exact products; the caller rounds once to the output dtype."""
    x = bf16_bits_to_f32(x_bits).astype(np.float64)
    w = dequantize_f64(wq, scales, biases, group_size, bits)
    return x @ w.T


# ---------------------------------------------------------------------------
# tolerance checks (the acceptance bounds, applied beyond the output format's own rounding)
# ---------------------------------------------------------------------------

def check_bf16_output(y_bits, y_exact, rel: float = 1e-2):
    """bf16 output: max |y - y_exact| <= rel * RMS(y_exact) + ulp_bf16(y_exact)/2.

    The half-ulp term is the error that rounding the exact value to bf16 already
    makes; no bf16 output can avoid it.  Returns (ok, worst_excess_over_rms)."""
    y = bf16_bits_to_f32(y_bits).astype(np.float64)
    y_exact = np.asarray(y_exact, dtype=np.float64)
    rms = float(np.sqrt(np.mean(y_exact ** 2))) if y_exact.size else 0.0
    excess = np.abs(y - y_exact) - 0.5 * bf16_ulp(y_exact)
    worst = float(excess.max()) if excess.size else 0.0
    bound = rel * rms
    return worst <= bound + 1e-30, (worst / rms if rms > 0 else worst)


def check_bf16_rounding(y_bits, y_exact, acc_rel: float = 1e-4):
    """The tighter property of a bf16 output computed by fp32 accumulation of exact
    products: each output is the round-to-nearest-even of some value within
    acc_rel * RMS(y_exact) of the exact result, i.e.
        |y - y_exact| <= ulp_bf16(y)/2 + acc_rel * RMS(y_exact)
    (values that round to y lie within half an ulp of y, also at a binade edge).
    Wherever the accumulation error stays below the distance to the nearest
    rounding boundary, y equals RNE(y_exact) exactly.  Returns (ok, worst excess
    over ulp(y)/2 as a fraction of RMS, fraction of outputs equal to RNE(y_exact))."""
    y_bits = np.asarray(y_bits, dtype=np.uint16)
    y = bf16_bits_to_f32(y_bits).astype(np.float64)
    y_exact = np.asarray(y_exact, dtype=np.float64)
    if not y.size:
        return True, 0.0, 1.0
    rms = float(np.sqrt(np.mean(y_exact ** 2)))
    excess = np.abs(y - y_exact) - 0.5 * bf16_ulp(y)
    worst = float(excess.max())
    equal = float(np.mean(f64_to_bf16_bits(y_exact) == y_bits))
    return worst <= acc_rel * rms + 1e-30, (worst / rms if rms > 0 else worst), equal


def check_f32_output(y, y_exact, rel: float = 2e-3):
    """fp32 output: max |y - y_exact| <= rel * RMS(y_exact).  Returns (ok, max_err/rms)."""
    y = np.asarray(y, dtype=np.float64)
    y_exact = np.asarray(y_exact, dtype=np.float64)
    rms = float(np.sqrt(np.mean(y_exact ** 2))) if y_exact.size else 0.0
    err = float(np.abs(y - y_exact).max()) if y.size else 0.0
    return err <= rel * rms + 1e-30, (err / rms if rms > 0 else err)


# ---------------------------------------------------------------------------
# synthetic inputs for the benchmark configurations (seeded, byte-identical CPU/GPU)
# ---------------------------------------------------------------------------

def make_weights(n: int, k: int, seed: int, std: float = 0.02, group_size: int = GROUP_SIZE,
                 bits: int = BITS, chunk_rows: int = 8192):
    """W ~ N(0, std) in fp32, rounded to bf16 (how bf16 checkpoints arise), then quantized.

    Generated and quantized `chunk_rows` rows at a time (quantization is per row, and
    the generator's stream continues across calls), which bounds the temporaries of a
    262144-row weight; the result equals one whole-matrix pass."""
    rng = np.random.Generator(np.random.PCG64(seed))
    wq = np.empty((n, k * bits // 32), np.uint32)
    s = np.empty((n, k // group_size), np.uint16)
    b = np.empty((n, k // group_size), np.uint16)
    for r0 in range(0, n, chunk_rows):
        r1 = min(n, r0 + chunk_rows)
        w = rng.standard_normal((r1 - r0, k), dtype=np.float32) * np.float32(std)
        wq[r0:r1], s[r0:r1], b[r0:r1] = quantize(round_to_bf16(w), group_size, bits)
    return wq, s, b


def make_activations(m: int, k: int, seed: int, outliers: bool = False) -> np.ndarray:
    """bf16 bits of x ~ N(0,1); with ``outliers`` 1% of entries are scaled by 20."""
    rng = np.random.Generator(np.random.PCG64(seed))
    x = rng.standard_normal((m, k), dtype=np.float32)
    if outliers:
        x = np.where(rng.random((m, k)) < 0.01, x * np.float32(20), x).astype(np.float32)
    return f32_to_bf16_bits(x)


# GeGLU constants of native_model.cc:379-380 (model_scalar makes them bf16 in the bf16
# model dtype, native_model.cc:342-347)
GEGLU_C_TANH = 0.7978845608028654
GEGLU_C_CUBIC = 0.044715


def geglu_ops(gate, up, bf16: bool) -> np.ndarray:
    """GeGLU of native_model.cc:378-386 evaluated op by op as the reference's array
    ops do: gelu = (0.5 * g) * (1 + tanh(c1 * (g + c2 * g**3))), h = gelu * up.

    Each op is one float32 operation.  With ``bf16`` (the model dtype) the inputs,
    the constants and every intermediate are bf16, so each op's result is rounded to
    bf16; otherwise (the float32 override, native_model.cc:330-347) all stay float32.
    ``g**3`` is ``g*g*g`` (exact in float32 for bf16 g).  Returns float32 values
    (bf16-representable when ``bf16``)."""
    f32 = np.float32
    g = np.asarray(gate, dtype=np.float32)
    u = np.asarray(up, dtype=np.float32)
    r = round_to_bf16 if bf16 else (lambda v: np.asarray(v, dtype=np.float32))
    c_tanh, c_cubic = r(f32(GEGLU_C_TANH)), r(f32(GEGLU_C_CUBIC))
    g, u = r(g), r(u)
    with np.errstate(over="ignore"):  # g**3 past the float32 range is inf, as in the reference's ops
        g3 = r(g * g * g)
        a = r(g + r(c_cubic * g3))
        t = r(np.tanh(r(c_tanh * a)))
        gelu = r(r(f32(0.5) * g) * r(f32(1.0) + t))
        return r(gelu * u)


def gelu_tanh_times(gate_bits, up_bits) -> np.ndarray:
    """bf16 GeGLU of bf16 gate/up bit patterns (``geglu_ops`` in the bf16 model
    dtype), as bf16 bits: the down_proj input of the prefill chain."""
    return f32_to_bf16_bits(geglu_ops(bf16_bits_to_f32(gate_bits), bf16_bits_to_f32(up_bits), bf16=True))


# lm_head final-logit softcap (native_model.cc:1794): tanh(logits / 30) * 30
LOGIT_SOFTCAP = 30.0


def softcap_ops(logits, cap: float = LOGIT_SOFTCAP, bf16: bool = True) -> np.ndarray:
    """The reference's softcap op by op: model_dtype(tanh(logits / cap) * cap).  With
    ``bf16`` the logits (the qmm output in the model dtype), the constant and each
    op's result are bf16-rounded; otherwise all are float32.  ``cap == 0`` returns the
    (rounded) logits unchanged.  Returns float32."""
    r = round_to_bf16 if bf16 else (lambda v: np.asarray(v, dtype=np.float32))
    l = r(np.asarray(logits, dtype=np.float32))
    if cap == 0:
        return l
    c = r(np.float32(cap))
    return r(r(np.tanh(r(l / c))) * c)


def greedy(values) -> tuple:
    """argmax along the last axis (the first maximum, as mlx::core::argmax and
    np.argmax return it) and the maximum itself."""
    v = np.asarray(values, dtype=np.float32)
    idx = np.argmax(v, axis=-1)
    return idx.astype(np.int32), np.take_along_axis(v, idx[..., None], axis=-1)[..., 0]


def lora_ops(x_bits, a, b, scale: float, base, bf16: bool = True) -> np.ndarray:
    """add_lora_delta_if_active (native_model.cc:316-328) on a base output:
    model_dtype(base + model_dtype((float32(x) @ A.T) @ B.T * scale)).  The two fp32
    products are accumulated in float64 and rounded once to fp32 (an fp32 matmul's
    own order is not pinned); with ``bf16`` the scale (model_scalar), base and delta
    are bf16 and the sum is rounded to bf16.  Returns float32."""
    x = bf16_bits_to_f32(x_bits).astype(np.float64)
    t = (x @ np.asarray(a, np.float64).T).astype(np.float32)
    d = (t.astype(np.float64) @ np.asarray(b, np.float64).T).astype(np.float32)
    if bf16:
        sc = round_to_bf16(np.float32(scale))
        delta = round_to_bf16(d * sc)
        return round_to_bf16(round_to_bf16(np.asarray(base, np.float32)) + delta)
    return (np.asarray(base, np.float32) + d * np.float32(scale)).astype(np.float32)
