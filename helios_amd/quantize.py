"""Affine quantization into the MLX format the kernels consume.

``quantize(w, group_size=64, bits=4)`` returns ``(w_q, scales, biases)`` like
``mlx.core.quantize(w, group_size, bits)`` in its "affine" mode, the op that produced
the reference's checkpoints (the format is read at native/gemma4_mlx/src/native_model.cc:281-287
and :349-376): codes packed LSB-first into uint32 words along K (8 per word at 4 bits,
4 at 8 bits), one bf16 scale and one bf16 bias per group, w ~ scale * q + bias.

Per group, in fp32: the edge is the extreme value of larger magnitude; the scale is
(max - min) / (2^bits - 1), at least 1e-7, signed so that the edge maps to a whole code
q0 = round(edge / scale); when q0 != 0 the scale is refined to edge / q0 and the bias
is the edge (else the bias is 0); codes are round((w - bias) / scale) clipped to
[0, 2^bits - 1] with the unrounded fp32 scale and bias; scale and bias are stored
rounded to bf16.  Rounding is to nearest even throughout.

Runs wherever ``w`` lives (CPU or GPU tensor); used to build weights for the
benchmark and by callers that quantize their own weights.
"""

from __future__ import annotations

__all__ = ["quantize"]


def quantize(w, group_size: int = 64, bits: int = 4):
    """(w_q int32 [N, K*bits/32], scales bf16 [N, K/group_size], biases bf16 [...]) of a
    float tensor ``w`` [N, K] (any float dtype; computed in fp32)."""
    import torch

    if bits not in (4, 8):
        raise ValueError("bits must be 4 or 8")
    if group_size != 64:
        raise ValueError("group_size must be 64")
    if w.dim() != 2 or w.shape[1] % group_size != 0:
        raise ValueError("w must be [N, K] with K a multiple of the group size")
    n, k = w.shape
    levels = float((1 << bits) - 1)
    g = w.to(torch.float32).reshape(n, k // group_size, group_size)
    w_max = g.amax(dim=2)
    w_min = g.amin(dim=2)
    min_is_edge = w_min.abs() > w_max.abs()
    scale = torch.clamp((w_max - w_min) / levels, min=1e-7)
    scale = torch.where(min_is_edge, scale, -scale)
    edge = torch.where(min_is_edge, w_min, w_max)
    q0 = torch.round(edge / scale)
    refine = q0 != 0
    scale = torch.where(refine, edge / torch.where(refine, q0, torch.ones_like(q0)), scale)
    bias = torch.where(refine, edge, torch.zeros_like(edge))
    q = torch.round((g - bias.unsqueeze(2)) / scale.unsqueeze(2)).clamp_(0.0, levels)
    per_word = 32 // bits
    q = q.reshape(n, k // per_word, per_word).to(torch.int64)
    shifts = torch.arange(per_word, device=w.device, dtype=torch.int64) * bits
    words = (q << shifts).sum(dim=2)  # < 2^32
    words = torch.where(words >= 2**31, words - 2**32, words).to(torch.int32)
    return words.contiguous(), scale.to(torch.bfloat16).contiguous(), bias.to(torch.bfloat16).contiguous()
