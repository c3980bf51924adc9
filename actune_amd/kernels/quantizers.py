"""Per-output-row weight codebooks (install time).

Same codebooks as actune/kernels/quantizers.py:4-94: signed W2 {-2..1} with
scale amax*r, signed W4 {-8..7} with scale amax*r/7, the nested W8 code
16*q4 + r4 used with A4 activations (scale s4/16), and plain W8 with scale
amax/127 (clip ratios ignored). amax is clamped to >= 1e-8.

Arithmetic is done in fp32 on the CPU. Every tensor/tensor division is the
IEEE quotient on either device; the divisions by the constants 7 and 127 are
the IEEE quotient by default and, with ``gpu_division``, a multiply by the
fp32 reciprocal, which is what torch computes for a GPU tensor divided by a
Python scalar. Callers pass ``gpu_division=weight.is_cuda`` to get the codes
the reference computes on the layer's own device. The resulting codes and
scales are returned on the weight's device. This runs once per (layer, mode)
at install time; the per-call path is the HIP library.
"""
from __future__ import annotations

import torch


def _validate_clip_ratios(clip_ratios, *, out_features, device):
    """Scalar or per-row clip ratios in (0, 1] as a contiguous fp32 vector
    (quantizers.py:4-21; same messages)."""
    ratio = torch.as_tensor(clip_ratios, dtype=torch.float32, device=device).reshape(-1)
    if ratio.numel() == 1:
        ratio = ratio.expand(out_features)
    if ratio.numel() != out_features:
        raise ValueError(f"expected {out_features} AWQ-style clip ratios, got {ratio.numel()}")
    if not bool(torch.isfinite(ratio).all()):
        raise ValueError("AWQ-style clip ratios must be finite")
    if not bool(((ratio > 0.0) & (ratio <= 1.0)).all()):
        raise ValueError("AWQ-style clip ratios must lie in (0, 1]")
    return ratio.contiguous()


def _fp32_cpu(weight):
    return weight.detach().to(device="cpu", dtype=torch.float32)


def _clipped_absmax(value, clip_ratios):
    amax = value.abs().amax(dim=1).clamp_min(1e-8)
    if clip_ratios is None:
        return amax
    return amax * _validate_clip_ratios(clip_ratios, out_features=value.shape[0], device=value.device)


def _div_const(value, constant, gpu_division):
    """value / constant in fp32: the IEEE quotient (torch-CPU), or, with
    gpu_division, value times the fp32 reciprocal 1.0f / constant, which is
    what torch computes for a GPU tensor divided by a Python scalar (the
    reference's own note, w4a8_triton.py:33-36)."""
    if not gpu_division:
        return value / constant
    reciprocal = torch.tensor(1.0, dtype=torch.float32) / constant
    return value * reciprocal


def _round_clamp(value, scale, lo, hi):
    """rint_half_even(value / scale[:, None]) clamped to [lo, hi], as int8."""
    return torch.clamp(torch.round(value / scale[:, None]), lo, hi).to(torch.int8)


def symmetric_int4_quantize(weight, *, clip_ratios=None, gpu_division=False):
    """W4 codes in [-8, 7] and the row scale (amax * r) / 7."""
    value = _fp32_cpu(weight)
    scale = _div_const(_clipped_absmax(value, clip_ratios), 7.0, gpu_division)
    codes = _round_clamp(value, scale, -8, 7)
    return codes.to(weight.device), scale.contiguous().to(weight.device)


def signed_r4_refine(weight, q4, scale4):
    """Signed residual r4 in [-8, 7] on top of q4 and the nested int8 code
    16*q4 + r4, with r4 bounded so the code stays in [-128, 127]."""
    value = _fp32_cpu(weight)
    q4c = q4.detach().to("cpu")
    s4 = scale4.detach().to("cpu", torch.float32)
    base = q4c.to(torch.int16)
    # 16 * (fl(v / s4) - q4): the subtraction rounds, the power-of-two product is exact
    res = torch.clamp(torch.round(16.0 * (value / s4[:, None] - q4c.float())), -8, 7).to(torch.int16)
    low = torch.clamp(-128 - 16 * base, min=-8)
    high = torch.clamp(127 - 16 * base, max=7)
    res = torch.minimum(torch.maximum(res, low), high)
    nested = (16 * base + res).to(torch.int8)
    return res.to(torch.int8).to(q4.device), nested.to(q4.device)


def symmetric_int2_quantize(weight, *, clip_ratios=None):
    """W2 codes in [-2, 1] and the row scale amax * r."""
    value = _fp32_cpu(weight)
    scale = _clipped_absmax(value, clip_ratios)
    codes = _round_clamp(value, scale, -2, 1)
    return codes.to(weight.device), scale.contiguous().to(weight.device)


def weight_codes(weight, w, a, *, clip_ratios=None, gpu_division=False):
    """(int8 codes [N, K], fp32 scale [N]) for weight width w used with
    activation width a (quantizers.py:83-94). gpu_division: divide by the
    constants 7 and 127 as torch does on a GPU (see _div_const); every
    module (group-64 and tokenwise) passes the device of the layer it is
    built from, as the reference evaluates these formulas there."""
    if w == 2:
        return symmetric_int2_quantize(weight, clip_ratios=clip_ratios)
    if w == 4:
        return symmetric_int4_quantize(weight, clip_ratios=clip_ratios, gpu_division=gpu_division)
    if a == 4:
        q4, s4 = symmetric_int4_quantize(weight, clip_ratios=clip_ratios, gpu_division=gpu_division)
        _, nested = signed_r4_refine(weight, q4, s4)
        return nested, s4 / 16.0
    value = _fp32_cpu(weight)
    scale = _div_const(value.abs().amax(dim=1).clamp_min(1e-8), 127.0, gpu_division)
    codes = _round_clamp(value, scale, -128, 127)
    return codes.to(weight.device), scale.to(weight.device)
