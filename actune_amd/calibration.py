"""Layer calibration on the HIP backend.

Same contract as actune/calibration.py:7-16 and :42-93:

* ``activation_reference(value, bits, group_size=64)`` returns the group-64
  dequantized activations codes * scale. The codes and scales come from the
  library's group-64 quantizer (the exact codebook of inference); the
  product codes * scale is the same fp32 multiply the reference performs.
* ``calibrate_linear(linear, inputs, row_weights=None, *, budget, group_size,
  clip_grid)`` fits the activation-guided channel scale (5 alphas), then the
  per-row clip ratio of every weight version over the clip grid, and the
  weighted error per (W, A) pair. Every candidate output is evaluated by the
  inference kernels themselves: x / scale quantized by the group-64
  quantizer and multiplied by the packed candidate weights in the packed
  GEMM, with fp32 output. The reference evaluates the same quantized
  operands with a float GEMM (F.linear of dequantized activations and
  weights); both are fp32 evaluations of the same exact sums, so scores
  differ only in the last bits and the selected scale and clips agree except
  on exact near-ties.
* Weight codebooks are evaluated with torch on the layer's device, as the
  reference does (quantizers.py:23-94): on a GPU the divisions by the
  constants 7 and 127 are reciprocal multiplies there as well.

Calibration runs on the GPU only: CPU tensors raise ValueError (the
reference's own module remains the CPU path). jacobian_row_weights, the
RNG-driven Hutchinson estimate (calibration.py:19-39), stays with the
reference's offline tooling.
"""
from __future__ import annotations

import torch

from . import _native
from .kernels.grouped import pack_rows

_CLIP_GRID = (1., .975, .95, .925, .9, .875, .85, .8, .75)


def _require_gpu(t, what):
    if not t.is_cuda:
        raise ValueError(f"{what}: the HIP calibration path needs CUDA tensors")


def _unpack_codes(packed, bits, k):
    """u8 [M, K*bits/8] -> int8 codes [M, K] (code j of byte b at bits (j*bits))."""
    if bits == 8:
        return packed.view(torch.int8)
    per = 8 // bits
    fields = [(packed >> (j * bits)) & ((1 << bits) - 1) for j in range(per)]
    u = torch.stack(fields, dim=-1).reshape(packed.shape[0], k).to(torch.int16)
    half = 1 << (bits - 1)
    return ((u ^ half) - half).to(torch.int8)


def activation_reference(value, bits, group_size=64):
    """The exact symmetric group-64 codebook used by inference, dequantized
    (calibration.py:7-16)."""
    if bits not in (2, 4, 8) or value.shape[-1] % group_size:
        raise ValueError("Unsupported activation width or unaligned input")
    if group_size != 64:
        raise ValueError("the HIP backend quantizes groups of 64")
    _require_gpu(value, "activation_reference")
    shape = value.shape
    flat = value.reshape(-1, shape[-1]).contiguous()
    packed, scales = _native.quantize_groups(flat, bits)
    codes = _unpack_codes(packed, bits, shape[-1]).float()
    deq = codes.reshape(flat.shape[0], -1, 64) * scales[:, :, None]
    return deq.reshape(shape)


def _clip(weight_rows, ratio):
    return weight_rows if ratio is None else weight_rows * ratio


def _codes_on_device(weight, w, a, ratio):
    """weight_codes (quantizers.py:23-94) evaluated by torch on the weight's
    device; ratio is a float in (0, 1] or None."""
    value = weight.detach().float()
    amax = value.abs().amax(dim=1).clamp_min(1e-8)
    if w == 8 and a != 4:
        scale = amax / 127.0
        return (value / scale[:, None]).round().clamp(-128, 127).to(torch.int8), scale
    amax = _clip(amax, ratio)
    if w == 2:
        return (value / amax[:, None]).round().clamp(-2, 1).to(torch.int8), amax
    scale4 = amax / 7.0
    q4 = (value / scale4[:, None]).round().clamp(-8, 7).to(torch.int8)
    if w == 4:
        return q4, scale4
    residual = (16.0 * (value / scale4[:, None] - q4.float())).round().clamp(-8, 7).to(torch.int16)
    q4i = q4.to(torch.int16)
    residual = torch.minimum(torch.maximum(residual, (-128 - 16 * q4i).clamp_min(-8)), (127 - 16 * q4i).clamp_max(7))
    return (16 * q4i + residual).to(torch.int8), scale4 / 16.0


def _candidate(x_scaled, weight, w, a, ratio):
    """fp32 output of the packed GEMM for x_scaled (already divided by the
    channel scale, in the layer dtype) against weight codes (w, a, ratio)."""
    codes, scale = _codes_on_device(weight, w, a, ratio)
    packed = pack_rows(codes, w)
    a_packed, a_scales = _native.quantize_groups(x_scaled, a)
    return _native.grouped_linear(a_packed, a_scales, packed, scale.contiguous(), None,
                                  tuple(x_scaled.shape), w, a, out_dtype=torch.float32)


@torch.no_grad()
def calibrate_linear(linear, inputs, row_weights=None, *, budget="w4a4", group_size=64, clip_grid=_CLIP_GRID):
    """Fit activation-guided scales, row clips and weighted errors per pair
    (calibration.py:42-93), with every candidate evaluated by the inference
    quantizer and packed GEMM."""
    if budget not in ("w4a4", "w4a8"):
        raise ValueError("Unknown precision budget")
    x = inputs.detach().reshape(-1, linear.in_features).to(linear.weight.device, linear.weight.dtype)
    if not len(x) or not torch.isfinite(x).all() or linear.in_features % group_size:
        raise ValueError("Nonempty finite aligned fitting inputs required")
    if group_size != 64:
        raise ValueError("the HIP backend quantizes groups of 64")
    _require_gpu(x, "calibrate_linear")
    gains = torch.ones(linear.out_features, device=x.device) if row_weights is None \
        else row_weights.to(x.device).float()
    if gains.shape != (linear.out_features,) or not torch.isfinite(gains).all() or (gains < 0).any():
        raise ValueError("Invalid action-Jacobian weights")
    if not bool(gains.sum()):
        gains = torch.ones_like(gains)
    reference = torch.nn.functional.linear(x.float(), linear.weight.float())
    base_a = 4 if budget == "w4a4" else 8
    moment = x.float().abs().mean(0).clamp_min(1e-4)
    best = None
    for alpha in (0., .25, .5, .75, 1.):
        scale = moment.pow(alpha)
        scale = (scale / (scale.max() * scale.min()).sqrt()).clamp(1 / 16, 16).to(x.dtype)
        weight = (linear.weight * scale[None, :]).to(x.dtype)
        y = _candidate((x / scale).contiguous(), weight, 4, base_a, None)
        score = float(((y - reference).square().mean(0) * gains).sum())
        if best is None or score < best[0]:
            best = score, scale
    scale = best[1]
    weight = (linear.weight * scale[None, :]).to(x.dtype)
    x_scaled = (x / scale).contiguous()
    errors, clips = {}, {}
    for w in (2, 4, 8):
        for a in ((8,) if budget == "w4a8" else (2, 4, 8)):
            row_error = torch.full((linear.out_features,), float("inf"), device=x.device)
            selected = torch.ones_like(row_error)
            for ratio in clip_grid:
                if not 0 < ratio <= 1:
                    raise ValueError("Clip ratios must lie in (0, 1]")
                output = _candidate(x_scaled, weight, w, a, ratio)
                loss = (output - reference).square().mean(0)
                improve = loss < row_error
                selected[improve], row_error[improve] = ratio, loss[improve]
            mode = f"w{w}a{a}"
            errors[mode] = float((row_error * gains).sum())
            clips[mode] = selected
    return dict(channel_scale=scale, clips=clips, errors=errors, group_size=group_size)
