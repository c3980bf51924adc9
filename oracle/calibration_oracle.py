"""CPU restatement of the reference's layer calibration (TEST INFRASTRUCTURE).

Only tests/ import this module, as the checker of actune_amd.calibration.
Follows actune/calibration.py:42-93 step by step in torch-CPU, with the
float GEMMs of the candidate evaluations in float64 (so its scores carry no
summation-order noise of their own) and the codebooks taken from the C
oracle: activation codes of calibration.py:7-16 (grouped_oracle.c) and
weight codes of quantizers.py:23-94 with the division semantics of the
device the reference runs them on (``gpu_division``: True for a layer on
the GPU, the product's case; False for torch-CPU, the case of the golden
vectors written by tests/golden/make_calibration_vectors.py).

Pinned by tests/test_calibration_cpu.py: against the reference's own outputs
on seeded layers (tests/golden/calibration_vectors.npz), and by invariants
(constant channel moments give a unit scale, every selected clip is the
first argmin of an independently computed row loss, each error is the
gain-weighted sum of the row minima, W4-grid weights dequantize exactly).
"""
from __future__ import annotations

import numpy as np
import torch

from . import oracle as O

CLIP_GRID = (1., .975, .95, .925, .9, .875, .85, .8, .75)


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _dequant_x(x_bf16, a):
    """activation_reference(x, a) of a bf16 tensor, float64."""
    _, scales, codes = O.quantize_groups(_bits(x_bf16), a, "bf16")
    m, k = codes.shape
    return (codes.astype(np.float32).reshape(m, k // 64, 64) * scales[:, :, None]).reshape(m, k).astype(np.float64)


def _dequant_w(weight_bf16, w, a, ratio, gpu_division=True):
    codes, scale = O.weight_codes(weight_bf16.float().numpy(), w, a, ratio, gpu_division=gpu_division)
    return (codes.astype(np.float32) * scale[:, None]).astype(np.float64)


def calibrate_linear(weight, x, gains=None, *, budget="w4a4", clip_grid=CLIP_GRID, scale=None, gpu_division=True):
    """weight: bf16 [N, K] (CPU), x: bf16 [M, K] (CPU). Returns the same dict
    as the reference. scale: an explicit channel scale (skips the alpha fit);
    gpu_division: weight codes as torch computes them on the GPU (else
    torch-CPU's IEEE quotient)."""
    n = weight.shape[0]
    gains = np.ones(n) if gains is None else np.asarray(gains, np.float64)
    reference = x.double().numpy() @ weight.double().numpy().T
    base_a = 4 if budget == "w4a4" else 8
    if scale is None:
        moment = x.float().abs().mean(0).clamp_min(1e-4)
        best = None
        for alpha in (0., .25, .5, .75, 1.):
            s = moment.pow(alpha)
            s = (s / (s.max() * s.min()).sqrt()).clamp(1 / 16, 16).to(x.dtype)
            wt = (weight * s[None, :]).to(x.dtype)
            y = _dequant_x((x / s).contiguous(), base_a) @ _dequant_w(wt, 4, base_a, None, gpu_division).T
            score = float((((y - reference) ** 2).mean(0) * gains).sum())
            if best is None or score < best[0]:
                best = score, s
        scale = best[1]
    wt = (weight * scale[None, :]).to(x.dtype)
    xs = (x / scale).contiguous()
    errors, clips = {}, {}
    for w in (2, 4, 8):
        for a in ((8,) if budget == "w4a8" else (2, 4, 8)):
            xq = _dequant_x(xs, a)
            row_error = np.full(n, np.inf)
            selected = np.ones(n, np.float32)
            for ratio in clip_grid:
                y = xq @ _dequant_w(wt, w, a, ratio, gpu_division).T
                loss = ((y - reference) ** 2).mean(0)
                improve = loss < row_error
                selected[improve], row_error[improve] = ratio, loss[improve]
            errors[f"w{w}a{a}"] = float((row_error * gains).sum())
            clips[f"w{w}a{a}"] = selected
    return dict(channel_scale=scale, clips=clips, errors=errors)
