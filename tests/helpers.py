"""Shared test helpers: seeded inputs generated on the CPU (so the oracle and
the GPU see identical bits) and conversions between torch and the oracle."""
from __future__ import annotations

import numpy as np
import torch

from oracle import oracle as O

PAIRS = [(w, a) for w in (2, 4, 8) for a in (2, 4, 8)]
CHUNKS = 16  # canonical reduction order of the library: 16 quad-aligned chunks


def bits(t: torch.Tensor) -> np.ndarray:
    """bf16/f16 tensor -> uint16 bit patterns; f32 -> float32 array."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.float32:
        return t.numpy()
    return t.view(torch.int16).numpy().view(np.uint16)


def dtype_name(dtype) -> str:
    return {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}[dtype]


def seeded_inputs(m, k, n, seed, dtype=torch.bfloat16, outliers=True, bias=False):
    """x ~ N(0,1) with 1 % of channels x10, W ~ N(0, 0.02), optional bias,
    all generated on the CPU from one seed."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g)
    if outliers:
        ch = torch.randperm(k, generator=g)[: max(1, k // 100)]
        x[:, ch] *= 10
    w = torch.randn(n, k, generator=g) * 0.02
    b = torch.randn(n, generator=g) * 0.1 if bias else None
    return x.to(dtype), w.to(dtype), (None if b is None else b.to(dtype))


def canonical_bounds(G):
    return O.chunk_bounds(G, 4, CHUNKS)


def oracle_weight(w: torch.Tensor, W, A, ratios=None):
    codes, scale = O.weight_codes(w.float().numpy(), W, A, ratios)
    return codes, scale


def oracle_activation(x: torch.Tensor, A, input_scale=None):
    return O.quantize_groups(bits(x), A, dtype_name(x.dtype),
                             None if input_scale is None else bits(input_scale))


def rel_err(got: np.ndarray, want: np.ndarray):
    g = got.astype(np.float64)
    w = want.astype(np.float64)
    abs_err = np.abs(g - w)
    return float(abs_err.max(initial=0.0)), float((abs_err / np.maximum(np.abs(w), 1e-3)).max(initial=0.0))
