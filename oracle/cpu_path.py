"""The reference's CPU dequantize-then-matmul path, restated in torch-CPU
(TEST / BASELINE INFRASTRUCTURE ONLY: used by bench.py's cpu_baseline leg).

Follows tests/test_kernels.py:42-44 of zanehpn/Actune:
  F.linear(activation_reference(x, A), q.float() * scale[:, None], bias).to(bf16)
with activation_reference from actune/calibration.py:7-16 (group-64
symmetric quantize/dequantize in fp32). ``dequantize_weight`` is the hoisted
weight dequant of the steady-state variant.
"""
from __future__ import annotations

import torch


def activation_reference(value: torch.Tensor, bits: int, group_size: int = 64) -> torch.Tensor:
    shape = value.shape
    v = value.float().reshape(*shape[:-1], -1, group_size)
    p = (1 << (bits - 1)) - 1
    s = v.abs().amax(-1, keepdim=True).clamp_min(1e-8) / p
    return (torch.round(v / s).clamp(-p - 1, p) * s).reshape(shape)


def dequantize_weight(codes: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    return codes.float() * scale.float()[:, None]


def linear(x: torch.Tensor, bits: int, w_dequant: torch.Tensor, bias=None) -> torch.Tensor:
    return torch.nn.functional.linear(activation_reference(x, bits), w_dequant, bias).to(x.dtype)
