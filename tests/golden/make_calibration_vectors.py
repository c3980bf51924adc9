"""Writes calibration_vectors.npz: input/output vectors of the reference's
``calibrate_linear`` (actune/calibration.py:42-93), the one function of the
path whose exact floating decisions (argmin over the alpha grid and the clip
grid) no closed form or invariant pins.

Run once in the build container, where the reference checkout exists:
    python tests/golden/make_calibration_vectors.py /root/reference
It imports the reference's pure-torch ``actune.calibration`` on the CPU
(weight codes then follow torch-CPU's IEEE division) and stores, per case,
the seeded bf16 weight and fitting inputs, the row gains, and the returned
channel scale, clip ratios and errors. Nothing of the reference's source is
stored; the tests read only this file.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

# (N, K, M, budget, gains): small layers with outlier channels, both budgets,
# unit and seeded non-uniform row gains
CASES = [(8, 64, 8, "w4a4", False), (24, 128, 16, "w4a4", True), (16, 256, 32, "w4a8", False),
         (32, 128, 12, "w4a8", True), (12, 192, 24, "w4a4", False)]


def bits16(t):
    return t.detach().contiguous().view(torch.int16).numpy().view(np.uint16)


def main(reference_root):
    sys.path.insert(0, str(reference_root))
    from actune.calibration import calibrate_linear
    out = {}
    for i, (n, k, m, budget, with_gains) in enumerate(CASES):
        g = torch.Generator().manual_seed(100 + i)
        weight = (torch.randn(n, k, generator=g) * 0.02).to(torch.bfloat16)
        x = torch.randn(m, k, generator=g)
        x[:, torch.randperm(k, generator=g)[: max(1, k // 32)]] *= 10
        x = x.to(torch.bfloat16)
        gains = torch.rand(n, generator=g) + 0.25 if with_gains else None
        lin = torch.nn.Linear(k, n, bias=False, dtype=torch.bfloat16)
        with torch.no_grad():
            lin.weight.copy_(weight)
        fit = calibrate_linear(lin, x, gains, budget=budget)
        p = f"c{i}_"
        out[p + "weight"] = bits16(weight)
        out[p + "x"] = bits16(x)
        out[p + "budget"] = np.array(budget)
        if gains is not None:
            out[p + "gains"] = gains.numpy()
        out[p + "channel_scale"] = bits16(fit["channel_scale"])
        for mode in sorted(fit["clips"]):
            out[p + "clips_" + mode] = fit["clips"][mode].numpy()
            out[p + "error_" + mode] = np.array(fit["errors"][mode], dtype=np.float64)
    dest = Path(__file__).with_name("calibration_vectors.npz")
    np.savez_compressed(dest, cases=np.array(len(CASES)), **out)
    print(f"wrote {dest} ({dest.stat().st_size} bytes, {len(CASES)} cases)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
