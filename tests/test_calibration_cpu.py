"""CPU checks of the calibration surface: the GPU-only path refuses CPU
tensors with the reference's validation order, and the oracle restatement
reproduces the reference test's shape (nine pairs, non-negative errors;
tests/test_kernels.py:17-25)."""
import numpy as np
import pytest
import torch

from actune_amd import calibration as C
from oracle import calibration_oracle as CO


def test_cpu_tensors_are_refused():
    lin = torch.nn.Linear(64, 8, bias=False, dtype=torch.bfloat16)
    x = torch.randn(4, 64).to(torch.bfloat16)
    with pytest.raises(ValueError, match="CUDA"):
        C.calibrate_linear(lin, x)
    with pytest.raises(ValueError, match="CUDA"):
        C.activation_reference(x, 4)
    with pytest.raises(ValueError, match="Unsupported activation width"):
        C.activation_reference(x, 3)


def test_oracle_restatement_nine_pairs():
    torch.manual_seed(7)
    lin = torch.nn.Linear(64, 8, bias=False).to(torch.bfloat16)
    x = torch.randn(8, 64).to(torch.bfloat16)
    fitted = CO.calibrate_linear(lin.weight.detach(), x, clip_grid=(1., .9))
    assert len(fitted["errors"]) == 9 and all(v >= 0 for v in fitted["errors"].values())
    assert all(set(np.unique(c)) <= {1.0, np.float32(0.9)} for c in fitted["clips"].values())
