"""GPU calibration (actune_amd.calibration) against the oracle restatement
of the reference's calibrate_linear (oracle/calibration_oracle.py) and the
bit-level oracle of its pieces."""
import numpy as np
import pytest
import torch

from actune_amd import calibration as C
from oracle import calibration_oracle as CO
from oracle import oracle as O
from tests.helpers import PAIRS, bits, canonical_bounds, seeded_inputs

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


@pytest.mark.parametrize("A", [2, 4, 8])
def test_activation_reference_is_the_inference_codebook(A):
    x, _, _ = seeded_inputs(13, 320, 1, seed=A)
    got = C.activation_reference(x.to(DEV).reshape(13, 5, 64).reshape(13, 320), A)
    np.testing.assert_array_equal(got.cpu().numpy(), O.activation_dequant(x.float().numpy(), A))
    assert got.dtype == torch.float32 and got.shape == (13, 320)


@pytest.mark.parametrize("W,A", PAIRS)
def test_device_codebooks_follow_gpu_division(W, A):
    _, w, _ = seeded_inputs(1, 256, 48, seed=W * 10 + A)
    for ratio in (None, 0.9):
        codes, scale = C._codes_on_device(w.to(DEV), W, A, ratio)
        want_c, want_s = O.weight_codes(w.float().numpy(), W, A, ratio, gpu_division=True)
        np.testing.assert_array_equal(codes.cpu().numpy(), want_c)
        np.testing.assert_array_equal(scale.cpu().numpy(), want_s)


@pytest.mark.parametrize("W,A", [(4, 4), (2, 8), (8, 4)])
def test_candidate_outputs_are_the_packed_gemm_in_fp32(W, A):
    """Each candidate evaluation is the inference GEMM with fp32 output,
    bit-exact against the oracle in the library's canonical order."""
    x, w, _ = seeded_inputs(24, 512, 40, seed=W + A)
    y = C._candidate(x.to(DEV), w.to(DEV), W, A, 0.95)
    codes, scale = O.weight_codes(w.float().numpy(), W, A, 0.95, gpu_division=True)
    _, a_s, a_c = O.quantize_groups(bits(x), A)
    want = O.linear(a_c, a_s, codes, scale, bounds=canonical_bounds(8))
    np.testing.assert_array_equal(y.cpu().numpy(), want)


@pytest.mark.parametrize("budget", ["w4a4", "w4a8"])
def test_calibrate_linear_matches_reference_restatement(budget):
    """Same channel scale and clips as the reference's algorithm (restated on
    the CPU with float64 GEMMs), errors within 1e-3 relative."""
    torch.manual_seed(11)
    lin = torch.nn.Linear(256, 64, bias=False, dtype=torch.bfloat16)
    x, _, _ = seeded_inputs(48, 256, 1, seed=21)
    gains = torch.rand(64, generator=torch.Generator().manual_seed(2))
    got = C.calibrate_linear(lin.to(DEV), x.to(DEV), gains.to(DEV), budget=budget, clip_grid=(1., .9, .8))
    want = CO.calibrate_linear(lin.weight.detach().cpu(), x, gains.numpy(), budget=budget, clip_grid=(1., .9, .8))
    assert torch.equal(got["channel_scale"].cpu(), want["channel_scale"])
    assert set(got["errors"]) == set(want["errors"]) and got["group_size"] == 64
    for mode in want["errors"]:
        np.testing.assert_array_equal(got["clips"][mode].cpu().numpy(), want["clips"][mode], err_msg=mode)
        np.testing.assert_allclose(got["errors"][mode], want["errors"][mode], rtol=1e-3)


def test_calibrate_linear_rejects_like_the_reference():
    lin = torch.nn.Linear(64, 8, bias=False, dtype=torch.bfloat16, device=DEV)
    x = torch.randn(4, 64, device=DEV).to(torch.bfloat16)
    with pytest.raises(ValueError, match="Unknown precision budget"):
        C.calibrate_linear(lin, x, budget="w2a2")
    with pytest.raises(ValueError, match="Invalid action-Jacobian weights"):
        C.calibrate_linear(lin, x, -torch.ones(8, device=DEV))
    with pytest.raises(ValueError, match="Nonempty finite aligned"):
        C.calibrate_linear(lin, x[:0])
    with pytest.raises(ValueError, match="Clip ratios must lie"):
        C.calibrate_linear(lin, x, clip_grid=(1.5,))
