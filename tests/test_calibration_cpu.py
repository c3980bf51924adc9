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


# ---------------------------------------------------------------- pins of the restatement
from pathlib import Path

from oracle import oracle as O

GOLDEN = Path(__file__).parent / "golden" / "calibration_vectors.npz"


def _bf16(bits_u16):
    return torch.from_numpy(bits_u16.view(np.int16)).view(torch.bfloat16)


def test_oracle_equals_reference_vectors():
    """The reference's own calibrate_linear outputs on five seeded layers
    (tests/golden/make_calibration_vectors.py; torch-CPU, so the IEEE
    weight-code division): channel scales and every row's clip ratio are
    identical, errors agree within 1e-4 relative (the reference scores in
    float32, the restatement in float64; measured differences <= 5e-6)."""
    d = np.load(GOLDEN)
    for i in range(int(d["cases"])):
        p = f"c{i}_"
        gains = d[p + "gains"] if p + "gains" in d else None
        fit = CO.calibrate_linear(_bf16(d[p + "weight"]), _bf16(d[p + "x"]), gains, budget=str(d[p + "budget"]),
                                  gpu_division=False)
        np.testing.assert_array_equal(fit["channel_scale"].view(torch.int16).numpy().view(np.uint16),
                                      d[p + "channel_scale"], err_msg=f"case {i}")
        assert sorted(fit["clips"]) == sorted(k[len(p) + 6:] for k in d.files if k.startswith(p + "clips_"))
        for mode, clips in fit["clips"].items():
            np.testing.assert_array_equal(clips, d[p + "clips_" + mode], err_msg=f"case {i} {mode}")
            want = float(d[p + "error_" + mode])
            assert abs(fit["errors"][mode] - want) <= 1e-4 * abs(want), (i, mode)


def test_constant_channel_moments_give_unit_scale():
    """Every channel with the same mean |x|: moment^alpha is constant, so the
    normalised scale s / sqrt(max * min) is exactly 1 for every alpha."""
    g = torch.Generator().manual_seed(3)
    signs = torch.randint(0, 2, (16, 128), generator=g) * 2 - 1
    x = (signs * 0.75).to(torch.bfloat16)
    w = (torch.randn(24, 128, generator=g) * 0.02).to(torch.bfloat16)
    fit = CO.calibrate_linear(w, x, clip_grid=(1., .9))
    assert torch.equal(fit["channel_scale"], torch.ones(128, dtype=torch.bfloat16))


@pytest.mark.parametrize("budget", ["w4a4", "w4a8"])
def test_selected_clips_are_first_argmins_of_row_losses(budget):
    """For a fixed channel scale, each row's selected ratio is the FIRST
    grid ratio reaching that row's minimum loss, computed here on its own
    from the codebooks (dequantized weights per ratio, float64 products),
    and errors[mode] is the gain-weighted sum of those row minima."""
    g = torch.Generator().manual_seed(11)
    n, k, m = 20, 128, 24
    w = (torch.randn(n, k, generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(m, k, generator=g)
    x[:, :4] *= 12
    x = x.to(torch.bfloat16)
    gains = np.linspace(0.5, 2.0, n)
    scale = torch.linspace(0.5, 2.0, k).to(torch.bfloat16)
    grid = (1., .95, .9, .85, .8)
    fit = CO.calibrate_linear(w, x, gains, budget=budget, clip_grid=grid, scale=scale)
    wt = (w * scale[None, :]).to(torch.bfloat16).float().numpy()
    target = x.double().numpy() @ w.double().numpy().T
    xs = (x / scale).contiguous()
    for mode, clips in fit["clips"].items():
        W, A = int(mode[1]), int(mode[3])
        _, a_scales, a_codes = O.quantize_groups(xs.view(torch.int16).numpy().view(np.uint16), A, "bf16")
        # activation_reference's codes * scale is a float32 product too (calibration.py:16)
        xq = (a_codes.astype(np.float32).reshape(m, k // 64, 64) * a_scales[:, :, None]).reshape(m, k)
        xq = xq.astype(np.float64)
        losses = []
        for r in grid:
            codes, sc = O.weight_codes(wt, W, A, r, gpu_division=True)
            # the dequantized weight q.float() * s is a float32 product (calibration.py:87)
            wq = (codes.astype(np.float32) * sc[:, None]).astype(np.float64)
            losses.append((((xq @ wq.T) - target) ** 2).mean(0))
        losses = np.array(losses)
        first = np.argmax(losses == losses.min(0)[None, :], axis=0)
        np.testing.assert_array_equal(clips, np.array(grid, np.float32)[first], err_msg=mode)
        assert fit["errors"][mode] == pytest.approx(float((losses.min(0) * gains).sum()), rel=1e-12)
        if W == 8 and A != 4:
            assert np.all(clips == 1.0)  # W8 codes ignore the ratio: every ratio ties, the first wins


def test_w4_grid_weights_dequantize_exactly():
    """A weight whose rows are integer multiples of amax / 7 in [-8, 7]
    (amax itself on the grid) dequantizes back to itself at ratio 1, so its
    W4 loss against a float product of the same codes is exactly zero."""
    rng = np.random.default_rng(5)
    codes = rng.integers(-7, 8, size=(6, 64)).astype(np.float32)
    codes[:, 0] = 7
    step = np.float32(2.0 ** -6)
    w = torch.from_numpy(codes * step).to(torch.bfloat16)
    assert torch.equal(w.float(), torch.from_numpy(codes * step))  # exactly representable
    for gpu_division in (True, False):
        back = CO._dequant_w(w, 4, 8, 1.0, gpu_division)
        np.testing.assert_array_equal(back, (codes * step).astype(np.float64))
