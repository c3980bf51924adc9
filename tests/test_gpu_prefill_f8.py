"""GPU parity of the fp8 prefill path (ACTUNE_CONFIG_PREFILL_F8, W, A <= 4):
the quantizer's fp8 operand mode and the fp8-MFMA GEMM, through the C ABI.

Bar: outputs bit-exact against the oracle in the library's canonical fp32
order and equal to the int8 prefill kernel's bit for bit, over ragged M, N
and K (a last quad short of 4 groups; canonical chunks of several quads),
bias and no bias, every input dtype, the fused channel scale and sibling
targets."""
import numpy as np
import pytest
import torch

from actune_amd import _native
from oracle import oracle as O
from tests.helpers import bits, canonical_bounds, dtype_name, oracle_activation, oracle_weight, seeded_inputs

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
F8_PAIRS = [(4, 4), (4, 2), (2, 4), (2, 2)]
INT8_PREFILL = 12  # gemm_prefill, 64x64 tiles: the same results on int8 MFMAs


def _weights(w, W, A):
    codes, scale = oracle_weight(w, W, A)
    return codes, scale, torch.from_numpy(O.pack_rows(codes, W)).to(DEV), torch.from_numpy(scale).to(DEV)


def _bias(b, A):
    return None if b is None else (b.float() if A == 4 else b)  # the reference's bias storage rule


@pytest.mark.parametrize("W,A", F8_PAIRS)
@pytest.mark.parametrize("shape", [(65, 256, 96), (64, 64, 64), (130, 448, 200), (200, 1088, 128),
                                   (66, 256, 16),
                                   # 68 groups: canonical chunks of one or two quads
                                   (70, 4352, 40),
                                   # 21 groups: a ragged last quad
                                   (96, 1344, 72)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_f8_forward_bit_exact(W, A, shape, with_bias):
    m, k, n = shape
    x, w, b = seeded_inputs(m, k, n, seed=W * 1000 + A * 100 + m + n, bias=with_bias)
    wc, wsc, w_dev, ws_dev = _weights(w, W, A)
    bias = _bias(b, A)
    xd, bd = x.to(DEV), None if bias is None else bias.to(DEV)
    got = _native.grouped_forward(xd, w_dev, ws_dev, bd, W, A, config=_native.CONFIG_PREFILL_F8)
    ref = _native.grouped_forward(xd, w_dev, ws_dev, bd, W, A, config=INT8_PREFILL)
    _, asc, ac = oracle_activation(x, A)
    want = O.linear(ac, asc, wc, wsc, None if bias is None else bias.float().numpy(),
                    bounds=canonical_bounds(k // 64))
    np.testing.assert_array_equal(bits(got), O.round_out(want, "bf16"))
    assert torch.equal(got, ref)


@pytest.mark.parametrize("W,A", F8_PAIRS)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_f8_forward_dtypes_and_channel_scale(W, A, dtype):
    m, k, n = 97, 576, 80
    x, w, _ = seeded_inputs(m, k, n, seed=W + 7 * A, dtype=dtype)
    scale = torch.linspace(0.5, 2.0, k).to(dtype)
    wc, wsc, w_dev, ws_dev = _weights(w, W, A)
    xd, sd = x.to(DEV), scale.to(DEV)
    got = _native.grouped_forward(xd, w_dev, ws_dev, None, W, A, input_scale=sd, config=_native.CONFIG_PREFILL_F8)
    ref = _native.grouped_forward(xd, w_dev, ws_dev, None, W, A, input_scale=sd, config=INT8_PREFILL)
    assert got.dtype == dtype and torch.equal(got, ref)
    _, asc, ac = oracle_activation(x, A, scale)
    want = O.linear(ac, asc, wc, wsc, None, bounds=canonical_bounds(k // 64))
    np.testing.assert_array_equal(bits(got), O.round_out(want, dtype_name(dtype)))


@pytest.mark.parametrize("W,A", [(4, 4), (2, 2)])
def test_f8_multi_target_and_auto(W, A):
    """Sibling targets share one quantization; ACTUNE_CONFIG_AUTO takes the
    fp8 kernel at prefill sizes and gives the same outputs."""
    m, k = 256, 1024
    x, _, _ = seeded_inputs(m, k, 1, seed=11 * W + A)
    xd = x.to(DEV)
    targets, refs = [], []
    for j, n in enumerate((192, 64, 320)):
        _, w, b = seeded_inputs(m, k, n, seed=j + 5, bias=True)
        _, _, w_dev, ws_dev = _weights(w, W, A)
        bd = _bias(b, A).to(DEV)
        targets.append((w_dev, ws_dev, bd, None))
        refs.append(_native.grouped_forward(xd, w_dev, ws_dev, bd, W, A, config=INT8_PREFILL))
    assert _native.forward_workspace_bytes(m, 576, k, W, A) == m * k
    outs = _native.grouped_forward_multi(xd, targets, W, A, config=_native.CONFIG_PREFILL_F8)
    auto = _native.grouped_forward_multi(xd, targets, W, A)
    for o, a, r in zip(outs, auto, refs):
        assert torch.equal(o, r) and torch.equal(a, r)


def test_f8_caller_workspace_and_errors():
    m, k, n, W, A = 128, 512, 64, 4, 4
    x, w, _ = seeded_inputs(m, k, n, seed=3)
    _, _, w_dev, ws_dev = _weights(w, W, A)
    xd = x.to(DEV)
    work = torch.empty(m * k, dtype=torch.uint8, device=DEV)
    got = _native.grouped_forward(xd, w_dev, ws_dev, None, W, A, config=_native.CONFIG_PREFILL_F8, workspace=work)
    ref = _native.grouped_forward(xd, w_dev, ws_dev, None, W, A, config=INT8_PREFILL)
    assert torch.equal(got, ref)
    with pytest.raises(RuntimeError, match="workspace too small"):
        _native.grouped_forward(xd, w_dev, ws_dev, None, W, A, config=_native.CONFIG_PREFILL_F8,
                                workspace=work[: m * k - 16])
    # packed-code calls have no fp8 operands
    a, s = _native.quantize_groups(xd, A)
    with pytest.raises(ValueError, match="fp8 prefill"):
        _native.grouped_linear(a, s, w_dev, ws_dev, None, xd, W, A, _native.CONFIG_PREFILL_F8)
