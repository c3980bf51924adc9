"""The Python binding rejects caller buffers of the wrong shape, dtype,
layout or device before anything is launched: the C ABI takes raw pointers
and cannot check sizes itself. No kernel runs in these tests."""
import pytest
import torch

from actune_amd import _native

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
M, K, N, W, A = 3, 256, 32, 4, 8


def _ops():
    x = torch.randn(M, K, device=DEV, dtype=torch.bfloat16)
    w = torch.zeros(N, K * W // 8, device=DEV, dtype=torch.uint8)
    ws = torch.ones(N, device=DEV)
    return x, w, ws


def _fwd(**kw):
    x, w, ws = _ops()
    args = dict(flat=x, w=w, ws=ws, bias=None, W=W, A=A)
    args.update(kw)
    return _native.grouped_forward(**args)


# buffers are built inside the test (a GPU is needed), so each case is a factory
CASES = [
    (lambda: dict(out=torch.empty(M, N - 1, device=DEV, dtype=torch.bfloat16)), "out must be a contiguous"),
    (lambda: dict(out=torch.empty(M, N, device=DEV, dtype=torch.float32)), "out must be torch.bfloat16"),
    (lambda: dict(out=torch.empty(N, M, device=DEV, dtype=torch.bfloat16).t()), "out must be a contiguous"),
    (lambda: dict(packed=torch.empty(M, K * A // 8 - 16, device=DEV, dtype=torch.uint8)), "packed must be a contiguous"),
    (lambda: dict(packed=torch.empty(M, K * A // 8, device=DEV, dtype=torch.int8)), "packed must be torch.uint8"),
    (lambda: dict(scales=torch.empty(M, K // 64 - 1, device=DEV)), "scales must be a contiguous"),
    (lambda: dict(scales=torch.empty(M, K // 64, device=DEV, dtype=torch.float16)), "scales must be torch.float32"),
    (lambda: dict(ws=torch.ones(N - 1, device=DEV)), "scale shape mismatch"),
    (lambda: dict(ws=torch.ones(N, device=DEV, dtype=torch.float16)), "float scales/bias required"),
    (lambda: dict(bias=torch.zeros(N + 1, device=DEV)), "bias shape mismatch"),
    (lambda: dict(bias=torch.zeros(N, device=DEV, dtype=torch.int32)), "float scales/bias required"),
    (lambda: dict(w=torch.zeros(N, K * W // 8 + 1, device=DEV, dtype=torch.uint8)), "packed shape mismatch"),
    (lambda: dict(flat=torch.randn(K, M, device=DEV, dtype=torch.bfloat16).t()), "contiguous"),
    (lambda: dict(flat=torch.randn(M, K, dtype=torch.bfloat16)), "CUDA required"),
    (lambda: dict(W=3), "Unsupported integer width"),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_grouped_forward_rejects(case):
    make, msg = CASES[case]
    with pytest.raises((RuntimeError, ValueError), match=msg):
        _fwd(**make())


def test_grouped_linear_rejects_bad_out_and_bias():
    x, w, ws = _ops()
    p, s = _native.quantize_groups(x, A)
    with pytest.raises(RuntimeError, match="out must"):
        _native.grouped_linear(p, s, w, ws, None, x, W, A, out=torch.empty(M, N, device=DEV))
    with pytest.raises(RuntimeError, match="float scales/bias required"):
        _native.grouped_linear(p, s, w, ws, torch.zeros(N, device=DEV, dtype=torch.int64), x, W, A)


def test_multi_rejects_short_target_out():
    x, w, ws = _ops()
    bad = torch.empty(M, N // 2, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match=r"out\[1\] must"):
        _native.grouped_forward_multi(x, [(w, ws, None, None), (w, ws, None, bad)], W, A)


def test_quantize_rejects_short_buffers():
    x, _, _ = _ops()
    with pytest.raises(RuntimeError, match="packed must"):
        _native.quantize_groups(x, A, packed=torch.empty(M, 8, device=DEV, dtype=torch.uint8))
    with pytest.raises(RuntimeError, match="scales must"):
        _native.quantize_groups(x, A, scales=torch.empty(1, device=DEV))
