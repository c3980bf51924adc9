"""actune_grouped_forward_noalloc (static device scratch) against
actune_grouped_forward (caller-owned scratch), through the C ABI.

Two calls in a row on the same device, the second with a smaller input, so
the second reads what it wrote itself over what the first left in the shared
array; each must equal the regular entry point bit for bit. Sizes beyond the
8 MiB array are rejected before anything is launched.
"""
import ctypes

import pytest
import torch

from actune_amd import _native
from oracle import oracle as O
from tests.helpers import seeded_inputs

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
_P, _I, _I64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64


def _lib():
    lib = _native.lib()
    lib.actune_grouped_forward_noalloc.argtypes = [_P, _I, _P, _P, _P, _P, _I, _P, _I64, _I64, _I64, _I, _I, _I, _P]
    return lib


def _case(m, k, n, W, A, seed, bias):
    x, w, b = seeded_inputs(m, k, n, seed=seed, bias=bias)
    codes, scale = O.weight_codes(w.float().numpy(), W, A)
    wd = torch.from_numpy(O.pack_rows(codes, W)).to(DEV)
    wsd = torch.from_numpy(scale).to(DEV)
    return x.to(DEV), wd, wsd, None if b is None else b.to(DEV)


def _noalloc(x, w, ws, b, W, A, config=-1):
    m, k = x.shape
    n = w.shape[0]
    out = torch.full((m, n), float("nan"), device=DEV, dtype=x.dtype)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = _lib().actune_grouped_forward_noalloc(
        x.data_ptr(), 0, None, w.data_ptr(), ws.data_ptr(), None if b is None else b.data_ptr(),
        2 if b is None else 0, out.data_ptr(), m, n, k, W, A, config, stream)
    assert rc == 0, _native.lib().actune_last_error().decode()
    return out


@pytest.mark.parametrize("W,A", [(4, 8), (2, 4), (8, 2), (8, 8)])
def test_noalloc_matches_regular_entry_point_twice(W, A):
    # first a large call (prefill-sized, quantizer launch + prefill GEMM),
    # then a smaller one (decode-sized) on the same scratch
    for m, k, n, seed, bias in ((300, 4096, 256, 1, True), (5, 1024, 96, 2, False)):
        x, w, ws, b = _case(m, k, n, W, A, seed + W * A, bias)
        want = _native.grouped_forward(x, w, ws, b, W, A)
        got = _noalloc(x, w, ws, b, W, A)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (m, k, n)
    # and an explicit config that always takes the quantizer's codes
    x, w, ws, b = _case(3, 512, 48, W, A, 7, False)
    assert torch.equal(_noalloc(x, w, ws, b, W, A, config=3), _native.grouped_forward(x, w, ws, b, W, A, config=3))


def test_noalloc_rejects_sizes_beyond_the_scratch():
    x = torch.zeros(1024, 8192, device=DEV, dtype=torch.bfloat16)  # 8 MiB of A8 codes + scales
    w = torch.zeros(16, 4096, device=DEV, dtype=torch.uint8)
    ws = torch.ones(16, device=DEV)
    out = torch.empty(1024, 16, device=DEV, dtype=torch.bfloat16)
    rc = _lib().actune_grouped_forward_noalloc(x.data_ptr(), 0, None, w.data_ptr(), ws.data_ptr(), None, 2,
                                               out.data_ptr(), 1024, 16, 8192, 4, 8, -1, None)
    assert rc == 1 and "static scratch" in _native.lib().actune_last_error().decode()
