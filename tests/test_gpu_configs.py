"""GPU parity at the BASELINE configurations C1 and C3, through the C ABI.

C1: one linear, M=16, K=N=4096, W4A8 (the reference's CPU-path case), every
output against the oracle. C3: the Llama-2-7B linears (4096x4096,
11008x4096, 4096x11008) at prefill M=512 for all nine (W, A) pairs through
the default (automatic) kernel configuration, 64 sampled rows x 64 sampled
columns per case.

Each case checks, on the same seeded CPU-generated inputs:
  * the packed activation codes and scales, bit-exact (all of x);
  * the bf16 output, bit-exact against the oracle in the library's
    canonical fp32 order (16 quad-aligned K-chunks);
  * the deviation from the reference kernels' sequential fp32 order
    (grouped_native.cu:75, grouped.py:91), bounded by the error analysis of
    the two summation orders: |y - bf16(y_seq)| <= 1 bf16 ulp of y_seq plus
    about 2 (G + 16) 2^-24 |ws| sum_g |d_g s_g| (chunked or sequential
    summation of G terms is within ~(G + 16) 2^-24 sum |terms| of the exact
    sum); the table records how many outputs are exact and within 1 ulp;
  * the reference's own float criterion (tests/test_kernels.py:42-48):
    within rtol = atol = 0.02 of F.linear(activation_reference(x),
    q.float() * scale) evaluated in float64 and rounded to bf16.

With ACTUNE_ERROR_TABLE=<path> every case appends one JSON line of its
error statistics to <path> (the per-pair table kept with the measurements).
"""
import json
import os

import numpy as np
import pytest
import torch

from actune_amd import _native
from oracle import oracle as O
from tests.helpers import PAIRS, bits, canonical_bounds, oracle_activation, seeded_inputs

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
LLAMA = [(4096, 4096), (11008, 4096), (4096, 11008)]


def _bf16_ulp(v):
    """Spacing of bf16 numbers at |v| (normal range)."""
    e = np.floor(np.log2(np.maximum(np.abs(v), 2.0**-126)))
    return 2.0 ** (e - 7)


def _check_case(name, m, n, k, W, A, rows, cols, seed):
    x, w, _ = seeded_inputs(m, k, n, seed=seed)
    xd = x.to(DEV)
    codes, scale = O.weight_codes(w.float().numpy(), W, A)
    w_dev = torch.from_numpy(O.pack_rows(codes, W)).to(DEV)
    ws_dev = torch.from_numpy(scale).to(DEV)
    out = _native.grouped_forward(xd, w_dev, ws_dev, None, W, A)
    p, s = _native.quantize_groups(xd, A)
    torch.cuda.synchronize()
    want_p, want_s, a_codes = oracle_activation(x, A)
    np.testing.assert_array_equal(p.cpu().numpy(), want_p)
    np.testing.assert_array_equal(s.cpu().numpy(), want_s)

    G = k // 64
    got_bits = bits(out)[rows][:, cols]
    canon = O.linear(a_codes, want_s, codes, scale, None, bounds=canonical_bounds(G), rows=rows, cols=cols)
    np.testing.assert_array_equal(got_bits, O.round_out(canon, "bf16"))

    got = O.bf16_bits_to_f32(got_bits).astype(np.float64)
    seq = O.linear(a_codes, want_s, codes, scale, None, rows=rows, cols=cols)
    seq_b = O.bf16_bits_to_f32(O.round_out(seq, "bf16")).astype(np.float64)
    dots = O.group_dots(a_codes, codes, rows, cols).astype(np.float64)
    terms = np.abs(dots * want_s[rows][:, None, :].astype(np.float64)).sum(-1) * np.abs(scale[cols][None, :])
    # chunked (canonical) and sequential summation each stay within
    # gamma_(G+16) * sum |t_g| of the exact sum, gamma_n ~ n * 2^-24; the
    # products by ws and the two bf16 roundings add at most one bf16 ulp of
    # the larger result and 2^-23 relative
    bound = (_bf16_ulp(np.maximum(np.abs(got), np.abs(seq_b))) + 2.02 * (G + 16) * 2.0**-24 * terms
             + 2.0**-23 * np.abs(seq_b))
    dev = np.abs(got - seq_b)
    assert np.all(dev <= bound), f"max excess {np.max(dev - bound):.3e}"
    ulps = dev / _bf16_ulp(seq_b)

    xq = O.activation_dequant(x[rows].float().numpy(), A).astype(np.float64)
    wf = codes[cols].astype(np.float64) * scale[cols].astype(np.float64)[:, None]
    ref = O.bf16_bits_to_f32(O.round_out((xq @ wf.T).astype(np.float32), "bf16")).astype(np.float64)
    np.testing.assert_allclose(got, ref, rtol=0.02, atol=0.02)

    row = dict(case=name, M=m, N=n, K=k, W=W, A=A, outputs=int(got.size),
               seq_exact_frac=round(float(np.mean(dev == 0)), 4),
               seq_within_1ulp_frac=round(float(np.mean(ulps <= 1)), 4),
               seq_max_ulps=round(float(ulps.max()), 2),
               seq_max_abs=float(dev.max()),
               seq_max_rel=float((dev / np.maximum(np.abs(seq_b), 1e-3)).max()),
               float_max_abs=float(np.abs(got - ref).max()),
               float_max_rel=float((np.abs(got - ref) / np.maximum(np.abs(ref), 1e-3)).max()))
    path = os.environ.get("ACTUNE_ERROR_TABLE")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps(row) + "\n")
    print(json.dumps(row))


def test_c1_single_linear_all_outputs():
    """C1: M=16, 4096x4096, W4A8, seed 0, default path; every output."""
    m, n, k = 16, 4096, 4096
    _check_case("C1", m, n, k, 4, 8, np.arange(m), np.arange(n), seed=0)


@pytest.mark.parametrize("n,k", LLAMA)
@pytest.mark.parametrize("W,A", PAIRS)
def test_c3_prefill_all_pairs(W, A, n, k):
    """C3: M=512 on the three Llama-2-7B shapes, all nine pairs."""
    m = 512
    rng = np.random.default_rng(n + k + W * 10 + A)
    rows = np.sort(rng.choice(m, size=64, replace=False))
    cols = np.sort(rng.choice(n, size=64, replace=False))
    _check_case("C3", m, n, k, W, A, rows, cols, seed=3000 + n + k + W * 10 + A)
