"""Seeded random sweep of the group-64 path on the GPU against the oracle.

Each case draws M (1-300), N (1-699), K (64-3072), the (W, A) pair, the
input dtype (= output dtype), a bias and its dtype, a channel scale and a
kernel config (AUTO or any config valid at M) from its own seed, runs the
forward through the C ABI, and checks every output bit against the oracle in
the canonical chunked fp32 order. The multi-target cases give each of one
to four targets its own N and weight width. The hand-picked shapes of the
other parity tests cover the known edges; this sweep covers combinations
of them that no one picked. The exact-zero test builds outputs that are 0
in the canonical order under every config, where a leaked term of any size
shows.
"""
import numpy as np
import pytest
import torch

from actune_amd import _native
from oracle import oracle as O
from tests.helpers import PAIRS, bits, canonical_bounds, dtype_name, oracle_weight, seeded_inputs

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
DTYPES = (torch.bfloat16, torch.float16, torch.float32)
MS = (1, 2, 3, 5, 8, 13, 16, 17, 31, 50, 64, 65, 96, 130, 257, 300)


def _draw(rng):
    m = int(rng.choice(MS))
    k = 64 * int(rng.integers(1, 49))
    A = int(rng.choice((2, 4, 8)))
    dtype = DTYPES[int(rng.integers(3))]
    bias_dtype = DTYPES[int(rng.integers(3))] if rng.random() < 0.5 else None
    scale = rng.random() < 0.3
    valid = [c for c in range(_native.num_configs()) if _native.config_valid(c, m)]
    config = _native.CONFIG_AUTO if rng.random() < 0.4 else int(rng.choice(valid))
    return m, k, A, dtype, bias_dtype, scale, config


def _target(rng, seed, m, k, n, W, A, dtype, bias_dtype):
    """Weights from seeded_inputs (CPU), their oracle codes and device buffers."""
    _, w, _ = seeded_inputs(1, k, n, seed=seed, dtype=dtype)
    wc, wsc = oracle_weight(w, W, A)
    bias = None
    if bias_dtype is not None:
        g = torch.Generator().manual_seed(seed + 1)
        bias = (torch.randn(n, generator=g) * 0.1).to(bias_dtype)
    dev = (torch.from_numpy(O.pack_rows(wc, W)).to(DEV), torch.from_numpy(wsc).to(DEV),
           None if bias is None else bias.to(DEV))
    return wc, wsc, bias, dev


def _inputs(seed, m, k, dtype, scale):
    x, _, _ = seeded_inputs(m, k, 1, seed=seed, dtype=dtype)
    s = None
    if scale:
        g = torch.Generator().manual_seed(seed + 2)
        s = (torch.rand(k, generator=g) * 1.5 + 0.25).to(dtype)
    return x, s


def _want(x, s, A, wc, wsc, bias, dtype, k):
    _, asc, ac = O.quantize_groups(bits(x), A, dtype_name(dtype), None if s is None else bits(s))
    y = O.linear(ac, asc, wc, wsc, None if bias is None else bias.float().numpy(), bounds=canonical_bounds(k // 64))
    return O.round_out(y, dtype_name(dtype))


@pytest.mark.parametrize("case", range(48))
def test_random_forward_against_oracle(case):
    rng = np.random.default_rng(7000 + case)
    m, k, A, dtype, bias_dtype, scale, config = _draw(rng)
    W = int(rng.choice((2, 4, 8)))
    n = int(rng.integers(1, 700))
    wc, wsc, bias, (w_dev, ws_dev, b_dev) = _target(rng, 100 * case, m, k, n, W, A, dtype, bias_dtype)
    x, s = _inputs(100 * case + 50, m, k, dtype, scale)
    out = _native.grouped_forward(x.to(DEV), w_dev, ws_dev, b_dev, W, A,
                                  input_scale=None if s is None else s.to(DEV), config=config)
    np.testing.assert_array_equal(bits(out), _want(x, s, A, wc, wsc, bias, dtype, k),
                                  err_msg=f"M={m} N={n} K={k} W{W}A{A} {dtype} bias={bias_dtype} "
                                          f"scale={scale} config={config}")


@pytest.mark.parametrize("case", range(24))
def test_random_multi_target_forward_against_oracle(case):
    rng = np.random.default_rng(9000 + case)
    m, k, A, dtype, bias_dtype, scale, config = _draw(rng)
    count = int(rng.integers(1, _native.MAX_TARGETS + 1))
    widths = [int(rng.choice((2, 4, 8))) for _ in range(count)]
    ns = [int(rng.integers(1, 400)) for _ in range(count)]
    targets, expect = [], []
    x, s = _inputs(100 * case + 77, m, k, dtype, scale)
    for j, (W, n) in enumerate(zip(widths, ns)):
        wc, wsc, bias, (w_dev, ws_dev, b_dev) = _target(rng, 100 * case + 10 * j, m, k, n, W, A, dtype, bias_dtype)
        targets.append((w_dev, ws_dev, b_dev, None, W))
        expect.append(_want(x, s, A, wc, wsc, bias, dtype, k))
    outs = _native.grouped_forward_multi(x.to(DEV), targets, widths[0], A,
                                         input_scale=None if s is None else s.to(DEV), config=config)
    for j, (out, want) in enumerate(zip(outs, expect)):
        np.testing.assert_array_equal(bits(out), want,
                                      err_msg=f"target {j}: M={m} N={ns} K={k} W={widths} A{A} {dtype} "
                                              f"bias={bias_dtype} scale={scale} config={config}")


@pytest.mark.parametrize("case", range(12))
def test_random_wide_forward_against_oracle(case):
    """AUTO forwards at 9-64 tokens on wide N (one to three targets of
    256-16416 rows, same or mixed widths, K up to 11008): the selection's
    wide-N branches, shared row tiles and x quantized in the launch with
    16-token blocks. Random codes and scales; 24 sampled columns per target
    against the oracle."""
    rng = np.random.default_rng(31000 + case)
    m = int(rng.integers(9, 65))
    k = 64 * int(rng.choice([16, 32, 64, 172]))
    A = int(rng.choice((2, 4, 8)))
    count = int(rng.integers(1, 4))
    widths = [int(rng.choice((2, 4, 8))) for _ in range(count)]
    if case % 2:
        widths = [widths[0]] * count
    ns = [int(rng.choice((256, 4096, 8192, 11008, 16384))) + 16 * int(rng.integers(0, 3)) for _ in range(count)]
    g = torch.Generator().manual_seed(case)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    _, asc, ac = O.quantize_groups(bits(x), A, "bf16")
    targets, expect = [], []
    for W, n in zip(widths, ns):
        q = (1 << (W - 1)) - 1
        wc = rng.integers(-q - 1, q + 1, size=(n, k), dtype=np.int8)
        wsc = (rng.random(n) * 0.02 + 0.001).astype(np.float32)
        cols = np.sort(rng.choice(n, size=24, replace=False))
        want = O.round_out(O.linear(ac, asc, wc, wsc, None, bounds=canonical_bounds(k // 64), cols=cols), "bf16")
        targets.append((torch.from_numpy(O.pack_rows(wc, W)).to(DEV), torch.from_numpy(wsc).to(DEV), None, None, W))
        expect.append((cols, want))
    outs = _native.grouped_forward_multi(x.to(DEV), targets, widths[0], A)
    for j, (out, (cols, want)) in enumerate(zip(outs, expect)):
        np.testing.assert_array_equal(bits(out)[:, cols], want,
                                      err_msg=f"target {j}: M={m} N={ns} K={k} W={widths} A{A}")


@pytest.mark.parametrize("W,A,ns,k,m", [(4, 4, (4096, 4096), 1024, 50), (4, 8, (16384,), 2048, 24),
                                         (2, 4, (8192,), 320, 64), (4, 2, (12288,), 576, 40),
                                         (8, 8, (8192, 8192), 1024, 64)])
def test_compact_partials_on_large_grids(W, A, ns, k, m):
    """4-wave launches of 16-token blocks with two row tiles per workgroup
    whose grid exceeds one round of resident workgroups, below 16 quads
    (G = 5, 9, 16, 32): the launch keeps one partial slot per nonempty chunk
    (decode_compact). Forward with x quantized in the launch or not (config
    14, the library's own choice), the same on the oracle's codes, and the
    exact-zero construction after a launch that leaves nonzero partials in
    LDS; sampled columns against the oracle."""
    rng = np.random.default_rng(k + m + W)
    g = torch.Generator().manual_seed(k + m)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    packed, asc, ac = O.quantize_groups(bits(x), A, "bf16")
    targets, expect = [], []
    for n in ns:
        q = (1 << (W - 1)) - 1
        wc = rng.integers(-q - 1, q + 1, size=(n, k), dtype=np.int8)
        wsc = (rng.random(n) * 0.02 + 0.001).astype(np.float32)
        cols = np.sort(rng.choice(n, size=32, replace=False))
        want = O.round_out(O.linear(ac, asc, wc, wsc, None, bounds=canonical_bounds(k // 64), cols=cols), "bf16")
        targets.append((torch.from_numpy(O.pack_rows(wc, W)).to(DEV), torch.from_numpy(wsc).to(DEV), None, None))
        expect.append((cols, want))
    outs = _native.grouped_forward_multi(x.to(DEV), targets, W, A, config=14)
    for j, (out, (cols, want)) in enumerate(zip(outs, expect)):
        np.testing.assert_array_equal(bits(out)[:, cols], want, err_msg=f"forward, target {j}")
    a_dev, s_dev = torch.from_numpy(packed).to(DEV), torch.from_numpy(asc).to(DEV)
    w_dev, ws_dev, _, _ = targets[0]
    cols, want = expect[0]
    got = _native.grouped_linear(a_dev, s_dev, w_dev, ws_dev, None, (m, k), W, A, 14)
    np.testing.assert_array_equal(bits(got)[:, cols], want, err_msg="on codes")
    # exact zeros on the same grid: group 4 of x repeats group 0 and every
    # weight row holds c in group 0, -c in group 4 (quads 0 and 1, so two
    # chunks below 16 quads) and zeros elsewhere
    xz = torch.randn(m, k, generator=g)
    xz[:, 256:320] = xz[:, 0:64]
    xz = xz.to(torch.bfloat16)
    q = (1 << (W - 1)) - 1
    zero_targets = []
    for (w_dev, ws_dev, _, _), n in zip(targets, ns):
        wz = np.zeros((n, k), np.int8)
        c = rng.integers(-q, q + 1, size=(n, 64), dtype=np.int8)
        wz[:, 0:64], wz[:, 256:320] = c, -c
        zero_targets.append((torch.from_numpy(O.pack_rows(wz, W)).to(DEV), ws_dev, None, None))
    _native.grouped_forward_multi(x.to(DEV), targets, W, A, config=14)
    for j, got in enumerate(_native.grouped_forward_multi(xz.to(DEV), zero_targets, W, A, config=14)):
        assert not bits(got).any(), f"a term leaked into a zero output, target {j}"


@pytest.mark.parametrize("W,A", PAIRS)
@pytest.mark.parametrize("m", [1, 2, 4, 17, 65])
def test_exact_zero_outputs_every_config(W, A, m):
    """Outputs that are exactly 0 in the canonical order stay exactly 0 under
    every config, on the forward (x quantized in the launch where the config
    does so, with and without a channel scale) and on packed codes: group 4
    of x (and of the channel scale) repeats group 0, each weight row holds
    codes c in group 0 and -c in group 4 (two canonical chunks) and zeros
    elsewhere. A term leaked into a partial sum (a group past K, a stale LDS
    row, a scale from outside the range) would show as a nonzero output,
    however small. Ragged G (5, 9, 21: tails of 1, 1 and 1 groups in the last
    quad), each call after a launch that leaves nonzero codes in LDS."""
    n = 40
    q = (1 << (W - 1)) - 1
    junk_x = torch.full((m, 4096), 30.0, dtype=torch.bfloat16, device=DEV)
    junk_w = torch.full((64, 4096 * W // 8), 0x5A, dtype=torch.uint8, device=DEV)
    junk_ws = torch.ones(64, device=DEV)
    configs = [_native.CONFIG_AUTO] + [c for c in range(_native.num_configs()) if _native.config_valid(c, m)]
    for G in (5, 9, 21):
        k = 64 * G
        gen = torch.Generator().manual_seed(100 * G + 10 * W + A + 1000 * m)
        x = torch.randn(m, k, generator=gen)
        x[:, 256:320] = x[:, 0:64]
        x = x.to(torch.bfloat16)
        scale = torch.rand(k, generator=gen) + 0.5
        scale[256:320] = scale[0:64]
        scale = scale.to(torch.bfloat16)
        wc = np.zeros((n, k), np.int8)
        c = torch.randint(-q, q + 1, (n, 64), generator=gen).numpy().astype(np.int8)
        wc[:, 0:64], wc[:, 256:320] = c, -c
        wsc = (torch.rand(n, generator=gen) * 0.05 + 0.01).numpy().astype(np.float32)
        w_dev = torch.from_numpy(O.pack_rows(wc, W)).to(DEV)
        ws_dev = torch.from_numpy(wsc).to(DEV)
        packed, a_scales, _ = O.quantize_groups(bits(x), A, "bf16")
        a_dev, s_dev = torch.from_numpy(packed).to(DEV), torch.from_numpy(a_scales).to(DEV)
        zero = np.zeros((m, n), np.uint16)
        for config in configs:
            for sc in (None, scale.to(DEV)):
                _native.grouped_forward(junk_x, junk_w, junk_ws, None, W, A, config=config)
                got = _native.grouped_forward(x.to(DEV), w_dev, ws_dev, None, W, A, input_scale=sc, config=config)
                np.testing.assert_array_equal(bits(got), zero, err_msg=f"G={G} config {config} scale={sc is not None}")
            got = _native.grouped_linear(a_dev, s_dev, w_dev, ws_dev, None, (m, k), W, A, config)
            np.testing.assert_array_equal(bits(got), zero, err_msg=f"G={G} config {config} (packed)")
