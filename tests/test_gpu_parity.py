"""GPU parity of the HIP path against the CPU oracle, through the C ABI.

Bar: packed activation codes, activation scales and int32 group dots are
bit-exact; the output is bit-exact against the oracle evaluated in the
library's canonical fp32 order (16 quad-aligned K-chunks); against the
reference's own float criterion (dequantize-then-matmul,
tests/test_kernels.py:42-48) it is within rtol = atol = 0.02; the max
abs/rel deviation from the reference's sequential fp32 order is reported and
bounded by 2 bf16 ulps (2 * 2^-8 relative) plus 1e-3 absolute.
"""
import numpy as np
import pytest
import torch

from actune_amd import _native
from oracle import oracle as O
from tests.helpers import PAIRS, bits, canonical_bounds, dtype_name, oracle_activation, oracle_weight, rel_err, seeded_inputs

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _packed_weight(w, W, A, ratios=None):
    codes, scale = oracle_weight(w, W, A, ratios)
    return codes, scale, torch.from_numpy(O.pack_rows(codes, W)).to(DEV), torch.from_numpy(scale).to(DEV)


# ---------------------------------------------------------------- quantizer
@pytest.mark.parametrize("A", [2, 4, 8])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("shape", [(1, 64), (17, 128), (3, 4096), (50, 1024), (64, 11008)])
def test_quantizer_bit_exact(A, dtype, shape):
    m, k = shape
    x, _, _ = seeded_inputs(m, k, 1, seed=m * 7 + k + A, dtype=dtype)
    x[0, :64] = 0  # an all-zero group
    packed, scales = _native.quantize_groups(x.to(DEV), A)
    want_p, want_s, _ = oracle_activation(x, A)
    np.testing.assert_array_equal(packed.cpu().numpy(), want_p)
    np.testing.assert_array_equal(scales.cpu().numpy(), want_s)


@pytest.mark.parametrize("A", [2, 4, 8])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_quantizer_fused_input_scale_bit_exact(A, dtype):
    x, _, _ = seeded_inputs(9, 384, 1, seed=A, dtype=dtype)
    scale = torch.linspace(0.3, 3.0, 384).to(dtype)
    packed, scales = _native.quantize_groups(x.to(DEV), A, scale.to(DEV))
    want_p, want_s, _ = oracle_activation(x, A, scale)
    np.testing.assert_array_equal(packed.cpu().numpy(), want_p)
    np.testing.assert_array_equal(scales.cpu().numpy(), want_s)
    # and it equals quantizing torch's own x / scale (layers.py:41-42)
    p2, s2 = _native.quantize_groups((x.to(DEV) / scale.to(DEV)).contiguous(), A)
    assert torch.equal(p2, packed) and torch.equal(s2, scales)


# ---------------------------------------------------------------- int32 dots
SHAPES = [(1, 64, 32), (17, 128, 96), (5, 320, 48), (16, 1024, 80), (3, 192, 16), (40, 256, 72)]


@pytest.mark.parametrize("W,A", PAIRS)
@pytest.mark.parametrize("shape", SHAPES)
def test_int32_group_dots_bit_exact_every_config(W, A, shape):
    m, k, n = shape
    x, w, _ = seeded_inputs(m, k, n, seed=W * 100 + A + m)
    a_packed, _, a_codes = oracle_activation(x, A)
    w_codes, _, w_dev, _ = _packed_weight(w, W, A)
    want = O.group_dots(a_codes, w_codes)
    a_dev = torch.from_numpy(a_packed).to(DEV)
    for config in range(_native.num_configs()):
        if not _native.config_valid(config, m):
            continue
        got = _native.grouped_dots(a_dev, w_dev, m, k, W, A, config).cpu().numpy()
        np.testing.assert_array_equal(got, want, err_msg=f"config {config}")


# ---------------------------------------------------------------- outputs
def _run_linear(x, w, b, W, A, config, out_dtype=None):
    a_packed, a_scales, a_codes = oracle_activation(x, A)
    w_codes, w_scale, w_dev, ws_dev = _packed_weight(w, W, A)
    a_dev = torch.from_numpy(a_packed).to(DEV)
    s_dev = torch.from_numpy(a_scales).to(DEV)
    bias = None
    if b is not None:
        bias = b.float() if A == 4 else b  # the reference's bias storage rule
    out = _native.grouped_linear(a_dev, s_dev, w_dev, ws_dev, None if bias is None else bias.to(DEV),
                                 (x.shape[0], x.shape[1]), W, A, config, out_dtype=out_dtype or x.dtype)
    return out, (a_codes, a_scales, w_codes, w_scale, None if bias is None else bias.float().numpy())


@pytest.mark.parametrize("W,A", PAIRS)
@pytest.mark.parametrize("shape", [(1, 64, 32), (17, 128, 96), (8, 4096, 64), (50, 1024, 48),
                                   # G = 21: a ragged last quad, and canonical chunks of 0 or 1 quads
                                   # (the prefill kernel's one-chunk-per-stage form)
                                   (12, 1344, 40), (70, 1344, 40)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_output_bit_exact_in_canonical_order(W, A, shape, with_bias):
    m, k, n = shape
    x, w, b = seeded_inputs(m, k, n, seed=W + 10 * A + m, bias=with_bias)
    G = k // 64
    outs = {}
    for config in range(_native.num_configs()):
        if not _native.config_valid(config, m):
            continue
        out, (ac, asc, wc, wsc, bf) = _run_linear(x, w, b, W, A, config)
        outs[config] = out
        want = O.linear(ac, asc, wc, wsc, bf, bounds=canonical_bounds(G))
        np.testing.assert_array_equal(bits(out), O.round_out(want, "bf16"), err_msg=f"config {config}")
    first = next(iter(outs.values()))
    assert all(torch.equal(first, o) for o in outs.values())  # every config bit-identical


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("n,offset", [(96, 0), (42, 0), (96, 1)])
def test_prefill_epilogue_store_forms(out_dtype, n, offset):
    """The prefill kernel stores a lane's four consecutive outputs in one
    vector store when N % 4 == 0 and the output pointer is aligned to four
    elements, and one element at a time otherwise (N = 42; an output view one
    element into its storage): every config valid at M = 70 matches the
    oracle bit for bit in each form."""
    m, k = 70, 320
    W, A = 4, 8
    x, w, b = seeded_inputs(m, k, n, seed=n + offset, bias=True)
    a_packed, a_scales, ac = oracle_activation(x, A)
    wc, wsc, w_dev, ws_dev = _packed_weight(w, W, A)
    a_dev = torch.from_numpy(a_packed).to(DEV)
    s_dev = torch.from_numpy(a_scales).to(DEV)
    want = O.round_out(O.linear(ac, a_scales, wc, wsc, b.float().numpy(), bounds=canonical_bounds(k // 64)),
                       dtype_name(out_dtype))
    for config in range(_native.num_configs()):
        if not _native.config_valid(config, m):
            continue
        store = torch.full((m * n + offset,), float("nan"), device=DEV, dtype=out_dtype)
        out = store[offset:].view(m, n)
        _native.grouped_linear(a_dev, s_dev, w_dev, ws_dev, b.to(DEV), (m, k), W, A, config, out=out,
                               out_dtype=out_dtype)
        np.testing.assert_array_equal(bits(out), want, err_msg=f"config {config}")
        if offset:
            assert torch.isnan(store[:offset]).all()  # nothing written before the view


@pytest.mark.parametrize("W", [2, 4, 8])
@pytest.mark.parametrize("m", [1, 2, 3])
def test_decode_ragged_tail_adds_nothing(W, m):
    """The decode kernel's last weight slot of the wave whose K-range ends at
    G also spans up to 3 groups past G (4 groups per slot at W2, 2 at W4).
    Their weights are the next row's bytes and their slab rows unwritten
    LDS, so each such group must get scale 0. The one-token path with x
    quantized in the launch once gave them the quantizer's 1e-8 floor scale
    instead (x reads past K are zeros): a run-dependent error of about 1e-8
    per output, below a bf16 ulp unless the output is 0 or near a rounding
    boundary. Here every output is exactly 0 (group 4 of x repeats group 0;
    each weight row holds codes c in group 0 and -c in group 4, in two
    canonical chunks, and zeros elsewhere), so any such term shows. G = 5..11
    and 21 under every decode config, each call after a launch that leaves
    nonzero codes in LDS."""
    A, n = 4, 48
    bf16 = torch.bfloat16
    junk_x = torch.full((m, 4096), 30.0, dtype=bf16, device=DEV)
    _, junk_w, _ = seeded_inputs(1, 4096, 64, seed=3)
    _, _, junk_dev, junk_ws = _packed_weight(junk_w, W, A)
    configs = [c for c in range(14, _native.num_configs()) if _native.config_valid(c, m)]
    q = (1 << (W - 1)) - 1  # symmetric code range, so -c is a code too
    fused = 0
    for G in list(range(5, 12)) + [21]:
        k = 64 * G
        gen = torch.Generator().manual_seed(100 * G + W + m)
        x = torch.randn(m, k, generator=gen)
        x[:, 256:320] = x[:, 0:64]
        x = x.to(bf16)
        wc = np.zeros((n, k), np.int8)
        c = torch.randint(-q, q + 1, (n, 64), generator=gen).numpy().astype(np.int8)
        wc[:, 0:64], wc[:, 256:320] = c, -c
        wsc = (torch.rand(n, generator=gen) * 0.05 + 0.01).numpy().astype(np.float32)
        w_dev = torch.from_numpy(O.pack_rows(wc, W)).to(DEV)
        ws_dev = torch.from_numpy(wsc).to(DEV)
        _, a_scales, ac = oracle_activation(x, A)
        want = O.round_out(O.linear(ac, a_scales, wc, wsc, None, bounds=canonical_bounds(G)), "bf16")
        assert not want.any()  # every output +0
        x_dev = x.to(DEV)
        for config in configs:
            fused += _native.forward_fuses_quantizer(m, n, k, W, A, bf16, config)
            _native.grouped_forward(junk_x, junk_dev, junk_ws, None, W, A, config=config)
            got = _native.grouped_forward(x_dev, w_dev, ws_dev, None, W, A, config=config)
            np.testing.assert_array_equal(bits(got), want, err_msg=f"G={G} config {config}")
    assert fused > 0  # the in-launch quantization ran


@pytest.mark.parametrize("W,A", PAIRS)
@pytest.mark.parametrize("shape", [(1, 64, 32), (17, 128, 96)])
def test_reference_float_criterion(W, A, shape):
    """tests/test_kernels.py:28-49 restated: nn.Linear init with bias, x ~ randn,
    output vs F.linear(activation_reference(x), q.float() * scale, bias)."""
    m, k, n = shape
    torch.manual_seed(7)
    lin = torch.nn.Linear(k, n, bias=True, dtype=torch.bfloat16)
    x = torch.randn(m, k, dtype=torch.bfloat16)
    out, (ac, asc, wc, wsc, bf) = _run_linear(x, lin.weight.detach(), lin.bias.detach(), W, A, _native.CONFIG_AUTO)
    exp = O.reference_float_linear(x.float().numpy(), A, wc, wsc, bf)
    exp_bf16 = O.bf16_bits_to_f32(O.f32_to_bf16_bits(exp))
    got = out.float().cpu().numpy()
    np.testing.assert_allclose(got, exp_bf16, rtol=0.02, atol=0.02)
    assert out.shape == (m, n)


@pytest.mark.parametrize("W,A", PAIRS)
def test_deviation_from_sequential_order_is_bounded(W, A):
    m, k, n = 8, 4096, 256
    x, w, _ = seeded_inputs(m, k, n, seed=3 * W + A)
    out, (ac, asc, wc, wsc, _) = _run_linear(x, w, None, W, A, _native.CONFIG_AUTO)
    seq = O.linear(ac, asc, wc, wsc)  # the reference kernels' sequential order
    got = out.float().cpu().numpy()
    abs_e, rel_e = rel_err(got, seq)
    print(f"W{W}A{A}: max abs {abs_e:.3e} max rel {rel_e:.3e} vs sequential fp32 order")
    assert np.all(np.abs(got - seq) <= 2 * 2.0**-8 * np.abs(seq) + 1e-3)


@pytest.mark.parametrize("out_dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("W,A", [(4, 8), (2, 4), (8, 2)])
def test_output_dtypes(out_dtype, W, A):
    m, k, n = 5, 256, 40
    x, w, b = seeded_inputs(m, k, n, seed=5, bias=True)
    out, (ac, asc, wc, wsc, bf) = _run_linear(x, w, b, W, A, _native.CONFIG_AUTO, out_dtype=out_dtype)
    want = O.linear(ac, asc, wc, wsc, bf, bounds=canonical_bounds(k // 64))
    np.testing.assert_array_equal(bits(out), O.round_out(want, dtype_name(out_dtype)))


def test_grouped_forward_matches_two_step_path():
    m, k, n, W, A = 6, 512, 64, 4, 8
    x, w, b = seeded_inputs(m, k, n, seed=9, bias=True)
    _, _, w_dev, ws_dev = _packed_weight(w, W, A)
    xd = x.to(DEV)
    one = _native.grouped_forward(xd, w_dev, ws_dev, b.to(DEV), W, A)
    p, s = _native.quantize_groups(xd, A)
    two = _native.grouped_linear(p, s, w_dev, ws_dev, b.to(DEV), xd, W, A)
    assert torch.equal(one, two)


# ---------------------------------------------------------------- full sizes
@pytest.mark.parametrize("m,n,k,W,A", [
    (1, 4096, 4096, 4, 8), (8, 11008, 4096, 4, 8), (1, 4096, 11008, 4, 8),
    (512, 4096, 4096, 8, 8), (512, 11008, 4096, 4, 8), (256, 2048, 2048, 4, 4),
    (50, 4096, 1024, 2, 4), (1, 256, 2048, 4, 4), (256, 2048, 16384, 4, 4),
    # C4 (Gemma-2B) remainder: gate/up 16384x2048 at M = 256 and 1, q at M = 1,
    # kv at M = 256, down at M = 1, and the bank's W4A8 / W4A2 versions
    (256, 16384, 2048, 4, 4), (1, 16384, 2048, 4, 4), (1, 2048, 2048, 4, 4), (256, 256, 2048, 4, 4),
    (1, 2048, 16384, 4, 4), (256, 16384, 2048, 4, 8), (1, 16384, 2048, 4, 8), (256, 2048, 2048, 4, 8),
    (256, 256, 2048, 4, 2), (1, 256, 2048, 4, 2),
])
def test_full_size_sampled_parity(m, n, k, W, A):
    """BASELINE shapes: every output row against the oracle on 64 sampled
    columns (bit-exact, canonical order), plus the quantizer on all of x."""
    x, w, _ = seeded_inputs(m, k, n, seed=m + n + k)
    xd = x.to(DEV)
    codes, scale = O.weight_codes(w.float().numpy(), W, A)
    w_dev = torch.from_numpy(O.pack_rows(codes, W)).to(DEV)
    ws_dev = torch.from_numpy(scale).to(DEV)
    out = _native.grouped_forward(xd, w_dev, ws_dev, None, W, A)
    p, s = _native.quantize_groups(xd, A)
    want_p, want_s, a_codes = oracle_activation(x, A)
    np.testing.assert_array_equal(p.cpu().numpy(), want_p)
    np.testing.assert_array_equal(s.cpu().numpy(), want_s)
    cols = np.random.default_rng(0).choice(n, size=min(64, n), replace=False)
    rows = np.arange(m) if m <= 64 else np.random.default_rng(1).choice(m, size=64, replace=False)
    want = O.linear(a_codes, want_s, codes, scale, None, bounds=canonical_bounds(k // 64), rows=rows, cols=cols)
    got = bits(out)[rows][:, cols]
    np.testing.assert_array_equal(got, O.round_out(want, "bf16"))


@pytest.mark.parametrize("m,n,k,W,A", [
    (1, 65536, 8192, 4, 8), (8, 8192, 65536, 4, 8), (3, 131072, 4096, 8, 8), (64, 100003, 1024, 2, 4),
    (1024, 4096, 65536, 8, 8), (1, 16, 262144, 4, 8),
])
def test_extreme_shapes_sampled_every_config(m, n, k, W, A):
    """Shapes far from the BASELINE ones, up to the buffer limits' order of
    magnitude (512 MiB of weights, K = 262144 = 4096 groups, N = 131072 and a
    ragged 100003): every config valid at M against the oracle on sampled
    columns and rows, the first and last of each included."""
    g = torch.Generator().manual_seed(m + n + k)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    codes, scale = O.weight_codes((torch.randn(n, k, generator=g) * 0.02).numpy(), W, A)
    w_dev = torch.from_numpy(O.pack_rows(codes, W)).to(DEV)
    ws_dev = torch.from_numpy(scale).to(DEV)
    rng = np.random.default_rng(0)
    cols = np.unique(np.concatenate([rng.choice(n, size=min(60, n), replace=False), [0, n - 1]]))
    rows = np.arange(m) if m <= 64 else np.unique(np.concatenate([rng.choice(m, size=60, replace=False), [0, m - 1]]))
    _, a_scales, a_codes = oracle_activation(x, A)
    want = O.round_out(O.linear(a_codes, a_scales, codes, scale, None, bounds=canonical_bounds(k // 64),
                                rows=rows, cols=cols), "bf16")
    xd = x.to(DEV)
    for config in [_native.CONFIG_AUTO] + [c for c in range(_native.num_configs()) if _native.config_valid(c, m)]:
        out = _native.grouped_forward(xd, w_dev, ws_dev, None, W, A, config=config)
        np.testing.assert_array_equal(bits(out)[rows][:, cols], want, err_msg=f"config {config}")


# ---------------------------------------------------------------- fused / siblings
@pytest.mark.parametrize("W,A", PAIRS)
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 12, 16])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_fused_small_m_equals_two_step(W, A, m, dtype):
    """Small-M (fused for M <= 4) and decode configs (fused for bf16 x up to
    M = 8, quantizer launch + packed codes otherwise): forward on x and the
    GEMM on the quantizer's codes both equal the oracle bit for bit, with and
    without the fused channel scale."""
    k, n = 704, 80  # G = 11: ragged chunks and a partial weight step
    x, w, b = seeded_inputs(m, k, n, seed=W * A + m, dtype=dtype, bias=True)
    _, _, w_dev, ws_dev = _packed_weight(w, W, A)
    xd, bd = x.to(DEV), b.to(DEV)
    wc, wsc = oracle_weight(w, W, A)
    for scale in (None, torch.linspace(0.5, 2.0, k).to(dtype)):
        sd = None if scale is None else scale.to(DEV)
        a_packed, a_scales, a_codes = oracle_activation(x, A, scale)
        want = O.round_out(O.linear(a_codes, a_scales, wc, wsc, b.float().numpy(), bounds=canonical_bounds(k // 64)),
                           dtype_name(dtype))
        p, s = _native.quantize_groups(xd, A, sd)
        for config in (0, 1, 2, 14, 15, 16):  # small-M and decode kernels
            fused = _native.grouped_forward(xd, w_dev, ws_dev, bd, W, A, input_scale=sd, config=config)
            two = _native.grouped_linear(p, s, w_dev, ws_dev, bd, xd, W, A, config)
            assert torch.equal(fused, two), (config, scale is None)
            np.testing.assert_array_equal(bits(fused), want, err_msg=f"config {config}")


@pytest.mark.parametrize("W,A", [(4, 8), (2, 4), (8, 8), (8, 2)])
@pytest.mark.parametrize("m", [1, 4, 8, 16])
@pytest.mark.parametrize("k", [4096, 8192, 11008])
def test_decode_full_ring_equals_small_m(W, A, m, k):
    """Decode configs at K where a wave's weight range fills its load ring
    (and, for K = 11008 with 4 or 8 waves, exceeds it: those run the small-M
    kernel; at M = 8 the longer ranges take the quantizer's codes) equal the
    small-M kernel bit for bit, with a ragged N."""
    n = 72
    x, w, b = seeded_inputs(m, k, n, seed=k + W * A + m, bias=True)
    _, _, w_dev, ws_dev = _packed_weight(w, W, A)
    xd, bd = x.to(DEV), b.to(DEV)
    want = _native.grouped_forward(xd, w_dev, ws_dev, bd, W, A, config=2)
    for config in (14, 15, 16):
        got = _native.grouped_forward(xd, w_dev, ws_dev, bd, W, A, config=config)
        assert torch.equal(got, want), config


@pytest.mark.parametrize("W,A", [(4, 8), (2, 2), (8, 4), (4, 4)])
@pytest.mark.parametrize("m", [1, 3, 6, 8])
def test_decode_full_ring_with_channel_scale(W, A, m):
    """K = 4096: every wave of the 4-wave (W2/W4) or 8-wave (W8) decode
    config fills its load ring exactly, which runs the bound-free slot
    pipeline; with and without the fused channel scale it equals quantize +
    GEMM and the oracle bit for bit (N ragged)."""
    k, n = 4096, 88
    x, w, b = seeded_inputs(m, k, n, seed=7 * W + A + m, bias=True)
    _, _, w_dev, ws_dev = _packed_weight(w, W, A)
    xd, bd = x.to(DEV), b.to(DEV)
    scale = torch.linspace(0.5, 2.0, k).to(torch.bfloat16)
    for sd in (None, scale.to(DEV)):
        p, s = _native.quantize_groups(xd, A, sd)
        ref = _native.grouped_linear(p, s, w_dev, ws_dev, bd, xd, W, A, 2)
        for config in (14, 15, 16):
            out = _native.grouped_forward(xd, w_dev, ws_dev, bd, W, A, input_scale=sd, config=config)
            assert torch.equal(out, ref), (config, sd is None)
    a_packed, a_scales, a_codes = oracle_activation(x, A, scale)
    wc, wsc = oracle_weight(w, W, A)
    want = O.linear(a_codes, a_scales, wc, wsc, b.float().numpy(), bounds=canonical_bounds(k // 64))
    np.testing.assert_array_equal(bits(out), O.round_out(want, "bf16"))


@pytest.mark.parametrize("m", [1, 4, 8, 50, 100])
@pytest.mark.parametrize("W,A", [(4, 8), (2, 4), (8, 2)])
def test_multi_target_equals_separate_calls(m, W, A):
    k = 512
    x, _, _ = seeded_inputs(m, k, 1, seed=m)
    xd = x.to(DEV)
    targets = []
    for j, n in enumerate((96, 32, 160)):
        _, w, b = seeded_inputs(1, k, n, seed=100 + j, bias=True)
        _, _, w_dev, ws_dev = _packed_weight(w, W, A)
        targets.append((w_dev, ws_dev, b.to(DEV), None))
    outs = _native.grouped_forward_multi(xd, targets, W, A)
    for (w_dev, ws_dev, bd, _), out in zip(targets, outs):
        assert torch.equal(out, _native.grouped_forward(xd, w_dev, ws_dev, bd, W, A))


# widths of q/k/v-like sibling targets, output widths, K
MIXED = [((4, 8, 4), (1024, 256, 256), 1024), ((2, 4), (96, 200), 512), ((8, 2, 4, 8), (64, 48, 160, 32), 4096),
         ((4, 8), (4096, 4096), 4096)]


@pytest.mark.parametrize("m", [1, 3, 8, 13, 50, 100])
@pytest.mark.parametrize("A", [4, 8, 2])
@pytest.mark.parametrize("case", range(len(MIXED)))
def test_mixed_width_multi_against_oracle(m, A, case):
    """Sibling targets of different weight widths at one A in one call (one
    decode launch where the kernel takes every width, else one quantization
    and a launch per width): every output equals its own single-width
    forward bit for bit and the oracle in the canonical order, with and
    without the channel scale."""
    widths, ns, k = MIXED[case]
    if m == 100 and k == 4096 and max(ns) == 4096:
        pytest.skip("covered at the smaller M (oracle time)")
    x, _, _ = seeded_inputs(m, k, 1, seed=m * 13 + A + case)
    scale = torch.linspace(0.5, 2.0, k).to(torch.bfloat16)
    xd = x.to(DEV)
    targets, oracle_side = [], []
    for j, (W, n) in enumerate(zip(widths, ns)):
        _, w, b = seeded_inputs(1, k, n, seed=900 + 10 * case + j, bias=j % 2 == 1)
        codes, wscale, w_dev, ws_dev = _packed_weight(w, W, A)
        targets.append((w_dev, ws_dev, None if b is None else b.to(DEV), None, W))
        oracle_side.append((codes, wscale, b))
    biases = {t[2] is None for t in targets}
    if len(biases) > 1:  # one bias dtype (or none) per call: give every target a bias
        targets = [(t[0], t[1], torch.zeros(t[0].shape[0], device=DEV).to(torch.bfloat16) if t[2] is None else t[2],
                    None, t[4]) for t in targets]
    cols_all = max(ns) <= 1024
    for sd in (None, scale.to(DEV)):
        outs = _native.grouped_forward_multi(xd, targets, widths[0], A, input_scale=sd)
        _, a_scales, a_codes = oracle_activation(x, A, None if sd is None else scale)
        for (w_dev, ws_dev, bd, _, W), (codes, wscale, _), out in zip(targets, oracle_side, outs):
            single = _native.grouped_forward(xd, w_dev, ws_dev, bd, W, A, input_scale=sd)
            assert torch.equal(out, single), (W, sd is None)
            n = w_dev.shape[0]
            cols = None if cols_all else np.sort(np.random.default_rng(n + m).choice(n, size=64, replace=False))
            bias = None if bd is None else bd.float().cpu().numpy()
            want = O.linear(a_codes, a_scales, codes, wscale, bias, bounds=canonical_bounds(k // 64), cols=cols)
            got = bits(out) if cols is None else bits(out)[:, cols]
            np.testing.assert_array_equal(got, O.round_out(want, "bf16"), err_msg=f"W{W} n={n}")


@pytest.mark.parametrize("config", [-1, 14, 15, 16, 0, 7, 10])
def test_mixed_width_multi_explicit_configs(config):
    """Mixed widths under explicit configs: the decode configs (one launch
    where each width fits, else per-width launches), the small-M, streaming
    and prefill configs (per-width launches on one quantization): outputs
    equal the single-width calls with the same config."""
    m, k, A = 8, 1024, 4
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(config + 50)).to(torch.bfloat16).to(DEV)
    targets = []
    for j, (W, n) in enumerate(zip((4, 8, 2), (256, 64, 128))):
        _, w, _ = seeded_inputs(1, k, n, seed=950 + j)
        _, _, w_dev, ws_dev = _packed_weight(w, W, A)
        targets.append((w_dev, ws_dev, None, None, W))
    outs = _native.grouped_forward_multi(x, targets, 4, A, config=config)
    for (w_dev, ws_dev, _, _, W), out in zip(targets, outs):
        assert torch.equal(out, _native.grouped_forward(x, w_dev, ws_dev, None, W, A, config=config)), W


@pytest.mark.parametrize("m", [1, 8])
@pytest.mark.parametrize("n,k,count", [(4096, 4096, 3), (11008, 4096, 2)])
def test_full_size_sibling_launches_against_oracle(m, n, k, count):
    """The sibling launches the C2 benchmark times (q/k/v 3 x 4096x4096 and
    gate/up 2 x 11008x4096, W4A8, default config, M = 1 and 8): each target
    against the oracle on 64 sampled columns, bit-exact in the canonical
    order, and equal to its own single-target forward."""
    W, A = 4, 8
    x, _, _ = seeded_inputs(m, k, 1, seed=n + m)
    xd = x.to(DEV)
    _, a_scales, a_codes = oracle_activation(x, A)
    targets, oracle_side = [], []
    for j in range(count):
        _, w, _ = seeded_inputs(1, k, n, seed=7000 + 10 * j + m)
        codes, scale, w_dev, ws_dev = _packed_weight(w, W, A)
        targets.append((w_dev, ws_dev, None, None))
        oracle_side.append((codes, scale))
    outs = _native.grouped_forward_multi(xd, targets, W, A)
    cols = np.sort(np.random.default_rng(n + m).choice(n, size=64, replace=False))
    for (w_dev, ws_dev, _, _), (codes, scale), out in zip(targets, oracle_side, outs):
        want = O.linear(a_codes, a_scales, codes, scale, None, bounds=canonical_bounds(k // 64), cols=cols)
        np.testing.assert_array_equal(bits(out)[:, cols], O.round_out(want, "bf16"))
        assert torch.equal(out, _native.grouped_forward(xd, w_dev, ws_dev, None, W, A))


@pytest.mark.parametrize("W,A", PAIRS)
@pytest.mark.parametrize("m", [1, 3, 8, 13, 16])
def test_streaming_fused_equals_two_step(W, A, m):
    """Streaming configs (fused quantizer for M <= 4, LDS-staged packed
    activations above) equal quantize + GEMM and the oracle bit for bit
    (bf16 and f16, with and without the channel scale)."""
    k, n = 1344, 200  # G = 21: uneven wave ranges; N not a multiple of 16
    for dtype in (torch.bfloat16, torch.float16):
        x, w, b = seeded_inputs(m, k, n, seed=W * 11 + A + m, dtype=dtype, bias=True)
        _, _, w_dev, ws_dev = _packed_weight(w, W, A)
        xd, bd = x.to(DEV), b.to(DEV)
        scale = torch.linspace(0.5, 2.0, k).to(dtype)
        for sd in (None, scale.to(DEV)):
            p, s = _native.quantize_groups(xd, A, sd)
            ref = _native.grouped_linear(p, s, w_dev, ws_dev, bd, xd, W, A, 3)
            for config in (7, 8, 9):
                out = _native.grouped_forward(xd, w_dev, ws_dev, bd, W, A, input_scale=sd, config=config)
                assert torch.equal(out, ref), (dtype, config, sd is None)
        a_packed, a_scales, a_codes = oracle_activation(x, A, scale)
        wc, wsc = oracle_weight(w, W, A)
        want = O.linear(a_codes, a_scales, wc, wsc, b.float().numpy(), bounds=canonical_bounds(k // 64))
        np.testing.assert_array_equal(bits(out), O.round_out(want, dtype_name(dtype)))


# ---------------------------------------------------------------- activation regimes
def _regime(x: torch.Tensor, regime: str) -> torch.Tensor:
    xf = x.float()
    if regime == "small":
        xf = xf * 1e-4
    elif regime == "large":
        xf = xf * 1e3
    elif regime == "near_floor":  # group maxima around the 1e-8 scale floor
        xf = xf * 3e-9
    elif regime == "tiny":  # every group below the floor: all codes 0
        xf = xf * 1e-30
    elif regime == "zero_rows":
        xf[::2] = 0
    return xf.to(x.dtype)


@pytest.mark.parametrize("regime", ["small", "large", "near_floor", "tiny", "zero_rows"])
@pytest.mark.parametrize("W,A", [(4, 8), (2, 4), (8, 2)])
def test_activation_regimes_bit_exact_every_config(regime, W, A):
    """Activation magnitudes of 1e-4, 1e3, around and below the quantizer's
    1e-8 scale floor, and all-zero token rows, through every kernel config
    valid for M = 1, 8 and 80: codes, scales and outputs equal the oracle bit
    for bit."""
    k, n = 1024, 96
    wsets = {}
    for m in (1, 8, 80):
        x, w, b = seeded_inputs(m, k, n, seed=31 * m + W + A, bias=True)
        x = _regime(x, regime)
        if m not in wsets:
            wsets[m] = _packed_weight(w, W, A)
        wc, wsc, w_dev, ws_dev = wsets[m]
        xd, bd = x.to(DEV), b.to(DEV)
        want_p, want_s, a_codes = oracle_activation(x, A)
        p, s = _native.quantize_groups(xd, A)
        np.testing.assert_array_equal(p.cpu().numpy(), want_p)
        np.testing.assert_array_equal(s.cpu().numpy(), want_s)
        want = O.round_out(O.linear(a_codes, want_s, wc, wsc, b.float().numpy(), bounds=canonical_bounds(k // 64)), "bf16")
        for config in range(_native.num_configs()):
            if not _native.config_valid(config, m):
                continue
            out = _native.grouped_forward(xd, w_dev, ws_dev, bd, W, A, config=config)
            np.testing.assert_array_equal(bits(out), want, err_msg=f"m={m} config={config}")


@pytest.mark.parametrize("W,A", [(4, 8), (2, 4), (8, 2)])
@pytest.mark.parametrize("m", [2, 4, 5, 8, 12, 16])
@pytest.mark.parametrize("n", [6000, 10200])
def test_decode_shared_row_tiles(W, A, m, n):
    """Decode launches (4- and 8-token tiles) wide enough to share a
    workgroup between two (N = 6000) or four (N = 10200) 16-row tiles, N
    ragged: x quantized in the launch (with and without the channel scale)
    and the quantizer's codes both equal the oracle bit for bit, and so do
    three sibling targets of ragged widths in one launch."""
    k = 1024
    x, w, b = seeded_inputs(m, k, n, seed=n + 13 * W + A + m, bias=True)
    wc, wsc, w_dev, ws_dev = _packed_weight(w, W, A)
    xd, bd = x.to(DEV), b.to(DEV)
    scale = torch.linspace(0.5, 2.0, k).to(torch.bfloat16)
    for sc in (None, scale):
        sd = None if sc is None else sc.to(DEV)
        _, a_scales, a_codes = oracle_activation(x, A, sc)
        want = O.round_out(O.linear(a_codes, a_scales, wc, wsc, b.float().numpy(), bounds=canonical_bounds(k // 64)), "bf16")
        fused = _native.grouped_forward(xd, w_dev, ws_dev, bd, W, A, input_scale=sd, config=16)
        np.testing.assert_array_equal(bits(fused), want, err_msg=f"fused scale={sc is not None}")
        p, s = _native.quantize_groups(xd, A, sd)
        for config in (15, 16):
            packed = _native.grouped_linear(p, s, w_dev, ws_dev, bd, xd, W, A, config)
            np.testing.assert_array_equal(bits(packed), want, err_msg=f"packed config={config}")
    # three siblings of ragged widths around n / 3 share one launch (the
    # narrower ones leave workgroups and tiles of the shared grid empty)
    nt = (n // 3) // 8 * 8
    targets, wants = [], []
    _, a_scales, a_codes = oracle_activation(x, A)
    for j, nj in enumerate((nt, nt // 4 // 8 * 8, nt + 40)):
        _, wj, bj = seeded_inputs(1, k, nj, seed=500 + j + n, bias=True)
        wcj, wscj, wdj, wsdj = _packed_weight(wj, W, A)
        targets.append((wdj, wsdj, bj.to(DEV), None))
        wants.append(O.round_out(O.linear(a_codes, a_scales, wcj, wscj, bj.float().numpy(),
                                          bounds=canonical_bounds(k // 64)), "bf16"))
    outs = _native.grouped_forward_multi(xd, targets, W, A, config=16)
    for j, (out, want) in enumerate(zip(outs, wants)):
        np.testing.assert_array_equal(bits(out), want, err_msg=f"sibling {j}")


@pytest.mark.parametrize("W,A", [(4, 8), (2, 4), (8, 4)])
@pytest.mark.parametrize("m", [17, 24, 50, 64, 100, 256])
@pytest.mark.parametrize("k", [1024, 4096])
def test_decode_token_blocks(W, A, m, k):
    """M = 17..1024 runs the decode kernel in 16-token blocks (the last one
    ragged): the GEMM on the quantizer's codes with 4, 8 and 16 waves, the
    forward on bf16 x with each of them (x quantized per block inside the
    launch where a wave's K-range is at most 4 groups, with and without the
    channel scale) and the default forward equal the oracle bit for bit (N
    ragged)."""
    n = 700
    x, w, b = seeded_inputs(m, k, n, seed=m * 7 + k + W * A, bias=True)
    wc, wsc, w_dev, ws_dev = _packed_weight(w, W, A)
    xd, bd = x.to(DEV), b.to(DEV)
    _, a_scales, a_codes = oracle_activation(x, A)
    want = O.round_out(O.linear(a_codes, a_scales, wc, wsc, b.float().numpy(), bounds=canonical_bounds(k // 64)), "bf16")
    p, s = _native.quantize_groups(xd, A)
    for config in (14, 15, 16):
        out = _native.grouped_linear(p, s, w_dev, ws_dev, bd, xd, W, A, config)
        np.testing.assert_array_equal(bits(out), want, err_msg=f"config {config}")
    np.testing.assert_array_equal(bits(_native.grouped_forward(xd, w_dev, ws_dev, bd, W, A)), want)
    scale = torch.linspace(0.5, 2.0, k).to(torch.bfloat16)
    _, sa_scales, sa_codes = oracle_activation(x, A, scale)
    want_s = O.round_out(O.linear(sa_codes, sa_scales, wc, wsc, b.float().numpy(), bounds=canonical_bounds(k // 64)), "bf16")
    fused_any = False
    for config in (14, 15, 16):
        fused_any |= _native.forward_fuses_quantizer(m, n, k, W, A, torch.bfloat16, config)
        out = _native.grouped_forward(xd, w_dev, ws_dev, bd, W, A, config=config)
        np.testing.assert_array_equal(bits(out), want, err_msg=f"forward config {config}")
        out = _native.grouped_forward(xd, w_dev, ws_dev, bd, W, A, input_scale=scale.to(DEV), config=config)
        np.testing.assert_array_equal(bits(out), want_s, err_msg=f"forward config {config}, channel scale")
    # at K = 1024 the in-launch quantization is light up to M = 100 here
    assert fused_any or k != 1024 or m > 100
