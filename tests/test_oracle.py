"""Pins the CPU oracle against answers fixed by the mathematics.

The reference ships no golden vectors for this path (its only kernel test is a
0.02-tolerance GPU comparison, tests/test_kernels.py:28-49), so every oracle
function is pinned here by hand-derived known answers, exact-rational
arithmetic, brute force on tiny inputs and invariants, chosen so that a
plausible mistake (round-half-away instead of half-even, reciprocal-multiply
instead of IEEE division, a missing FMA, a wrong bit offset, a transposed
operand) fails at least one check.
"""
from fractions import Fraction
import itertools

import numpy as np
import pytest

from oracle import oracle as O


def f32_round(q: Fraction) -> np.float32:
    """Exact round-to-nearest-even of a rational to float32 (independent of
    the C oracle): pick the nearest of the neighbouring float32 values."""
    c = np.float32(float(q))
    cands = {c, np.nextafter(c, np.float32(np.inf)), np.nextafter(c, np.float32(-np.inf))}
    best = None
    for v in cands:
        err = abs(Fraction(float(v)) - q)
        key = (err, int(np.asarray(v, np.float32).view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, v)
    return np.float32(best[1])


def rint_half_even(q: Fraction) -> int:
    f = q.numerator // q.denominator
    r = q - f
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and f % 2):
        return f + 1
    return f


def bf16(vals):
    return O.f32_to_bf16_bits(np.asarray(vals, np.float32))


def one_group(vals):
    g = np.zeros(64, np.float32)
    g[:len(vals)] = vals
    return bf16(g)[None, :]


# ------------------------------------------------------------------ dtypes
def test_bf16_rounding_known_answers():
    # 1 + 2^-8 is a tie between 0x3F80 (even) and 0x3F81 -> 0x3F80;
    # 1 + 3*2^-8 is a tie between 0x3F81 and 0x3F82 (even) -> 0x3F82.
    got = O.round_out(np.array([1.0, 1 + 2**-8, 1 + 3 * 2**-8, -2.0], np.float32), "bf16")
    assert got.tolist() == [0x3F80, 0x3F80, 0x3F82, 0xC000]
    assert O.f32_to_bf16_bits(np.array([1 + 2**-8, 1 + 3 * 2**-8], np.float32)).tolist() == [0x3F80, 0x3F82]


def test_f16_rounding_known_answers():
    vals = np.array([65519.0, 65520.0, 2**-25, 3 * 2**-25, 1.0, -0.5], np.float32)
    assert O.round_out(vals, "f16").tolist() == [0x7BFF, 0x7C00, 0x0000, 0x0002, 0x3C00, 0xB800]


# ------------------------------------------------------------------ quantizer
def test_a2_half_even_ties_and_packing():
    x = one_group([1.0, -1.0, 0.5, -0.5, 0.75, -0.75, 0.25, -0.25])
    packed, s, c = O.quantize_groups(x, 2)
    assert s.tolist() == [[1.0]]  # p = 1, s = amax / 1
    assert c[0, :8].tolist() == [1, -1, 0, 0, 1, -1, 0, 0]  # 0.5 -> 0 (half-even)
    assert not c[0, 8:].any()
    # 4 codes per byte at bit (k%4)*2: 1 | 3<<2 = 0x0D
    assert packed[0, :2].tolist() == [0x0D, 0x0D] and not packed[0, 2:].any()


def test_a4_known_codes_and_nibbles():
    # amax = 0.875 = 7 * 2^-3 so s = 0.125 exactly; quotients are exact.
    x = one_group([0.875, -0.875, 0.4375, 0.3125, -0.3125, 0.8125, -0.0625, 0.1875])
    packed, s, c = O.quantize_groups(x, 4)
    assert s.tolist() == [[0.125]]
    assert c[0, :8].tolist() == [7, -7, 4, 2, -2, 6, 0, 2]
    assert packed[0, :4].tolist() == [0x97, 0x24, 0x6E, 0x20]


def test_a8_known_codes_and_bytes():
    x = one_group([127, -127, 126.5, 125.5, -125.5, 0.5, 1.5, -2.5])
    packed, s, c = O.quantize_groups(x, 8)
    assert s.tolist() == [[1.0]]
    assert c[0, :8].tolist() == [127, -127, 126, 126, -126, 0, 2, -2]
    assert packed[0, :8].tolist() == [0x7F, 0x81, 0x7E, 0x7E, 0x82, 0x00, 0x02, 0xFE]


@pytest.mark.parametrize("A", [2, 4, 8])
def test_zero_and_tiny_groups_clamp_amax(A):
    p = (1 << (A - 1)) - 1
    x = np.zeros((1, 128), np.uint16)
    x[0, 64:] = bf16(np.full(64, 1e-30, np.float32))  # below the 1e-8 floor
    _, s, c = O.quantize_groups(x, A)
    want = f32_round(Fraction(float(np.float32(1e-8))) / p)
    assert s[0].tolist() == [want, want]
    assert not c.any()


def test_ieee_division_not_reciprocal_multiply():
    # Find inputs where fl(v / s) and fl(v * fl(1/s)) round to different
    # codes; the oracle must follow the exact quotient (calibration.py:14).
    rng = np.random.default_rng(3)
    hits = 0
    for _ in range(4000):
        vals = rng.standard_normal(64).astype(np.float32) * 3
        vals = O.bf16_bits_to_f32(bf16(vals))
        amax = float(np.max(np.abs(vals)))
        s = f32_round(Fraction(amax) / 127)
        inv = f32_round(1 / Fraction(float(s)))
        exact = [rint_half_even(Fraction(float(f32_round(Fraction(float(v)) / Fraction(float(s)))))) for v in vals]
        recip = [rint_half_even(Fraction(float(f32_round(Fraction(float(v)) * Fraction(float(inv)))))) for v in vals]
        if exact != recip:
            _, so, co = O.quantize_groups(bf16(vals)[None, :], 8)
            assert so[0, 0] == s
            assert co[0].tolist() == exact
            hits += 1
            if hits == 3:
                break
    assert hits == 3


def test_input_scale_rounds_quotient_to_dtype():
    # 1/3 in bf16 is 0x3EAB = 0.333984375 (layers.py:41-42 then quantize).
    x = one_group([1.0, -0.5])
    scale = bf16(np.full(64, 3.0, np.float32))
    _, s, c = O.quantize_groups(x, 8, input_scale=scale)
    amax = Fraction(0.333984375)
    assert s[0, 0] == f32_round(amax / 127)
    # -0.5/3 -> bf16 0xBE2B = -0.1669921875
    q = f32_round(Fraction(-0.1669921875) / Fraction(float(s[0, 0])))
    assert c[0, :2].tolist() == [127, rint_half_even(Fraction(float(q)))]


@pytest.mark.parametrize("A", [2, 4, 8])
def test_quantizer_invariants_random(A):
    rng = np.random.default_rng(A)
    x = rng.standard_normal((5, 256)).astype(np.float32)
    x[:, rng.integers(0, 256, 4)] *= 10
    xb = bf16(x)
    packed, s, c = O.quantize_groups(xb, A)
    p = (1 << (A - 1)) - 1
    v = O.bf16_bits_to_f32(xb).reshape(5, 4, 64)
    cg = c.reshape(5, 4, 64).astype(np.int32)
    assert cg.min() >= -p - 1 and cg.max() <= p
    at_max = np.abs(v) == np.abs(v).max(-1, keepdims=True)
    assert (np.abs(cg[at_max]) == p).all()
    err = np.abs(cg * s[:, :, None] - v)
    assert (err <= s[:, :, None] * 0.5 * (1 + 1e-6)).all()
    np.testing.assert_array_equal(O.unpack_rows(packed, A, 256), c)
    np.testing.assert_array_equal(O.pack_rows(c, A), packed)


# ------------------------------------------------------------------ weights
def test_w4_known_codes_and_clip():
    w = np.zeros((2, 64), np.float32)
    w[0, :4] = [7.0, -3.5, 2.5, 1.0]
    w[1, :3] = [7.0, -7.0, 1.0]
    c, s = O.weight_codes(w, 4, 8)
    assert s.tolist() == [1.0, 1.0]
    assert c[0, :4].tolist() == [7, -4, 2, 1]
    c, s = O.weight_codes(w, 4, 8, clip_ratios=0.5)  # s = 3.5/7 = 0.5
    assert s.tolist() == [0.5, 0.5]
    assert c[1, :3].tolist() == [7, -8, 2]  # +-14 clamps to [-8, 7]


def test_w2_known_codes_and_clip():
    w = np.zeros((1, 64), np.float32)
    w[0, :6] = [4.0, -4.0, 2.0, -2.0, 1.0, 3.0]
    c, s = O.weight_codes(w, 2, 8)
    assert s.tolist() == [4.0]
    assert c[0, :6].tolist() == [1, -1, 0, 0, 0, 1]  # 0.5 -> 0, -0.5 -> 0, 0.75 -> 1
    c, s = O.weight_codes(w, 2, 4, clip_ratios=[0.5])
    assert s.tolist() == [2.0]
    assert c[0, :6].tolist() == [1, -2, 1, -1, 0, 1]  # 2 -> 1 (clamp), 0.5 -> 0, 1.5 -> 2 -> 1


def test_w8a8_ignores_clip_ratios():
    w = np.zeros((1, 64), np.float32)
    w[0, :4] = [127.0, -64.5, 63.5, 0.5]
    c, s = O.weight_codes(w, 8, 8, clip_ratios=0.5)
    c2, s2 = O.weight_codes(w, 8, 2)
    assert s.tolist() == [1.0] and s2.tolist() == [1.0]
    assert c[0, :4].tolist() == [127, -64, 64, 0]
    np.testing.assert_array_equal(c, c2)


def test_w8a4_nested_codes():
    w = np.zeros((2, 64), np.float32)
    w[0, :4] = [7.0, -7.0, 2.3, -0.7]
    w[1, :2] = [7.0, -7.0]
    c, s = O.weight_codes(w, 8, 4)
    assert s.tolist() == [1.0 / 16, 1.0 / 16]
    # 2.3f: q4 = 2, 16*(2.29999995 - 2) = 4.7999992 -> 5 -> 37
    # -0.7f: q4 = -1, 16*(-0.69999999 + 1) = 4.8000002 -> 5 -> -11
    assert c[0, :4].tolist() == [112, -112, 37, -11]
    # ratio 0.5: s4 = 0.5. +7 -> t = 14, q4 = 7, residual 16*(14-7) = 112
    # clamps to 7 -> 119. -7 -> q4 = -8 (clamped); residual bounded to >= 0 -> -128
    c, s = O.weight_codes(w, 8, 4, clip_ratios=0.5)
    assert s.tolist() == [0.5 / 16, 0.5 / 16]
    assert c[1, :2].tolist() == [119, -128]
    q4 = np.floor_divide(c.astype(np.int32) + 8, 16)
    assert (np.abs(c.astype(np.int32)) <= 128).all() and (q4 >= -8).all() and (q4 <= 7).all()


def test_clip_ratio_validation_messages():
    w = np.ones((3, 64), np.float32)
    with pytest.raises(ValueError, match="expected 3"):
        O.weight_codes(w, 4, 8, clip_ratios=[0.5, 0.5])
    with pytest.raises(ValueError, match="finite"):
        O.weight_codes(w, 2, 8, clip_ratios=float("nan"))
    with pytest.raises(ValueError, match=r"\(0, 1\]"):
        O.weight_codes(w, 4, 4, clip_ratios=1.5)


@pytest.mark.parametrize("bits,codes,expect", [
    (4, [1, -1], [0xF1]),
    (2, [1, -1, -2, 0], [0x2D]),
    (8, [-128, 127], [0x80, 0x7F]),
])
def test_pack_rows_known_bytes(bits, codes, expect):
    c = np.zeros((1, 64), np.int8)
    c[0, :len(codes)] = codes
    assert O.pack_rows(c, bits)[0, :len(expect)].tolist() == expect


# ------------------------------------------------------------------ GEMM
def test_group_dots_brute_force():
    rng = np.random.default_rng(0)
    a = rng.integers(-128, 128, (3, 192), dtype=np.int8)
    w = rng.integers(-8, 8, (4, 192), dtype=np.int8)
    d = O.group_dots(a, w)
    for m, n, g in itertools.product(range(3), range(4), range(3)):
        want = sum(int(a[m, k]) * int(w[n, k]) for k in range(64 * g, 64 * g + 64))
        assert d[m, n, g] == want
    # subset selection and extreme magnitudes: 64 * (-128) * (-128) = 2^20
    a2 = np.full((2, 64), -128, np.int8)
    w2 = np.full((3, 64), -128, np.int8)
    w2[1] = 127
    assert O.group_dots(a2, w2, rows=[1], cols=[0, 1])[0, :, 0].tolist() == [2**20, -64 * 128 * 127]


def _fma(a, b, c):
    return f32_round(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def test_epilogue_uses_fused_multiply_add():
    rng = np.random.default_rng(1)
    fused_differs = 0
    for _ in range(300):
        d = rng.integers(-5000, 5000, 2).astype(np.int32)
        s = rng.uniform(1e-3, 1.0, 2).astype(np.float32)
        ws = np.float32(rng.uniform(0.01, 1.0))
        acc0 = f32_round(Fraction(int(d[0])) * Fraction(float(s[0])))
        acc1 = _fma(int(d[1]), s[1], acc0)
        want = f32_round(Fraction(float(acc1)) * Fraction(float(ws)))
        got = O.group_epilogue(d.reshape(1, 1, 2), s.reshape(1, 2), np.array([ws]))
        assert got[0, 0] == want
        unfused = f32_round(Fraction(float(f32_round(Fraction(int(d[1])) * Fraction(float(s[1]))))) + Fraction(float(acc0)))
        fused_differs += unfused != acc1
        bias = np.float32(rng.uniform(-1, 1))
        got_b = O.group_epilogue(d.reshape(1, 1, 2), s.reshape(1, 2), np.array([ws]), np.array([bias]))
        assert got_b[0, 0] == _fma(acc1, ws, bias)
    assert fused_differs > 0  # the cases above actually distinguish fma from mul+add


def test_epilogue_chunked_order():
    d = np.array([[[7, -3, 11, 5]]], np.int32)
    s = np.array([[0.1, 0.3, 0.7, 0.9]], np.float32)
    got = O.group_epilogue(d, s, np.array([1.0], np.float32), bounds=[0, 1, 1, 4])
    p0 = f32_round(Fraction(7) * Fraction(float(s[0, 0])))
    p2 = f32_round(Fraction(-3) * Fraction(float(s[0, 1])))
    p2 = _fma(11, s[0, 2], p2)
    p2 = _fma(5, s[0, 3], p2)
    want = f32_round(Fraction(float(p0)) + Fraction(float(p2)))  # + the empty chunk's +0
    assert got[0, 0] == want
    assert O.chunk_bounds(4, 2, 3).tolist() == [0, 0, 2, 4]
    assert O.chunk_bounds(172, 2, 8).tolist()[-1] == 172


def test_exact_sum_when_everything_is_representable():
    # Scales that are powers of two make every product and partial sum exact.
    a = np.ones((1, 256), np.int8)
    w = np.ones((1, 256), np.int8)
    s = np.array([[0.5, 0.25, 0.125, 2.0]], np.float32)
    y = O.linear(a, s, w, np.array([0.5], np.float32))
    assert y[0, 0] == 64 * (0.5 + 0.25 + 0.125 + 2.0) * 0.5


@pytest.mark.parametrize("shape", [(1, 64, 32), (17, 128, 96)])
@pytest.mark.parametrize("W", [2, 4, 8])
@pytest.mark.parametrize("A", [2, 4, 8])
def test_oracle_meets_reference_float_criterion(shape, W, A):
    """tests/test_kernels.py:28-49 restated on the CPU oracle: nn.Linear-like
    init with bias, x ~ randn, rtol = atol = 0.02 against float dequant-matmul."""
    m, k, n = shape
    rng = np.random.default_rng(7)
    bound = 1 / np.sqrt(k)
    wf = O.bf16_bits_to_f32(bf16(rng.uniform(-bound, bound, (n, k))))
    bias = O.bf16_bits_to_f32(bf16(rng.uniform(-bound, bound, n)))
    xb = bf16(rng.standard_normal((m, k)))
    x = O.bf16_bits_to_f32(xb)
    q, ws = O.weight_codes(wf, W, A)
    _, s, c = O.quantize_groups(xb, A)
    y = O.linear(c, s, q, ws, bias)
    out = O.bf16_bits_to_f32(O.round_out(y, "bf16"))
    exp = O.bf16_bits_to_f32(bf16(O.reference_float_linear(x, A, q, ws, bias)))
    np.testing.assert_allclose(out, exp, rtol=0.02, atol=0.02)


def test_f16_widening_known_answers():
    """oracle_f16_to_f32 (f16 x and channel scales): normals, subnormals,
    signed zero, infinities and NaN, each against its value fixed by the
    IEEE binary16 definition."""
    cases = {0x3C00: 1.0, 0xC000: -2.0, 0x0001: 2.0**-24, 0x03FF: 1023 * 2.0**-24, 0x0400: 2.0**-14,
             0x7BFF: 65504.0, 0x3555: (1 + 0x155 / 1024) * 2.0**-2,
             0x7C00: float("inf"), 0xFC00: float("-inf"), 0x0000: 0.0}
    got = O.f16_bits_to_f32(np.array(list(cases), np.uint16))
    for (b, want), g in zip(cases.items(), got):
        assert g == np.float32(want), hex(b)
    neg_zero = O.f16_bits_to_f32(np.array([0x8000], np.uint16))[0]
    assert neg_zero == 0.0 and np.signbit(neg_zero)
    assert np.isnan(O.f16_bits_to_f32(np.array([0x7E00, 0xFE01], np.uint16))).all()


def test_f16_widening_all_patterns_match_ieee_conversion():
    """Every finite f16 bit pattern widens to the value numpy's binary16
    conversion gives (an exact conversion: every f16 is an f32)."""
    b = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    finite = (b & 0x7C00) != 0x7C00
    want = b[finite].view(np.float16).astype(np.float32)
    got = O.f16_bits_to_f32(b[finite])
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
