"""Pins of the tokenwise oracle (oracle/tokenwise_oracle.c and the K-major
packers in oracle/oracle.py) against answers fixed by the mathematics:
exact rational arithmetic with an independent round-to-nearest-even fp32
rounding, hand-derived packed bytes, and brute-force integer dots."""
from fractions import Fraction

import numpy as np
import pytest

from oracle import oracle as O


def rn32(q: Fraction) -> np.float32:
    """Round a rational to the nearest fp32 (ties to even), normal range,
    with integer arithmetic only."""
    if q == 0:
        return np.float32(0.0)
    sign = -1 if q < 0 else 1
    q = abs(q)
    e = q.numerator.bit_length() - q.denominator.bit_length()
    if Fraction(2) ** e > q:
        e -= 1
    # q in [2^e, 2^(e+1)): 24 significant bits -> scale by 2^(23 - e)
    scaled = q * Fraction(2) ** (23 - e)
    lo = scaled.numerator // scaled.denominator
    rem = scaled - lo
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and lo % 2):
        lo += 1
    return np.float32(sign * lo * 2.0 ** (e - 23))


def rint_even(q: Fraction) -> int:
    lo = q.numerator // q.denominator
    rem = q - lo
    return lo + 1 if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and lo % 2) else lo


F = lambda v: Fraction(float(v))  # noqa: E731


def test_reciprocal_constants_match_both_reference_forms():
    """torch's GPU tensor/scalar division uses 1.0f / p computed in fp32;
    Triton rounds the Python double 1.0 / p to fp32. Both equal the correctly
    rounded reciprocal for p = 127 and p = 7."""
    for p in (127, 7):
        exact = rn32(Fraction(1, p))
        assert O.tw_recip(p) == exact
        assert rn32(Fraction(1.0 / p)) == exact  # double first, then fp32


def _bf16_row(vals):
    return O.f32_to_bf16_bits(np.asarray(vals, np.float32))[None, :]


def _find_recip_case(p):
    """A bf16 amax whose reciprocal-multiply scale differs from the IEEE
    quotient (the reference's note: about 10% of rows for p = 127)."""
    r = rn32(Fraction(1, p))
    for bits in range(0x3F80, 0x4080):
        a = float(O.bf16_bits_to_f32(np.array([bits], np.uint16))[0])
        if rn32(F(a) * F(r)) != rn32(F(a) / p):
            return a
    raise AssertionError("no case found")


@pytest.mark.parametrize("bits,p", [(8, 127), (4, 7)])
def test_quantize_rows_uses_reciprocal_scale(bits, p):
    amax = _find_recip_case(p)
    row = np.zeros(128, np.float32)
    row[5] = -amax
    row[17] = amax * 0.5
    row[40] = amax * 0.123
    codes, scales = O.tw_quantize_rows(_bf16_row(row), bits)
    s = rn32(F(amax) * F(O.tw_recip(p)))
    assert scales[0] == s and s != rn32(F(amax) / p)
    xs = O.bf16_bits_to_f32(_bf16_row(row))[0]
    want = [max(-p - 1, min(p, rint_even(F(rn32(F(v) / F(s)))))) for v in xs]
    assert codes[0].tolist() == want
    assert codes[0, 5] == -p  # the absmax element maps to the bound


@pytest.mark.parametrize("bits,p", [(8, 127), (4, 7)])
def test_quantize_rows_zero_row_and_floor(bits, p):
    rows = np.zeros((2, 64), np.float32)
    rows[1, 3] = 1e-30  # below the 1e-8 floor
    codes, scales = O.tw_quantize_rows(O.f32_to_bf16_bits(rows), bits)
    floor = rn32(F(np.float32(1e-8)) * F(O.tw_recip(p)))
    assert scales.tolist() == [floor, floor]
    assert not codes.any()


@pytest.mark.parametrize("bits", [8, 4])
def test_quantize_rows_brute_force(bits):
    """Random bf16 rows with outliers: scales and codes from exact rational
    arithmetic and an independent rounding."""
    p = (1 << (bits - 1)) - 1
    rng = np.random.default_rng(bits)
    x = rng.standard_normal((3, 96)).astype(np.float32)
    x[:, 7] *= 40
    xb = O.f32_to_bf16_bits(x)
    codes, scales = O.tw_quantize_rows(xb, bits)
    xv = O.bf16_bits_to_f32(xb)
    for m in range(3):
        amax = max(abs(float(v)) for v in xv[m])
        s = rn32(F(amax) * F(O.tw_recip(p)))
        assert scales[m] == s
        want = [max(-p - 1, min(p, rint_even(F(rn32(F(v) / F(s)))))) for v in xv[m]]
        assert codes[m].tolist() == want


def test_weight_codes_gpu_division_semantics():
    """W4 / W8 scales: amax * fl(1/p) with gpu_division, the IEEE quotient
    without; a row where they differ shows both."""
    a4, a8 = _find_recip_case(7), _find_recip_case(127)
    w = np.zeros((2, 64), np.float32)
    w[0, 0], w[1, 0] = a4, a8
    w[0, 1:] = np.linspace(-a4, a4, 63)
    w[1, 1:] = np.linspace(-a8, a8, 63)
    _, s4_gpu = O.weight_codes(w[:1], 4, 8, gpu_division=True)
    _, s4_cpu = O.weight_codes(w[:1], 4, 8)
    assert s4_gpu[0] == rn32(F(a4) * F(O.tw_recip(7))) and s4_cpu[0] == rn32(F(a4) / 7)
    assert s4_gpu[0] != s4_cpu[0]
    _, s8_gpu = O.weight_codes(w[1:], 8, 8, gpu_division=True)
    _, s8_cpu = O.weight_codes(w[1:], 8, 8)
    assert s8_gpu[0] == rn32(F(a8) * F(O.tw_recip(127))) and s8_cpu[0] == rn32(F(a8) / 127)
    c8, _ = O.weight_codes(w[1:], 8, 8, gpu_division=True)
    want = [max(-128, min(127, rint_even(F(rn32(F(v) / F(s8_gpu[0])))))) for v in w[1]]
    assert c8[0].tolist() == want
    # W2 has no division by a constant: both semantics agree
    assert all(np.array_equal(u, v) for u, v in zip(O.weight_codes(w, 2, 8, gpu_division=True),
                                                    O.weight_codes(w, 2, 8)))


def test_kmajor_packing_hand_derived_bytes():
    # W4, K = 4: byte j holds code j (low nibble) and code j + 2 (high nibble)
    c4 = np.array([[1, -2, 3, -8]], np.int8)
    assert O.pack_kmajor(c4, 4).tolist() == [[0x31], [0x8E]]
    # W2, K = 8: byte j holds codes j, j+2, j+4, j+6 at bits 0, 2, 4, 6
    c2 = np.array([[1, -2, 0, -1, 1, 1, -2, 0]], np.int8)
    assert O.pack_kmajor(c2, 2).tolist() == [[0x91], [0x1E]]
    # W8: the transpose
    c8 = np.array([[1, -1], [127, -128]], np.int8)
    assert O.pack_kmajor(c8, 8).tolist() == [[1, 127], [-1, -128]]
    # two output rows stay two columns
    c = np.array([[1, 2, 3, 4], [-1, -2, -3, -4]], np.int8)
    assert O.pack_kmajor(c, 4).tolist() == [[0x31, 0xDF], [0x42, 0xCE]]


@pytest.mark.parametrize("bits", [8, 4, 2])
def test_kmajor_round_trip(bits):
    lo = -(1 << (bits - 1))
    c = np.random.default_rng(bits).integers(lo, -lo, (7, 256)).astype(np.int8)
    assert np.array_equal(O.unpack_kmajor(O.pack_kmajor(c, bits), bits, 256), c)


def test_dots_brute_force_and_extremes():
    rng = np.random.default_rng(0)
    a = rng.integers(-128, 128, (3, 192)).astype(np.int8)
    w = rng.integers(-128, 128, (5, 192)).astype(np.int8)
    acc = O.tw_dots(a, w)
    for m in range(3):
        for n in range(5):
            assert acc[m, n] == sum(int(a[m, k]) * int(w[n, k]) for k in range(192))
    # K = 131071 full-scale (-128)^2 products stay below 2^31
    big = O.tw_dots(np.full((1, 131071), -128, np.int8), np.full((1, 131071), -128, np.int8))
    assert big[0, 0] == 131071 * 16384
    with pytest.raises(OverflowError):
        O.tw_dots(np.full((1, 131072), -128, np.int8), np.full((1, 131072), -128, np.int8))


def test_epilogue_orders_exact_rational():
    """mode 0: fmaf(fl(f32(acc) * as), ws, bias); mode 1: fmaf(f32(acc),
    fl(as * ws), bias); without a bias every product rounds on its own.
    Values chosen so that fused and unfused rounding differ."""
    acc = np.array([[3, 2**25 + 1]], np.int32)          # 2^25 + 1 is not an fp32
    as_ = np.array([1 + 2.0**-12], np.float32)
    ws = np.array([1 + 2.0**-11, 1 - 2.0**-13], np.float32)
    bias = np.array([-3.0, 5.0], np.float32)
    for mode in (0, 1):
        for b in (None, bias):
            got = O.tw_epilogue(acc, as_, ws, b, mode)
            for n in range(2):
                a = F(rn32(Fraction(int(acc[0, n]))))
                if mode == 0:
                    t = F(rn32(a * F(as_[0])))
                    want = rn32(t * F(ws[n]) + (F(b[n]) if b is not None else 0)) if b is not None \
                        else rn32(t * F(ws[n]))
                else:
                    q = F(rn32(F(as_[0]) * F(ws[n])))
                    want = rn32(a * q + F(b[n])) if b is not None else rn32(a * q)
                assert got[0, n] == want, (mode, b is None, n)
    # the fused form is observable: unfused rounding gives another value here
    t = rn32(F(np.float32(3)) * F(as_[0]))
    assert rn32(F(t) * F(ws[0]) + F(bias[0])) != rn32(F(rn32(F(t) * F(ws[0]))) + F(bias[0]))


def test_nested_r4_codes_hand_derived_and_wrap():
    """W4R4 codes: hand-derived values, including the wrapped (-8, r < 0)
    pairs; r = 0 is exactly 16 q; every non-wrapping pair dequantizes to
    q + r / 16 (the two-level grid the residual refines)."""
    pairs = {(0, 0): 0, (7, 7): 119, (-8, 0): -128, (-8, -1): 127, (-8, -8): 120, (7, -8): 104,
             (-1, -1): -17, (1, -8): 8, (-7, -8): -120, (3, 5): 53}
    q = np.array([p[0] for p in pairs], np.int8)
    r = np.array([p[1] for p in pairs], np.int8)
    np.testing.assert_array_equal(O.nested_r4_codes(q, r), np.array(list(pairs.values()), np.int8))
    grid = np.arange(-8, 8, dtype=np.int8)
    qq, rr = np.meshgrid(grid, grid, indexing="ij")
    codes = O.nested_r4_codes(qq, rr)
    np.testing.assert_array_equal(O.nested_r4_codes(grid, np.zeros(16, np.int8)), grid.astype(np.int16) * 16)
    wrap = (qq == -8) & (rr < 0)
    assert wrap.sum() == 8 and (codes[wrap] >= 120).all()
    for qv, rv, c in zip(qq[~wrap], rr[~wrap], codes[~wrap]):
        assert Fraction(int(c), 16) == qv + Fraction(int(rv), 16)
    # all 256 codes reached exactly once: the map is a bijection onto int8
    assert len(np.unique(codes)) == 256
    with pytest.raises(ValueError):
        O.nested_r4_codes(np.array([8], np.int8), np.array([0], np.int8))


def test_nested_r4_epilogue_with_zero_residual_is_w4():
    """With r = 0 the W4R4 result (codes 16 q, scale ws / 16) equals the
    plain W4 result bit for bit: the factor 16 is exact in int32 and fp32."""
    rng = np.random.default_rng(3)
    a = rng.integers(-127, 128, (5, 256)).astype(np.int8)
    q = rng.integers(-8, 8, (48, 256)).astype(np.int8)
    as_ = rng.uniform(1e-3, 1e-1, 5).astype(np.float32)
    ws = rng.uniform(1e-3, 1e-1, 48).astype(np.float32)
    bias = rng.standard_normal(48).astype(np.float32)
    w4 = O.tw_epilogue(O.tw_dots(a, q), as_, ws, bias, 0)
    nested = O.nested_r4_codes(q, np.zeros_like(q))
    r4 = O.tw_epilogue(O.tw_dots(a, nested), as_, ws / np.float32(16), bias, 0)
    np.testing.assert_array_equal(r4.view(np.uint32), w4.view(np.uint32))
