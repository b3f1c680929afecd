"""The bf16 quantizer's division (ma_quant.h quant_code): a / step from the group's
correctly rounded reciprocal y = RN(1/step) with one Markstein correction,

    q0 = RN(a * y),  r = RN(a - q0 * step) (exact, an FMA),  q = RN(q0 + r * y) (an FMA),

must equal the IEEE quotient RN(a / step) that the reference's torch CPU division gives
(reference.py:78-81, arithmetic in bf16 = each op in f32 rounded to bf16).  Both operands
are bf16 values (8 significant bits) and scaling by powers of two is exact in the normal
range, so the equality for every pair of bf16 significands is the equality for every pair
of normal bf16 values: checked here exhaustively with exact rational arithmetic (no
floating point involved).  Zero, subnormal quotients (code 0 either way) and non-finite
operands (an infinite a implies an infinite step: NaN either way) are covered by the
quantizer's own clamping, and the GPU tests compare the kernels with golden vectors."""

from fractions import Fraction as Fr


def _rn32(x: Fr) -> Fr:
    """Round a rational to the nearest binary32 value, ties to even (normal range)."""
    if x == 0:
        return Fr(0)
    sign = -1 if x < 0 else 1
    x = abs(x)
    e = x.numerator.bit_length() - x.denominator.bit_length()
    if Fr(2) ** e > x:
        e -= 1
    if Fr(2) ** (e + 1) <= x:
        e += 1
    sc = x / Fr(2) ** (e - 23)
    q, r = divmod(sc.numerator, sc.denominator)
    rem = Fr(r, sc.denominator)
    if rem > Fr(1, 2) or (rem == Fr(1, 2) and q % 2):
        q += 1
    return sign * Fr(q) * Fr(2) ** (e - 23)


def test_rn32_reference_points():
    assert _rn32(Fr(1, 3)) == Fr(11184811, 2 ** 25)          # 0x3eaaaaab
    assert _rn32(Fr(2 ** 24 + 1)) == Fr(2 ** 24)              # tie to even
    assert _rn32(Fr(2 ** 24 + 3)) == Fr(2 ** 24 + 4)


def test_corrected_reciprocal_division_is_exact_for_all_bf16_pairs():
    uncorrected_differs = 0
    for ma in range(128, 256):
        a = Fr(ma, 128)
        for ms in range(128, 256):
            s = Fr(ms, 128)
            y = _rn32(1 / s)
            q0 = _rn32(a * y)
            r_exact = a - q0 * s
            r = _rn32(r_exact)
            assert r == r_exact, (ma, ms)                    # the FMA residual is exact
            want = _rn32(a / s)
            assert _rn32(q0 + r * y) == want, (ma, ms)
            uncorrected_differs += q0 != want
    # the correction matters: without it some quotients are off by one ulp
    assert uncorrected_differs > 0
