"""Pins of the oracle's per-row embedding quantizer (oracle/embed.py), the restatement of
crates/syrinx-lm/src/cv2/quant.rs:38-89 and the dequant-on-gather of
crates/syrinx-lm/src/cv2/generate.rs:22-67.

Rows with max|x| = qmax have scale exactly 1.0 (qmax * f32(1/qmax) rounds to 1 and the
1e-12 is below half an ulp), so their codes are plain roundings, written out by hand here.
Each known answer names the slip it catches: half-even rounding, the nibble order, the
int8 offset, the odd-width fallback, the zero-row epsilon and the scale's affine form.
"""
from fractions import Fraction

import numpy as np

import embed as E


def test_int8_known_answers():
    row = np.array([127.0, -127.0, 2.5, -2.5, 0.5, 100.49999, -0.0, 3.0], np.float32)
    q, s, scheme = E.quantize(row[None, :], E.INT8)
    assert scheme == E.INT8 and s[0] == np.float32(1.0)
    # half away from zero (half-even gives 2, -2, 0); code + 128 (an offset of 127 shifts all)
    assert q[0].tolist() == [255, 1, 131, 125, 129, 228, 128, 131]
    back = E.gather(q, s, E.INT8, 8, [0])[0]
    np.testing.assert_array_equal(back, [127, -127, 3, -3, 1, 100, 0, 3])


def test_int4_known_answers_and_nibble_order():
    row = np.array([7.0, 2.5, -2.5, 1.5, -0.5, 0.49999997, 3.5, -6.5], np.float32)
    q, s, scheme = E.quantize(row[None, :], E.INT4)
    assert scheme == E.INT4 and s[0] == np.float32(1.0)
    # codes 7, 3, -3, 2, -1, 0, 4, -7 -> nibbles 15, 11, 5, 10, 7, 8, 12, 1; element 2j low
    assert q[0].tolist() == [0xBF, 0xA5, 0x87, 0x1C]
    np.testing.assert_array_equal(E.gather(q, np.float32([0.5]), E.INT4, 8, [0])[0],
                                  [3.5, 1.5, -1.5, 1.0, -0.5, 0.0, 2.0, -3.5])


def test_odd_width_falls_back_to_int8():
    q, s, scheme = E.quantize(np.ones((2, 5), np.float32), E.INT4)
    assert scheme == E.INT8 and q.shape == (2, 5)


def test_zero_row_keeps_a_finite_scale():
    q, s, _ = E.quantize(np.zeros((1, 6), np.float32), E.INT4)
    assert s[0] == np.float32(1e-12) and q[0].tolist() == [0x88] * 3
    assert (E.gather(q, s, E.INT4, 6, [0]) == 0).all()


def _f32(fr: Fraction) -> np.float32:
    """Round an exact rational to the nearest f32, ties to even (by bracketing)."""
    x = np.float32(float(fr))  # within an ulp; fix up by exact comparison
    best = min((np.nextafter(x, np.float32(-np.inf)), x, np.nextafter(x, np.float32(np.inf))),
               key=lambda c: (abs(Fraction(float(c)) - fr), int(np.float32(c).view(np.uint32)) & 1))
    return np.float32(best)


def test_scale_is_candles_affine_map():
    """scale = f32(f32(amax * f32(1/127)) + f32(1e-12)), computed here in exact rationals,
    on rows where that differs from the correctly rounded amax / 127."""
    m = Fraction(float(np.float32(1.0 / 127.0)))
    eps = Fraction(float(np.float32(1e-12)))
    rng = np.random.default_rng(3)
    differ = 0
    for amax in rng.uniform(0.01, 4.0, 400).astype(np.float32):
        want = _f32(Fraction(float(_f32(Fraction(float(amax)) * m))) + eps)
        got = E.row_scales(np.array([[amax, -amax / 3]], np.float32), 127)[0]
        assert got == want, amax
        differ += want != _f32(Fraction(float(_f32(Fraction(float(amax)) / 127))) + eps)
    assert differ > 0  # the two formulas do part on some of these rows
