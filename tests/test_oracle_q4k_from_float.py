"""Known answers for the oracle's Q4_K quantizer: make_qkx1_quants and BlockQ4K::from_float.

These pin the one part of the oracle that no closed form covers elsewhere: which bytes
Candle 0.8's Q4_K from_float writes for a given f32 block.  The algorithm (candle-core
src/quantized/utils.rs make_qkx1_quants with nmax = 15, ntry = 5, and k_quants.rs
BlockQ4K::from_float) is, per sub-block of 32 values:

  min = min(x.min, 0); iscale = 15 / (x.max - min)          (all equal -> (0, 0))
  repeat up to 5 times:
      l_i = clamp(nearest_int(iscale * (x_i - min)), 0, 15)   nearest_int = f32::round
      scale = sum (x_i - min) l_i / sum l_i^2
      min = min(mean(x_i - scale l_i), 0); iscale = 1 / scale
      stop if no l_i changed
  -> (scale, -min)

then per block ls_j = min(nearest_int(63 / max_scale * scale_j), 63), lm_j likewise for
the mins, d = f16(max_scale / 63), dmin = f16(max_min / 63), and each value's 4-bit
quant L = clamp(nearest_int((x + dmin lm_j) / (d ls_j)), 0, 15).

Every expected value below follows from that statement in exact arithmetic: by hand
for the grid and constructed blocks (derivations in the docstrings; the inputs make each
f32 operation exact, or put it far from a rounding decision), and, for the two
multi-iteration sub-blocks FIVE and STOP, from their exact-fraction trajectories
(tests/golden/q4k_trajectories.py prints them iteration by iteration).  Each check names
the slip it catches; test_planted_slips_are_caught plants each of those slips into a
copy of the oracle's C source on the CPU and checks that some known answer then fails.
"""
import ctypes
import os
import shutil
import subprocess
from fractions import Fraction as Fr

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_DIR = os.path.join(os.path.dirname(HERE), "oracle")
U = Fr(1, 256)
TWO = list(range(16)) * 2  # every level 0..15 twice: x.min and x.max both on the grid


def _f32(vals):
    a = np.array([float(v) for v in vals], np.float32)
    assert all(Fr(float(x)) == Fr(v) for x, v in zip(a, vals)), "inputs must be exact in f32"
    return a


def _qkx1(lib, x):
    x = np.ascontiguousarray(x, np.float32)
    s = np.zeros(1, np.float32)
    m = np.zeros(1, np.float32)
    lib.ora_make_qkx1_quants(15, 5, x.ctypes.data_as(ctypes.c_void_p), x.size, s.ctypes.data_as(ctypes.c_void_p),
                             m.ctypes.data_as(ctypes.c_void_p))
    return float(s[0]), float(m[0])


def _q4k(lib, x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(144, np.uint8)
    assert lib.ora_quantize_row(12, x.ctypes.data_as(ctypes.c_void_p), 256, out.ctypes.data_as(ctypes.c_void_p)) == 0
    return out


def _block_bytes(d_bits, dmin_bits, ls, lm, L):
    """Canonical BlockQ4K bytes: d, dmin (f16 bits), the 12 scale bytes (6-bit ls/lm: j < 4
    direct, j >= 4 split into low nibbles and the top 2 bits of bytes j-4 and j), and the
    quants of each 64-value chunk c as bytes 32c + i = L[64c + i] | L[64c + 32 + i] << 4
    (the layout test_q4k_dequant_known_answer pins through to_float)."""
    s = np.zeros(12, np.uint8)
    for j in range(8):
        if j < 4:
            s[j] |= ls[j]
            s[j + 4] |= lm[j]
        else:
            s[j + 4] = (ls[j] & 0xF) | ((lm[j] & 0xF) << 4)
            s[j - 4] |= (ls[j] >> 4) << 6
            s[j] |= (lm[j] >> 4) << 6
    L = np.asarray(L, np.uint8)
    qs = np.zeros(128, np.uint8)
    for c in range(4):
        qs[32 * c:32 * c + 32] = L[64 * c:64 * c + 32] | (L[64 * c + 32:64 * c + 64] << 4)
    return np.concatenate([np.array([d_bits, dmin_bits], np.uint16).view(np.uint8), s, qs])


# ------------------------------------------------------------- make_qkx1_quants
def check_qkx1_exact_grid(lib):
    """x = min + s l, l = 0..15 twice, s = 2^-4, min = -3/16.  Iteration 1: iscale =
    15 / (15 s) = 16 exactly, l_i = l, scale = s sum l^2 / sum l^2 = s, mean residual =
    min; iteration 2 changes nothing.  -> (1/16, 3/16).  Catches: a wrong sign of the
    returned min, a scale not refitted by least squares."""
    x = _f32([Fr(-3, 16) + Fr(l, 16) for l in TWO])
    assert _qkx1(lib, x) == (0.0625, 0.1875)


def check_qkx1_positive_values(lib):
    """x = 7/256 l, l = 1..15 twice and 8, 8: every value positive, so min = min(x.min, 0)
    = 0; iscale = 15 / (105/256), l_i = l (the product is within 2^-23 of l), scale =
    7/256, residuals 0.  -> (7/256, 0).  Catches: the min not clamped at 0 on entry
    (min = 7/256 would give l_i = round(15 (l - 1) / 14) and another scale)."""
    x = _f32([7 * U * l for l in list(range(1, 16)) * 2 + [8, 8]])
    s, m = _qkx1(lib, x)
    assert s == 7 / 256 and m == 0.0


def check_qkx1_all_equal(lib):
    """All values equal: (0, 0) before any iteration.  Catches: a missing max == min exit
    (15 / 0 would follow)."""
    for v in (0.7, 0.0, -3.0):
        assert _qkx1(lib, np.full(32, v, np.float32)) == (0.0, 0.0)


def check_qkx1_updated_min_clamped(lib):
    """x = 12/256 (l + 1/8), l = 0..15 twice.  min = 0 (all positive); iscale = 15/(12/256
    * 15.125) gives l_i = l (off by at most 0.124); scale = (12/256) * 2510/2480
    (sum x l = 12/256 (sum l^2 + sum l / 8) = 12/256 * 2510, sum l^2 = 2480); the mean
    residual (12/256)(244 - 2510/2480 * 240)/32 > 0 is clamped to 0; iteration 2 keeps
    every l.  -> (f32(12/256 * 2510/2480), 0).  Catches: the updated min not clamped at 0."""
    x = _f32([12 * U * (l + Fr(1, 8)) for l in TWO])
    s, m = _qkx1(lib, x)
    assert s == float(np.float32(12 / 256 * 2510 / 2480)) and m == 0.0


def check_qkx1_rounds_half_away(lib):
    """x = l/16, l = 0..15 twice, with the first l = 5 replaced by 2.5/16.  Iteration 1:
    min = 0, iscale = 15 / (15/16) = 16 exactly, so the replaced value lands exactly on
    2.5: f32::round gives 3.  Then sum l^2 = 2480 - 25 + 9 = 2464, sum x l = (2480 - 25 +
    7.5)/16, scale = 4925/78848; sum x = 237.5/16, sum l = 238, mean residual
    (237.5/16 - 238 * 4925/78848)/32 = -125/180224 (kept, < 0).  Iteration 2 (iscale
    78848/4925) keeps every l: scale = 13883675/222035968, min = -604875/507510784, stop.
    With half-even rounding the tie gives 2 and the end point is (0.0625254, 0).
    Catches: half-even (or truncating) nearest_int."""
    vals = [Fr(l, 16) for l in TWO]
    vals[5] = Fr(5, 32)
    s, m = _qkx1(lib, _f32(vals))
    assert abs(s - 13883675 / 222035968) <= 1e-6 * s
    assert abs(m - 604875 / 507510784) <= 1e-7  # a mean of residuals: absolute f32 error


# Values (times 1/16) of a sub-block whose quants change in every one of the five
# iterations: per iteration the quants of values 10, 23, 30 (iteration 2: 7 -> 6), 19
# and 22 (iteration 3: 4 -> 3), 12 (iteration 4: 10 -> 9) and 3 (iteration 5: 15 ->
# 14) change, every product at least 0.011 away from a rounding tie.  Exact end point
# after iteration 5: scale = 54906919943890885327/62891316700187197440 (0.87304453),
# min = -3643619068613465349167/2012522134405990318080 (-1.81047403); after four
# iterations it would be (0.86649675, -1.80460852).
FIVE = [-28, 48, -7, 172, 148, -31, 94, 138, -31, -7, 58, 41, 102, -11, -31, 14, 14, 41, 138, 18, 48, 14, 18, 58,
        41, 41, 66, 41, 29, 14, 58, 14]
FIVE_SCALE, FIVE_MIN = 54906919943890885327 / 62891316700187197440, 3643619068613465349167 / 2012522134405990318080
FIVE_L = [0, 6, 2, 14, 13, 0, 9, 12, 0, 2, 6, 5, 9, 1, 0, 3, 3, 5, 12, 3, 6, 3, 3, 6, 5, 5, 7, 5, 4, 3, 6, 3]
# Values (times 1/16) of a sub-block whose quants settle in iteration 1, so the loop stops
# after iteration 2, where the min has moved: the exact end point is (0.67508960,
# -2.42736893); iterating on (no early stop) would give (0.67419848, -2.41934880).
STOP = [-39, 92, 35, -39, 123, 35, 87, 92, -39, 123, 123, 19, 87, 123, 92, 92, 87, 92, 35, 92, 123, 35, 92, 92, -39,
        92, 19, 19, 92, 35, 35, -39]
STOP_SCALE, STOP_MIN = 0.6750896031723336, 2.4273689285510023
STOP_L = [0, 12, 7, 0, 15, 7, 12, 12, 0, 15, 15, 5, 12, 15, 12, 12, 12, 12, 7, 12, 15, 7, 12, 12, 0, 12, 5, 5, 12, 7,
          7, 0]


def check_qkx1_five_iterations(lib):
    """Catches: ntry = 4 (0.75 % off in scale)."""
    s, m = _qkx1(lib, _f32([Fr(v, 16) for v in FIVE]))
    assert abs(s - FIVE_SCALE) <= 1e-6 * FIVE_SCALE and abs(m - FIVE_MIN) <= 1e-6 * FIVE_MIN, (s, m)


def check_qkx1_stops_when_nothing_changes(lib):
    """Catches: a missing did_change break (0.13 % off in scale, 0.33 % in min)."""
    s, m = _qkx1(lib, _f32([Fr(v, 16) for v in STOP]))
    assert abs(s - STOP_SCALE) <= 1e-6 * STOP_SCALE and abs(m - STOP_MIN) <= 1e-6 * STOP_MIN, (s, m)


# ------------------------------------------------------------- BlockQ4K::from_float
def _grid(c, m, levels=TWO):
    return [-m * U + c * U * l for l in levels]


def check_block_constructed(lib):
    """Eight sub-blocks on exact grids (scale c/256, min -m/256; make_qkx1_quants returns
    (c/256, m/256) exactly, as in check_qkx1_exact_grid):

      j  c     m     why
      0  63    0     the largest scale: 63/max_scale = 256 exactly, ls = 63 (the clamp value)
      1  20.5  63    256 * scale = 20.5: ls = round(20.5) = 21; the largest min: lm = 63
      2  1     4.5   256 * min = 4.5: lm = 5; then (x + 5/256) / (1/256) = l + 1/2: L = l + 1 (<= 15)
      3  40    20
      4  7/256 l, l = 1..15 twice and 8, 8: min clamped to 0 on entry, ls 7, lm 0
      5  all 0.3: (0, 0), ls = lm = 0, quants left 0
      6  33    31
      7  12/256 (l + 1/8): updated min clamped to 0; 256 * scale = 12.145, ls 12, lm 0

    max_scale = max_min = 63/256, so d = dmin = f16(1/256) = 0x1C00 exactly, and every
    other quant is L = l (sub-block 1: 20.5 l / 21 rounds to l for l <= 15).  Catches:
    half-even nearest_int (ls_1 = 20, lm_2 = 4, L_2 = even neighbours), a clamp below 63,
    either min clamp missing (sub-block 4's scale, sub-block 7's lm wraps), d or dmin not
    f16(max / 63), truncating final quants."""
    subs = [_grid(63, 0), _grid(Fr(41, 2), 63), _grid(1, Fr(9, 2)), _grid(40, 20),
            [7 * U * l for l in list(range(1, 16)) * 2 + [8, 8]], [Fr(3, 10)] * 32, _grid(33, 31),
            [12 * U * (l + Fr(1, 8)) for l in TWO]]
    x = np.concatenate([_f32(s) if j != 5 else np.full(32, 0.3, np.float32) for j, s in enumerate(subs)])
    L = (TWO + TWO + [min(l + 1, 15) for l in TWO] + TWO + list(range(1, 16)) * 2 + [8, 8] + [0] * 32 + TWO + TWO)
    want = _block_bytes(0x1C00, 0x1C00, [63, 21, 1, 40, 7, 0, 33, 12], [0, 63, 5, 20, 0, 0, 31, 0], L)
    np.testing.assert_array_equal(_q4k(lib, x), want)


def check_block_five_iterations(lib):
    """The FIVE sub-block followed by seven all-zero sub-blocks: max_scale and max_min are
    its (scale, -min), so ls = lm = 63, d = f16(f32(FIVE_SCALE) / 63) = 0x2318 and dmin =
    f16(f32(FIVE_MIN) / 63) = 0x275B (both 0.35 f16 ulps or more from a rounding
    midpoint), and L = round((x + 63 dmin) / (63 d)) (every quotient 0.011 or more from a
    tie).  Four iterations would give d = 0x230B, dmin = 0x2755."""
    x = np.concatenate([_f32([Fr(v, 16) for v in FIVE]), np.zeros(224, np.float32)])
    want = _block_bytes(0x2318, 0x275B, [63] + [0] * 7, [63] + [0] * 7, FIVE_L + [0] * 224)
    np.testing.assert_array_equal(_q4k(lib, x), want)


def check_block_stops(lib):
    """The STOP sub-block followed by seven all-zero sub-blocks: d = 0x217D, dmin = 0x28EF
    (without the early stop: 0x217B, 0x28EA)."""
    x = np.concatenate([_f32([Fr(v, 16) for v in STOP]), np.zeros(224, np.float32)])
    want = _block_bytes(0x217D, 0x28EF, [63] + [0] * 7, [63] + [0] * 7, STOP_L + [0] * 224)
    np.testing.assert_array_equal(_q4k(lib, x), want)


CHECKS = [check_qkx1_exact_grid, check_qkx1_positive_values, check_qkx1_all_equal, check_qkx1_updated_min_clamped,
          check_qkx1_rounds_half_away, check_qkx1_five_iterations, check_qkx1_stops_when_nothing_changes,
          check_block_constructed, check_block_five_iterations, check_block_stops]


@pytest.mark.parametrize("check", CHECKS, ids=[c.__name__[6:] for c in CHECKS])
def test_oracle_q4k_known_answer(ora, check):
    check(ora.lib())


# Each slip as a (description, original text, replacement) edit of oracle/sxq_oracle.c.
SLIPS = [
    ("half-even nearest_int", "static int32_t nearest_int(float v) { return cast_i32(roundf(v)); }",
     "static int32_t nearest_int(float v) { return cast_i32(rintf(v)); }"),
    ("truncating nearest_int", "static int32_t nearest_int(float v) { return cast_i32(roundf(v)); }",
     "static int32_t nearest_int(float v) { return cast_i32(truncf(v)); }"),
    ("four iterations", "for (int it = 0; it < ntry; ++it) {", "for (int it = 0; it < ntry - 1; ++it) {"),
    ("no early stop", "if (!did_change) break;", ""),
    ("min not clamped on entry", "float min = fmin_rs(mn, 0.0f);", "float min = mn;"),
    ("updated min not clamped", "if (min > 0.0f) min = 0.0f;", ""),
    ("ls clamp at 62", "uint8_t ls = (uint8_t)(lsi < 63 ? lsi : 63);", "uint8_t ls = (uint8_t)(lsi < 62 ? lsi : 62);"),
    ("lm clamp at 62", "uint8_t lm = (uint8_t)(lmi < 63 ? lmi : 63);", "uint8_t lm = (uint8_t)(lmi < 62 ? lmi : 62);"),
    ("d not max_scale / 63", "ora_f32_to_f16(max_scale / 63.0f)", "ora_f32_to_f16(max_scale / 64.0f)"),
    ("dmin not max_min / 63", "ora_f32_to_f16(max_min / 63.0f)", "ora_f32_to_f16(max_min / 62.0f)"),
    ("truncating final quants", "int32_t lv = nearest_int((x[32 * j + ii] + dm) / d);",
     "int32_t lv = (int32_t)((x[32 * j + ii] + dm) / d);"),
]


@pytest.mark.parametrize("slip", SLIPS, ids=[s[0] for s in SLIPS])
def test_planted_slips_are_caught(tmp_path, slip):
    """Plant one slip into a copy of the oracle (CPU only), build it, and check that at
    least one known answer above fails on it."""
    name, old, new = slip
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    src = open(os.path.join(ORACLE_DIR, "sxq_oracle.c")).read()
    assert src.count(old) == 1, f"slip site not found: {old}"
    shutil.copy(os.path.join(ORACLE_DIR, "sxq_oracle.h"), tmp_path / "sxq_oracle.h")
    (tmp_path / "sxq_oracle.c").write_text(src.replace(old, new))
    so = tmp_path / "libslip.so"
    subprocess.run([cc, "-O2", "-fPIC", "-std=c11", "-ffp-contract=off", "-fno-fast-math", "-D_GNU_SOURCE",
                    "-shared", "-o", str(so), str(tmp_path / "sxq_oracle.c"), "-lm", "-lpthread"], check=True)
    lib = ctypes.CDLL(str(so))
    lib.ora_make_qkx1_quants.restype = None
    lib.ora_make_qkx1_quants.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
                                         ctypes.c_void_p]
    lib.ora_quantize_row.restype = ctypes.c_int
    lib.ora_quantize_row.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
    failed = []
    for check in CHECKS:
        try:
            check(lib)
        except AssertionError:
            failed.append(check.__name__)
    assert failed, f"no known answer fails with the slip '{name}'"
