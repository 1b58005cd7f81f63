"""Pins for the CPU oracle (oracle/sxq_oracle.c), independent of the oracle's own code.

Every check here is a known-answer block, a closed form evaluated with a different
tool (numpy's float16, f64 brute force), an invariant, or one of the reference's own
golden fixtures (tests/golden/reference_toy/, copied from the reference's
tests/golden/parity/).  Each is chosen so that a plausible slip in the restatement
(round-half-even instead of half-away, last instead of first max, a dropped min
term, a wrong nibble order, a missing f16 rounding) fails at least one of them.
"""
import json
import os

import numpy as np
import pytest

GOLD = os.path.join(os.path.dirname(__file__), "golden", "reference_toy")


def _gold(name):
    with open(os.path.join(GOLD, name + ".json")) as f:
        return json.load(f)


# ---------------------------------------------------------------- block geometry
def test_block_sizes_match_ggml_layout(ora):
    L = ora.lib()
    assert [L.ora_type_size(t) for t in (ora.Q4_0, ora.Q8_0, ora.Q4K, ora.Q8K)] == [18, 34, 144, 292]
    assert [L.ora_block_size(t) for t in (ora.Q4_0, ora.Q8_0, ora.Q4K, ora.Q8K)] == [32, 32, 256, 256]


def test_storage_accounting_matches_published_figures(ora):
    # storage_size_in_bytes = N*K/bs*type_size (cv2/load.rs:103): the Qwen2-0.5B up-projection
    # in Q8_0 and the 36 Qwen3-4B layers in Q4_K
    assert 4864 * ora.row_bytes(ora.Q8_0, 896) == 4_630_528
    layer = (6144 * ora.row_bytes(ora.Q4K, 2560) + 2560 * ora.row_bytes(ora.Q4K, 4096)
             + 2 * 9728 * ora.row_bytes(ora.Q4K, 2560) + 2560 * ora.row_bytes(ora.Q4K, 9728))
    assert 36 * layer == 2_043_740_160
    assert 155776 * ora.row_bytes(ora.Q4K, 2560) == 224_317_440


# ---------------------------------------------------------------- f16 (half crate)
def test_f16_round_to_nearest_even_matches_numpy(ora):
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(3000).astype(np.float32) * np.float32(3.0),
        (rng.standard_normal(1000) * 1e-5).astype(np.float32),   # f16 subnormal range
        (rng.standard_normal(500) * 1e-8).astype(np.float32),    # underflow to 0
        np.array([65504.0, 65519.0, 65520.0, 1e6, -1e6, 0.0, -0.0, np.inf, -np.inf,
                  2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -14, 1.0 + 2.0 ** -11,
                  1.0 + 3 * 2.0 ** -11, 1.0 / 127.0, 127.0 / 127.0], np.float32),
    ])
    got = ora.f32_to_f16_bits(vals)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, want)
    back = ora.f16_bits_to_f32(want)
    np.testing.assert_array_equal(back.view(np.uint32), want.view(np.float16).astype(np.float32).view(np.uint32))
    nan = ora.f32_to_f16_bits(np.array([np.nan], np.float32))
    assert np.isnan(nan.view(np.float16)[0])


# ---------------------------------------------------------------- Q8_0 from_float
def _q8_0_fields(blocks):
    b = blocks.reshape(-1, 34)
    return b[:, :2].copy().view(np.uint16).ravel(), b[:, 2:].view(np.int8)


def test_q8_0_known_answer_integer_block(ora):
    x = np.array([127, -127, 0, 1, -1, 64, -64, 5] + list(range(-12, 12)), np.float32)
    d, q = _q8_0_fields(ora.quantize(ora.Q8_0, x))
    assert d[0] == 0x3C00  # d = 127/127 = 1.0
    np.testing.assert_array_equal(q[0], x.astype(np.int8))


def test_q8_0_rounds_half_away_from_zero(ora):
    # amax = 127 -> d = 1, id = 1: x*id is exact, so only the rounding rule decides.
    x = np.array([127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 126.5] + [0.0] * 24, np.float32)
    _, q = _q8_0_fields(ora.quantize(ora.Q8_0, x))
    np.testing.assert_array_equal(q[0, :8], [127, 3, -3, 1, -1, 2, -2, 127])


def test_q8_0_zero_block(ora):
    d, q = _q8_0_fields(ora.quantize(ora.Q8_0, np.zeros(32, np.float32)))
    assert d[0] == 0 and not q.any()


def test_q8_0_uses_f32_inverse_scale_and_f16_stored_scale(ora):
    # Random blocks: q must come from the *f32* id = 1/(amax/127), d stored as f16-RNE.
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((64, 32)) * 0.37).astype(np.float32)
    d, q = _q8_0_fields(ora.quantize(ora.Q8_0, x))
    amax = np.abs(x).max(axis=1)
    d32 = (amax / np.float32(127.0)).astype(np.float32)
    id32 = (np.float32(1.0) / d32).astype(np.float32)
    v = (x * id32[:, None]).astype(np.float32).astype(np.float64)
    want = np.trunc(v + np.copysign(0.5, v)).clip(-128, 127).astype(np.int8)
    np.testing.assert_array_equal(q, want)
    np.testing.assert_array_equal(d, d32.astype(np.float16).view(np.uint16))


# ---------------------------------------------------------------- Q4_0 from_float
def test_q4_0_known_answers(ora):
    # max = -8 (largest magnitude, negative) -> d = -8/-8 = 1, q = min(15, trunc(x + 8.5)).
    x = np.zeros(32, np.float32)
    x[:6] = [-8.0, 7.0, 0.5, -0.5, 3.0, -7.9]
    x[16:20] = [1.0, -1.0, 6.5, -6.5]
    b = ora.quantize(ora.Q4_0, x).ravel()
    assert b[:2].view(np.uint16)[0] == 0x3C00
    lo = b[2:] & 0xF
    hi = b[2:] >> 4
    np.testing.assert_array_equal(lo[:6], [0, 15, 9, 8, 11, 0])
    np.testing.assert_array_equal(hi[:4], [9, 7, 15, 2])
    # max = +8 -> d = -1: x = 8 -> q = trunc(-8 + 8.5) = 0
    x2 = np.zeros(32, np.float32)
    x2[0], x2[1] = 8.0, -7.0
    b2 = ora.quantize(ora.Q4_0, x2).ravel()
    assert b2[:2].view(np.uint16)[0] == np.float16(-1.0).view(np.uint16)
    assert (b2[2] & 0xF) == 0 and (b2[3] & 0xF) == 15


# ---------------------------------------------------------------- Q8_K from_float
def _q8k_fields(blocks):
    b = blocks.reshape(-1, 292)
    d = b[:, :4].copy().view(np.float32).ravel()
    qs = b[:, 4:260].view(np.int8)
    bsums = b[:, 260:292].copy().view(np.int16)
    return d, qs, bsums


def test_q8k_first_max_wins_and_caps_at_127(ora):
    x = np.zeros(256, np.float32)
    x[0], x[1] = 1.0, -1.0
    d, q, bs = _q8k_fields(ora.quantize(ora.Q8K, x))
    # signed max = +1 (first of the tied magnitudes) -> iscale = -128
    assert d[0] == np.float32(-1.0 / 128.0)
    assert q[0, 0] == -128 and q[0, 1] == 127
    assert bs[0, 0] == -1


def test_q8k_zero_block(ora):
    d, q, bs = _q8k_fields(ora.quantize(ora.Q8K, np.zeros(256, np.float32)))
    assert d[0] == 0.0 and not q.any() and not bs.any()


def test_q8k_invariants(ora):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((32, 256)).astype(np.float32)
    d, q, bs = _q8k_fields(ora.quantize(ora.Q8K, x))
    np.testing.assert_array_equal(bs, q.reshape(32, 16, 16).astype(np.int32).sum(-1))
    i = np.abs(x).argmax(axis=1)  # first index of the largest magnitude
    np.testing.assert_array_equal(q[np.arange(32), i], -128)
    err = np.abs(d[:, None] * q - x)
    # half a step, except where round() gave +128 and the cap at 127 costs a full step
    bound = np.where(q == 127, 1.0001, 0.5001) * np.abs(d)[:, None] + 1e-7
    assert (err <= bound).all()


# ---------------------------------------------------------------- to_float KATs
def _pack_q4k_scales(sc, m):
    s = np.zeros(12, np.uint8)
    for j in range(8):
        if j < 4:
            s[j] = sc[j]
            s[j + 4] = m[j]
        else:
            s[j + 4] = (sc[j] & 0xF) | ((m[j] & 0xF) << 4)
            s[j - 4] |= (sc[j] >> 4) << 6
            s[j] |= (m[j] >> 4) << 6
    return s


def test_q4k_dequant_known_answer(ora):
    sc = np.array([1, 2, 3, 4, 17, 33, 48, 63], np.uint8)
    mn = np.array([0, 1, 2, 63, 16, 40, 5, 62], np.uint8)
    q = np.arange(256) % 16  # element value pattern
    qs = np.zeros(128, np.uint8)
    for c in range(4):
        for l in range(32):
            qs[32 * c + l] = q[64 * c + l] | (q[64 * c + 32 + l] << 4)
    blk = np.concatenate([np.array([np.float16(0.5), np.float16(0.25)]).view(np.uint8),
                          _pack_q4k_scales(sc, mn), qs]).astype(np.uint8)
    y = ora.dequantize(ora.Q4K, blk, 256).ravel()
    sub = np.arange(256) // 32
    want = 0.5 * sc[sub].astype(np.float64) * q - 0.25 * mn[sub].astype(np.float64)
    np.testing.assert_array_equal(y, want.astype(np.float32))


def test_q8_0_and_q4_0_dequant_known_answer(ora):
    qs = (np.arange(32) - 16).astype(np.int8)
    blk = np.concatenate([np.array([np.float16(0.5)]).view(np.uint8), qs.view(np.uint8)])
    np.testing.assert_array_equal(ora.dequantize(ora.Q8_0, blk, 32).ravel(), 0.5 * qs.astype(np.float32))
    nib = np.arange(16, dtype=np.uint8)
    blk4 = np.concatenate([np.array([np.float16(-2.0)]).view(np.uint8), (nib | (nib[::-1] << 4)).astype(np.uint8)])
    y = ora.dequantize(ora.Q4_0, blk4, 32).ravel()
    np.testing.assert_array_equal(y[:16], -2.0 * (nib.astype(np.float32) - 8))
    np.testing.assert_array_equal(y[16:], -2.0 * (nib[::-1].astype(np.float32) - 8))


# ---------------------------------------------------------------- round trips
@pytest.mark.parametrize("dt", ["Q8_0", "Q4_0", "Q4K"])
def test_quantize_dequantize_error_bound(ora, dt):
    dtype = getattr(ora, dt)
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((16, 512)) * 0.02).astype(np.float32)
    y = ora.dequantize(dtype, ora.quantize(dtype, x), 512)
    bs = ora.BLOCK[dtype]
    amax = np.abs(x).reshape(16, -1, bs).max(-1, keepdims=True)
    err = np.abs(y - x).reshape(16, -1, bs)
    levels = {"Q8_0": 127.0, "Q4_0": 8.0, "Q4K": 15.0}[dt]
    # one quantization step of a block spanning [-amax, amax] (Q4_K: [min, max] <= 2*amax);
    # Q8_0 quantizes with the f32 scale but stores it as f16: 127 * 2^-11 of a step more.
    step = (2.0 if dt == "Q4K" else 1.0) * amax / levels
    frac = 0.5 + 127 * 2.0 ** -11 if dt == "Q8_0" else 1.0
    assert (err <= step * frac * 1.001 + 1e-7).all()


def test_q4k_scale_packing_round_trip(ora):
    rng = np.random.default_rng(5)
    for _ in range(50):
        sc = rng.integers(0, 64, 8).astype(np.uint8)
        mn = rng.integers(0, 64, 8).astype(np.uint8)
        blk = np.concatenate([np.array([np.float16(1.0), np.float16(1.0)]).view(np.uint8),
                              _pack_q4k_scales(sc, mn), np.zeros(128, np.uint8)]).astype(np.uint8)
        y = ora.dequantize(ora.Q4K, blk, 256).ravel()
        np.testing.assert_array_equal(y.reshape(8, 32)[:, 0], -mn.astype(np.float32))


def test_make_qkx1_quants_reconstructs(ora):
    rng = np.random.default_rng(6)
    x = rng.standard_normal(32).astype(np.float32)
    scale, mn = ora.make_qkx1_quants(15, 5, x)
    assert scale > 0 and mn >= 0
    q = np.clip(np.round((x + mn) / scale), 0, 15)
    assert np.abs(scale * q - mn - x).max() <= scale  # within one level
    assert ora.make_qkx1_quants(15, 5, np.full(32, 0.7, np.float32)) == (0.0, 0.0)


# ---------------------------------------------------------------- vec_dot / matmul
@pytest.mark.parametrize("dt,k", [("Q8_0", 896), ("Q4_0", 896), ("Q4K", 2560), ("Q8_0", 4864), ("Q4K", 9728)])
def test_vec_dot_equals_f64_bilinear_form(ora, dt, k):
    dtype = getattr(ora, dt)
    rng = np.random.default_rng(7)
    w = (rng.standard_normal((8, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((1, k)).astype(np.float32)
    wb = ora.quantize(dtype, w)
    y = ora.matmul(dtype, x, wb, threads=1)[0]
    wd = ora.dequantize(dtype, wb, k).astype(np.float64)
    ab = ora.quantize(ora.VEC_DOT[dtype], x)
    ad = ora.dequantize(ora.VEC_DOT[dtype], ab, k).astype(np.float64)[0]
    exact = wd @ ad
    mag = np.abs(wd) @ np.abs(ad)
    assert (np.abs(y - exact) <= 2e-6 * mag + 1e-30).all(), (y, exact)
    for r in range(8):
        assert abs(ora.dot_f64(dtype, wb[r], x[0]) - exact[r]) <= 1e-12 * mag[r]


@pytest.mark.parametrize("dt", ["Q8_0", "Q4_0", "Q4K"])
def test_one_hot_activation_selects_weight(ora, dt):
    dtype = getattr(ora, dt)
    k = 512
    rng = np.random.default_rng(8)
    w = (rng.standard_normal((4, k)) * 0.02).astype(np.float32)
    wb = ora.quantize(dtype, w)
    wd = ora.dequantize(dtype, wb, k)
    for i in (0, 5, 31, 32, 63, 64, 200, 255, 256, 300, 511):
        x = np.zeros((1, k), np.float32)
        x[0, i] = 2.0
        # Q8 activation of a one-hot block is exactly 2.0 (127 * 2/127 resp. -128 * -2/128... )
        ad = ora.dequantize(ora.VEC_DOT[dtype], ora.quantize(ora.VEC_DOT[dtype], x), k)[0]
        y = ora.matmul(dtype, x, wb, threads=1)[0]
        np.testing.assert_allclose(y, wd[:, i] * ad[i], rtol=2e-7, atol=0)


def test_matmul_rows_independent_and_thread_invariant(ora):
    rng = np.random.default_rng(9)
    k, n = 1024, 700
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((5, k)).astype(np.float32)
    for dtype in (ora.Q8_0, ora.Q4K):
        wb = ora.quantize(dtype, w)
        y1 = ora.matmul(dtype, x, wb, threads=1)
        y8 = ora.matmul(dtype, x, wb, threads=8)
        np.testing.assert_array_equal(y1, y8)
        for r in range(5):
            np.testing.assert_array_equal(ora.matmul(dtype, x[r:r + 1], wb, threads=3)[0], y1[r])
        ab = ora.quantize(ora.VEC_DOT[dtype], x[2:3])[0]
        assert ora.vec_dot(dtype, k, wb[17], ab) == y1[2, 17]


def test_misaligned_k_is_rejected(ora):
    with pytest.raises(ValueError):
        ora.quantize(ora.Q4K, np.zeros(896, np.float32))  # 896 % 256 != 0 (Qwen2-0.5B shape)


# ---------------------------------------------------------------- glue ops vs golden fixtures
def test_rmsnorm_golden(ora):
    g = _gold("rmsnorm")
    x = np.array(g["input"]["x"], np.float32)[0]
    w = np.array(g["input"]["w"], np.float32)
    y = ora.rms_norm(x, w, g["input"]["eps"])
    np.testing.assert_allclose(y, np.array(g["data"], np.float32), atol=g["tol"])
    # and the closed form in f64
    ref = x / np.sqrt((x.astype(np.float64) ** 2).mean() + 1e-5)
    np.testing.assert_allclose(y, ref, rtol=1e-6)


def test_rope_interleaved_golden(ora):
    g = _gold("rope")
    x = np.array(g["input"]["x"], np.float32)  # [T, heads, hd]
    pos = g["input"]["positions"]
    hd = x.shape[-1]
    c, s = ora.rope_tables_interleaved(max(pos) + 1, hd, g["input"]["theta"])
    out = np.stack([ora.rope_interleaved(x[t], c[p], s[p]) for t, p in enumerate(pos)])
    np.testing.assert_allclose(out.ravel(), np.array(g["data"], np.float32), atol=g["tol"])


def test_rope_half_is_complex_rotation(ora):
    rng = np.random.default_rng(10)
    hd, h = 64, 3
    x = rng.standard_normal((h, hd)).astype(np.float32)
    c, s = ora.rope_tables_half(600, hd, 1e6)
    for pos in (0, 1, 511, 599):
        got = ora.rope_half(x, c[pos], s[pos])
        inv = 1.0 / (1e6 ** (np.arange(hd // 2) * 2.0 / hd))
        z = (x[:, :hd // 2] + 1j * x[:, hd // 2:]) * np.exp(1j * pos * inv)
        want = np.concatenate([z.real, z.imag], axis=1)
        np.testing.assert_allclose(got, want, rtol=0, atol=2e-5 * max(1, pos / 50))


def test_silu_and_softmax_golden(ora):
    g = _gold("silu")
    np.testing.assert_allclose(ora.silu(np.array(g["input"]["x"], np.float32)[0]),
                               np.array(g["data"], np.float32), atol=g["tol"])
    g = _gold("softmax")
    np.testing.assert_allclose(ora.softmax(np.array(g["input"]["x"], np.float32)[0]),
                               np.array(g["data"], np.float32), atol=g["tol"])


def test_attend_one_properties(ora):
    rng = np.random.default_rng(11)
    hd = 128
    q = rng.standard_normal(hd).astype(np.float32)
    k = rng.standard_normal((1, hd)).astype(np.float32)
    v = rng.standard_normal((1, hd)).astype(np.float32)
    np.testing.assert_array_equal(ora.attend_one(q, k, v), v[0])  # one key: p = 1
    K = rng.standard_normal((300, hd)).astype(np.float32)
    V = rng.standard_normal((300, hd)).astype(np.float32)
    sc = (K.astype(np.float64) @ q) / np.sqrt(hd)
    p = np.exp(sc - sc.max())
    p /= p.sum()
    np.testing.assert_allclose(ora.attend_one(q, K, V), p @ V, rtol=1e-4, atol=1e-5)
