"""Pins of the oracle's token samplers (oracle/sampling.py), the reference the device
samplers are compared with.

* SplitMix64: published known answers of the generator (Steele, Lea and Flood's
  SplitMix64, the algorithm of crates/syrinx-fish/src/common/sampling.rs:20-37):
  seed 0 -> 0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4; seed 1234567 -> 6457827717110365317,
  3203168211198807973, 9817491932198370423.
* The reference's own sampler tests (tests/real_cv3_multinomial.rs,
  tests/real_cv3_ras.rs): a flat uniform, an unbiased and scale-invariant inverse-CDF
  draw, the RAS fallback on a forced repeat and none without history.
* logits_to_probs (common/sampling.rs:186-240) and nucleus_sampling
  (cv2/sampling.rs:64-87) on hand-computed cases.
"""
import math

import numpy as np
import pytest

import sampling as S


def test_splitmix64_known_answers():
    r = S.SplitMix64(0)
    assert [r.next_u64() for _ in range(2)] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4]
    r = S.SplitMix64(1234567)
    assert [r.next_u64() for _ in range(3)] == [6457827717110365317, 3203168211198807973, 9817491932198370423]


def test_uniform_is_flat_on_0_1():
    r = S.SplitMix64(0x5EED)
    u = np.array([r.next_f64() for _ in range(100_000)])
    assert u.min() >= 0.0 and u.max() < 1.0 and u.min() < 0.01 and u.max() > 0.99
    bins = np.bincount((u * 10).astype(int), minlength=10) / len(u)
    assert np.abs(bins - 0.1).max() < 7e-3, bins


def test_multinomial1_unbiased_and_scale_invariant():
    target = np.array([0.05, 0.10, 0.20, 0.50, 0.15], np.float32)
    for scale in (1.0, 7.3):
        r = S.SplitMix64(0xC0FFEE)
        d = np.array([S.multinomial1(target * np.float32(scale), r) for _ in range(60_000)])
        f = np.bincount(d, minlength=5) / len(d)
        assert np.abs(f - target).max() < 1e-2, (scale, f)
        assert (np.bincount(d, minlength=5) > 0).all()


def test_multinomial1_inverse_cdf_boundaries():
    """u < acc picks the first category whose running sum exceeds u: with probabilities
    [0.25, 0.25, 0.5] a uniform in [0, 0.25) gives 0, [0.25, 0.5) gives 1, the rest 2."""
    class Fixed:
        def __init__(self, u):
            self.u = u

        def next_f64(self):
            return self.u
    p = np.array([0.25, 0.25, 0.5], np.float32)
    assert [S.multinomial1(p, Fixed(u)) for u in (0.0, 0.2499, 0.25, 0.4999, 0.5, 0.9999)] == [0, 0, 1, 1, 2, 2]
    assert S.multinomial1(np.zeros(4, np.float32), Fixed(0.3)) == 0  # nothing to draw: index 0


def test_logits_to_probs_hand_computed():
    x = np.array([3.0, 1.0, 2.0, 0.0], np.float32)
    # sorted ids 0, 2, 1, 3; cum after rank 0 = 1 / (1 + e^-1 + e^-2 + e^-3) = 0.6439
    p = S.logits_to_probs(x, 1.0, 0.5, 30)       # 0.6439 > 0.5: only the top-1 survives
    np.testing.assert_array_equal(p, [1.0, 0.0, 0.0, 0.0])
    p = S.logits_to_probs(x, 1.0, 0.9, 2)        # rank 1 kept (0.644 <= 0.9), rank 2 cut by top_k
    np.testing.assert_allclose(p, [1 / (1 + math.e ** -1), 0.0, 1 - 1 / (1 + math.e ** -1), 0.0], rtol=1e-6)
    p = S.logits_to_probs(x, 0.5, 0.9, 2)        # temperature 0.5 doubles the logit gap
    np.testing.assert_allclose(p[[0, 2]], [1 / (1 + math.e ** -2), 1 - 1 / (1 + math.e ** -2)], rtol=1e-6)
    p = S.logits_to_probs(x, 1.0, 1.0, 0)        # top_k 0 = unbounded; cum stays <= 1 until the end
    np.testing.assert_allclose(p, np.exp(x - 3.0) / np.exp(x - 3.0).sum(), rtol=1e-6)
    # equal logits: the stable sort keeps ascending ids first
    p = S.logits_to_probs(np.array([1.0, 5.0, 5.0, 5.0], np.float32), 1.0, 0.1, 2)
    np.testing.assert_array_equal(p, [0.0, 1.0, 0.0, 0.0])


def test_repetition_penalty_hf_convention():
    x = np.array([2.0, -2.0, 1.0], np.float32)
    y = S.apply_repetition_penalty(x, [0, 1, 1], 2.0)  # positive / 2, negative * 2 (twice)
    np.testing.assert_array_equal(y, [1.0, -8.0, 1.0])
    np.testing.assert_array_equal(S.apply_repetition_penalty(x, [0], 1.0), x)


def test_semantic_draw_respects_the_constraint_and_ras():
    rng = np.random.default_rng(0)
    smp = S.FishSampler(7)
    for _ in range(50):
        x = (rng.standard_normal(300) * 3).astype(np.float32)
        t = smp.sample_semantic(x, [], 100, 199, 250)
        assert 100 <= t <= 199 or t == 250
    # a peaked row: the normal draw is id 150; with 150 in the window RAS takes the
    # high-temperature draw, which (same logits, same top_p) is also 150 -- but the
    # rng advanced by exactly two draws either way
    x = np.full(300, -30.0, np.float32)
    x[150] = 10.0
    a, b = S.FishSampler(3), S.FishSampler(3)
    assert a.sample_semantic(x, [150], 100, 199, 250) == 150 == b.sample_semantic(x, [], 100, 199, 250)
    assert a.rng.state == b.rng.state == S.SplitMix64(3).state + 2 * 0x9E3779B97F4A7C15 % (1 << 64)


def test_cv_log_softmax_and_nucleus():
    x = np.array([0.0, math.log(3.0), -np.inf], np.float32)
    lp = S.log_softmax_vec(x)
    np.testing.assert_allclose(lp[:2], [math.log(0.25), math.log(0.75)], rtol=1e-6)
    assert lp[2] == -np.inf

    class Fixed:
        def next_f64(self):
            return 0.5
    # probabilities 0.75, 0.25: top_p 0.8 keeps both (cum 0.75 < 0.8), the draw on u = 0.5 x
    # (0.75 + 0.25) lands in the first candidate (sorted order: id 1 first)
    assert S.nucleus_sampling(lp, 0.8, 25, Fixed()) == 1
    assert S.nucleus_sampling(lp, 0.7, 25, Fixed()) == 1   # cum 0.75 >= 0.7: one candidate
    assert S.nucleus_sampling(lp, 0.8, 1, Fixed()) == 1    # top_k 1


def test_ras_fallback_triggers_on_repeat_only():
    x = np.full(6564, -20.0, np.float32)
    x[5] = 5.0  # the nucleus pick is id 5
    r1, r2 = S.SplitMix64(9), S.SplitMix64(9)
    t_no = S.ras_sampling(x, [], r1, False, 6561, 6564)
    assert t_no == 5 and r1.state == S.SplitMix64(9).state + 0x9E3779B97F4A7C15 % (1 << 64)
    # one 5 in the last 10 decoded tokens (>= 10 * 0.1): the full-distribution draw follows
    t_rep = S.ras_sampling(x, [1, 2, 5], r2, False, 6561, 6564)
    assert r2.state == (S.SplitMix64(9).state + 2 * 0x9E3779B97F4A7C15) % (1 << 64)
    assert 0 <= t_rep < 6564
    # ignore_eos masks the stop ids even when they dominate
    y = np.full(6564, -20.0, np.float32)
    y[6562] = 9.0
    for seed in range(20):
        assert S.ras_sampling(y, [], S.SplitMix64(seed), True, 6561, 6564) < 6561
