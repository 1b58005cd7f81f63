"""Pins for the oracle of the CosyVoice generation loops (oracle/cv_generate.py), on the
CPU, over a scripted decoder whose logits force each draw: one id with logit 50 and the
rest 0 puts the whole nucleus on that id (its probability is 1 - 6563 e^-50), so every
output of the loop is known in closed form -- the tokens, the stop (not emitted), the
min_len mask (a masked stop leaves a flat distribution: the nucleus keeps the first 25
ids and the draw lands among them), the RAS fallback on a repeat (one extra uniform),
the rows fed to the model (the prompt as embeddings, then every emitted token as an id)
and the number of uniforms consumed (crates/syrinx-lm/src/cv2/generate.rs:136-163,
crates/syrinx-lm/src/cv3/generate.rs:55-101, cv2/sampling.rs:104-124).
"""
import numpy as np

import cv_generate as G
import sampling as S

V = 6564


class Scripted:
    """step_one returns logits peaked at the next scripted id; records what it is fed."""

    def __init__(self, script, vocab=V):
        self.script = list(script)
        self.fed = []
        self.vocab = vocab

    def reset(self, s):
        self.fed.append(("reset",))

    def step_one(self, s, frame=None, embed=None):
        self.fed.append(("embed", len(embed)) if embed is not None else ("id", int(frame[0])))
        x = np.zeros(self.vocab, np.float32)
        if self.script:
            x[self.script.pop(0)] = 50.0
        return x


def _uniforms_used(seed, rng):
    r = S.SplitMix64(seed)
    for k in range(64):
        if r.state == rng.state:
            return k
        r.next_u64()
    raise AssertionError("rng advanced by more than 64 draws")


def _prompt(n=3, dim=8):
    return np.zeros((n, dim), np.float32)


def test_tokens_stop_and_feedback():
    # the prompt's last row predicts 10; then 11, 12, a stop id
    orc = Scripted([0, 0, 10, 11, 12, 6562])
    out, rng, seen = G.generate(orc, _prompt(), 0, 20, 7, 6561, 6564)
    assert out == [10, 11, 12]
    assert len(seen) == 4                      # four draws, the last one the stop
    assert _uniforms_used(7, rng) == 4         # one uniform per nucleus draw
    assert orc.fed == [("reset",), ("embed", 8), ("embed", 8), ("embed", 8), ("id", 10), ("id", 11), ("id", 12)]


def test_max_len_caps_the_loop():
    orc = Scripted([0, 0, 5, 6, 7, 8, 9])
    out, rng, seen = G.generate(orc, _prompt(), 0, 3, 1, 6561, 6564)
    assert out == [5, 6, 7] and _uniforms_used(1, rng) == 3
    # as in the reference, the last emitted token is still fed through the model
    assert orc.fed[-3:] == [("id", 5), ("id", 6), ("id", 7)]


def test_repeat_triggers_the_full_distribution_draw():
    # 10 again within the 10-token window: ras_sampling draws once more from the full
    # (unmasked-by-repeat) distribution, which is still all on 10
    orc = Scripted([0, 0, 10, 11, 10, 6561])
    out, rng, _ = G.generate(orc, _prompt(), 0, 20, 3, 6561, 6564)
    assert out == [10, 11, 10]
    assert _uniforms_used(3, rng) == 5         # 1 + 1 + (1 + 1 fallback) + 1 (the stop)


def test_min_len_masks_stops():
    # the stop is scripted at step 1 but min_len = 3: it is masked, the draw falls in the
    # flat rest's nucleus (the first 25 ids), and the loop goes on
    orc = Scripted([0, 0, 10, 6562, 6562, 6562])
    out, rng, _ = G.generate(orc, _prompt(), 3, 20, 11, 6561, 6564)
    assert out[0] == 10 and all(0 <= t < 25 for t in out[1:3]) and len(out) == 3
    # step 3 (i = 3 >= min_len) draws the scripted stop


def test_cosyvoice3_stop_set_is_every_control_id():
    orc = Scripted([0, 0, 10, 6700], vocab=6761)
    out, _, _ = G.generate(orc, _prompt(), 0, 20, 2, 6561, 6761, stop=lambda t: t >= 6561)
    assert out == [10]
    # a planted CosyVoice2-style stop test ignores 6700 and emits it
    orc = Scripted([0, 0, 10, 6700, 6561], vocab=6761)
    bad, _, _ = G.generate(orc, _prompt(), 0, 20, 2, 6561, 6761, stop=lambda t: t in (6561, 6562, 6563))
    assert bad == [10, 6700]
