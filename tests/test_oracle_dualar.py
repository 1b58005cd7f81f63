"""Pins of the oracle's dual-AR driver (oracle/dualar.py) on a scripted backend whose
draws are forced (one-hot logits), so every output of the loop is known in closed form:
the frames and their order, the stop (no frame, no fast draws), max_new_frames, the
cache-length cap, per-sample seeds and the frozen streams of drive_batch, the RAS window,
and the number of uniforms each sampler consumed (two per semantic draw, one per
residual code) -- the reference's draw order (crates/syrinx-fish/src/common/dualar.rs:
163-360).  The reference has no test of its own for this loop.
"""
import numpy as np

import dualar as DA
import sampling as S

GAMMA = 0x9E3779B97F4A7C15
V, BEGIN, END, STOP, NCB, R = 24, 10, 17, 3, 3, 8


def onehot(tok, n=V):
    x = np.full(n, -60.0, np.float32)
    x[tok] = 60.0
    return x


class Scripted:
    """Slow logits force the next semantic token from a per-stream script (advanced once
    per slow step); fast logits force code cb = (first + cb) % R."""

    def __init__(self, scripts):
        self.scripts = scripts
        self.t = [0] * len(scripts)
        self.fed = [[] for _ in scripts]

    def reset(self):
        self.t = [0] * len(self.scripts)

    def _out(self, s):
        tok = self.scripts[s][min(self.t[s], len(self.scripts[s]) - 1)]
        return onehot(tok), np.full(4, float(s), np.float32)

    def prefill(self, s, prompt):
        return self._out(s)

    def slow_step(self, s, frame):
        self.fed[s].append(list(frame))
        self.t[s] += 1
        return self._out(s)

    def first_code(self, tok):
        return min(max(int(tok) - BEGIN, 0), R - 1)

    def fast_expand(self, s, hidden, first, smp):
        codes = [first]
        for cb in range(1, NCB):
            codes.append(int(smp.sample_codebook(onehot((first + cb) % R, R), [])))
        return codes


def rng_after(seed, draws):
    return (seed + draws * GAMMA) % (1 << 64)


SP = dict(temperature=1.0, top_p=0.9, top_k=30, repetition_penalty=1.1, ras_win_size=2)
CONS = DA.Constraint(BEGIN, END, STOP)
PROMPT = np.zeros((1 + NCB, 5), np.int64)


def frame_of(tok):
    f = tok - BEGIN
    return [f, (f + 1) % R, (f + 2) % R]


def test_drive_frames_stop_and_draw_count():
    be = Scripted([[12, 15, 12, STOP, 11]])
    codes, smp, window = DA.drive(be, PROMPT, 7, SP, CONS, NCB, max_seq=100, max_new_frames=50)
    want = np.array([frame_of(12), frame_of(15), frame_of(12)]).T
    np.testing.assert_array_equal(codes, want)
    # 4 semantic draws (3 frames + the stop) x 2 uniforms, 3 frames x 2 residual codes
    assert smp.rng.state == rng_after(7, 4 * 2 + 3 * 2)
    assert window == [15, 12]  # the last ras_win_size non-stop semantic ids
    # the slow AR was fed each full frame [semantic, codes...]
    assert be.fed[0] == [[12] + frame_of(12), [15] + frame_of(15), [12] + frame_of(12)]


def test_drive_immediate_stop_is_empty():
    codes, smp, _ = DA.drive(Scripted([[STOP]]), PROMPT, 1, SP, CONS, NCB, 100, 50)
    assert codes.shape == (NCB, 0) and smp.rng.state == rng_after(1, 2)


def test_drive_caps():
    be = Scripted([[11, 12, 13, 14, 15, 16]])
    codes, _, _ = DA.drive(be, PROMPT, 0, SP, CONS, NCB, max_seq=100, max_new_frames=2)
    assert codes.shape == (NCB, 2) and len(be.fed[0]) == 1  # no slow step after the last frame
    be = Scripted([[11, 12, 13, 14, 15, 16]])
    codes, _, _ = DA.drive(be, PROMPT, 0, SP, CONS, NCB, max_seq=8, max_new_frames=50)
    assert codes.shape == (NCB, 8 - PROMPT.shape[1])  # positions 5, 6, 7 then the cache is full


def test_first_code_clamps():
    be = Scripted([[11]])
    assert [be.first_code(t) for t in (BEGIN - 3, BEGIN, BEGIN + 5, BEGIN + R + 4)] == [0, 0, 5, R - 1]


def test_drive_batch_freezes_finished_streams():
    scripts = [[12, STOP, 14], [16, 11, 13, 12, 15]]
    be = Scripted(scripts)
    outs, smps, windows = DA.drive_batch(be, [PROMPT, PROMPT[:, :3]], 40, SP, CONS, NCB, 100, 4)
    np.testing.assert_array_equal(outs[0], np.array([frame_of(12)]).T)
    np.testing.assert_array_equal(outs[1], np.array([frame_of(t) for t in (16, 11, 13, 12)]).T)
    # stream 0: 2 semantic draws then frozen; stream 1: 4 frames
    assert smps[0].rng.state == rng_after(40, 2 * 2 + 1 * 2)
    assert smps[1].rng.state == rng_after(41, 4 * 2 + 4 * 2)
    assert windows == [[12], [13, 12]]
    # a frozen stream is fed the inert zero frame
    assert be.fed[0][1:] == [[0] * (1 + NCB)] * (len(be.fed[0]) - 1)
    # sample i of the batch reproduces drive seeded seed + i
    for i, (p, sc) in enumerate(zip([PROMPT, PROMPT[:, :3]], scripts)):
        single, smp, _ = DA.drive(Scripted([sc]), p, 40 + i, SP, CONS, NCB, 100, 4)
        np.testing.assert_array_equal(single, outs[i])
        assert smp.rng.state == smps[i].rng.state


def test_semantic_window_triggers_high_draw():
    """With a two-way tie among semantic ids the normal and the high-temperature draws can
    differ; the high one is taken only when the normal pick is in the window."""
    x = np.full(V, -60.0, np.float32)
    x[[12, 13]] = 5.0
    hits = 0
    for seed in range(40):
        a, b = S.FishSampler(seed, ras_win_size=2), S.FishSampler(seed, ras_win_size=2)
        n0 = a.sample_semantic(x, [], BEGIN, END, STOP)
        r = S.SplitMix64(seed)
        u1, u2 = r.next_f64(), r.next_f64()
        want_normal = 12 if u1 < 0.5 else 13
        want_high = 12 if u2 < 0.5 else 13
        assert n0 == want_normal
        got = b.sample_semantic(x, [want_normal], BEGIN, END, STOP)
        assert got == want_high
        hits += want_high != want_normal
    assert hits > 5
