"""CPU oracle of the Fish dual-AR generation loop and the s2 fast AR (test infrastructure
only: tests/ import it as the checker).

Restates, over any backend with the reference's DualArBackend methods:
  drive          crates/syrinx-fish/src/common/dualar.rs:163-238
  drive_batch    crates/syrinx-fish/src/common/dualar.rs:240-360
  is_stop        crates/syrinx-fish/src/common/dualar.rs:96-98
and, for the s2 backend over oracle decoders (oracle/model.py):
  first_code     crates/syrinx-fish/src/s2/fast_ar.rs:105-110
  expand         crates/syrinx-fish/src/s2/fast_ar.rs:116-160 (a fresh cache per frame,
                 position 0 = the slow hidden, then the shared embedding of each code)
  head's hidden  crates/syrinx-fish/src/s2/slow_ar.rs:207-246 (the post-norm hidden).
Sampling is oracle/sampling.py's FishSampler, one per sample seeded seed + i.
"""
from __future__ import annotations

import numpy as np

import sampling as S


class Constraint:
    def __init__(self, begin: int, end: int, stop: int):
        self.begin, self.end, self.stop = begin, end, stop


def _sampler(seed, sp: dict):
    return S.FishSampler(seed, **sp)


def drive(backend, prompt, seed: int, sp: dict, cons: Constraint, n_cb: int, max_seq: int, max_new_frames: int):
    """Returns (codes [n_cb, T] int64, the sampler, the final RAS window)."""
    smp = _sampler(seed, sp)
    ras_win = max(1, sp.get("ras_win_size", 10))
    frames, window = [], []
    prompt = np.asarray(prompt).reshape(1 + n_cb, -1)
    backend.reset()
    logits, hidden = backend.prefill(0, prompt)
    pos = prompt.shape[1]
    while True:
        sem = smp.sample_semantic(logits, window, cons.begin, cons.end, cons.stop)
        if sem == cons.stop:
            break
        frame = backend.fast_expand(0, hidden, backend.first_code(sem), smp)
        frames.append(frame)
        window.append(sem)
        if len(window) > ras_win:
            window.pop(0)
        if len(frames) >= max_new_frames or pos + 1 >= max_seq:
            break
        logits, hidden = backend.slow_step(0, [sem] + list(frame))
        pos += 1
    codes = np.array(frames, np.int64).T.reshape(n_cb, len(frames))
    return codes, smp, window


def drive_batch(backend, prompts, seed: int, sp: dict, cons: Constraint, n_cb: int, max_seq: int,
                max_new_frames: int):
    """Returns (list of codes [n_cb, T_i], samplers, windows)."""
    n = len(prompts)
    smps = [_sampler(seed + i, sp) for i in range(n)]
    ras_win = max(1, sp.get("ras_win_size", 10))
    frames = [[] for _ in range(n)]
    windows = [[] for _ in range(n)]
    finished = [False] * n
    prompts = [np.asarray(p).reshape(1 + n_cb, -1) for p in prompts]
    pos = max(p.shape[1] for p in prompts)
    backend.reset()
    steps = [backend.prefill(i, prompts[i]) for i in range(n)]
    n_generated = 0
    while True:
        sems, firsts = [0] * n, [0] * n
        for i in range(n):
            if finished[i]:
                continue
            s = smps[i].sample_semantic(steps[i][0], windows[i], cons.begin, cons.end, cons.stop)
            if s == cons.stop:
                finished[i] = True
                continue
            sems[i], firsts[i] = s, backend.first_code(s)
        if all(finished):
            break
        batch = [None if finished[i] else backend.fast_expand(i, steps[i][1], firsts[i], smps[i]) for i in range(n)]
        for i in range(n):
            if finished[i]:
                continue
            frames[i].append(batch[i])
            windows[i].append(sems[i])
            if len(windows[i]) > ras_win:
                windows[i].pop(0)
        n_generated += 1
        if n_generated >= max_new_frames or pos + 1 >= max_seq:
            break
        for i in range(n):
            full = [0] * (1 + n_cb) if finished[i] else [sems[i]] + list(batch[i])
            steps[i] = backend.slow_step(i, full)
        pos += 1
    out = [np.array(f, np.int64).T.reshape(n_cb, len(f)) for f in frames]
    return out, smps, windows


class S2Backend:
    """The s2 backend over oracle decoders: `slow` an OracleDecoder of the slow AR (one
    stream per sample), `fast` an OracleDecoder of the fast AR (same stream count)."""

    def __init__(self, slow, fast, semantic_begin: int):
        self.slow, self.fast, self.begin = slow, fast, semantic_begin

    def reset(self):
        for s in range(len(self.slow.k)):
            self.slow.reset(s)

    def prefill(self, s, prompt):
        prompt = np.asarray(prompt)
        logits = None
        for t in range(prompt.shape[1]):
            logits = self.slow.step_one(s, frame=prompt[:, t])
        return logits, self.slow.hidden.copy()

    def slow_step(self, s, frame):
        logits = self.slow.step_one(s, frame=np.asarray(frame))
        return logits, self.slow.hidden.copy()

    def first_code(self, tok: int) -> int:
        return min(max(int(tok) - self.begin, 0), self.fast.c.vocab - 1)

    def fast_expand(self, s, hidden, first_code: int, smp, n_codes: int = None):
        n_codes = n_codes or self.fast.c.max_seq
        self.fast.reset(s)
        self.fast.step_one(s, embed=hidden)  # position 0: logits unused
        codes = [int(first_code)]
        for _ in range(1, n_codes):
            logits = self.fast.step_one(s, frame=[codes[-1]])
            codes.append(int(smp.sample_codebook(logits, [])))
        return codes
