"""CPU oracle of the CosyVoice speech-token generation loops (test infrastructure only:
tests/ import it as the checker).

Restates, over an oracle decoder (oracle/model.py) whose dense input table is the
speech embedding:
  Qwen2Lm::generate   crates/syrinx-lm/src/cv2/generate.rs:136-163
  Cv3Lm::generate     crates/syrinx-lm/src/cv3/generate.rs:55-101
  (generate_instruct, cv3/generate.rs:14-44, is the same loop on another step-0 input)
with the samplers of oracle/sampling.py (log_softmax_vec + ras_sampling, the stop ids
masked while i < min_len).  The step-0 input is given as embedding rows (the prompt
assembly, cv2/generate.rs:89-101 and cv3/lm.rs:81-132, is a gather of table rows).
"""
from __future__ import annotations

import numpy as np

import sampling as S


def generate(orc, lm_input0, min_len: int, max_len: int, seed: int, stop_begin: int, stop_end: int,
             stop=None, stream: int = 0):
    """Returns (tokens, rng, logits of every sampled step).  `stop(t)` is the loop's stop
    test (cv2: t in STOP_TOKENS 6561..6563; cv3: t >= 6561); the default is
    stop_begin <= t < stop_end."""
    stop = stop or (lambda t: stop_begin <= t < stop_end)
    rng = S.SplitMix64(seed)
    orc.reset(stream)
    logits = None
    for row in np.asarray(lm_input0, np.float32):   # the cached prefill, one position at a time
        logits = orc.step_one(stream, embed=row)
    out, seen = [], []
    for i in range(max_len):
        seen.append(logits)
        top = S.ras_sampling(logits, out, rng, i < min_len, stop_begin, stop_end)
        if stop(top):
            break
        out.append(top)
        logits = orc.step_one(stream, frame=[top])  # its speech_embedding row fed back
    return out, rng, seen
