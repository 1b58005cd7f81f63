"""CPU oracle of the reference's token samplers (test infrastructure only).

Restates, on numpy, the two seeded samplers the decode loops call after the head:
  Fish dual-AR   crates/syrinx-fish/src/common/sampling.rs:20-37 (SplitMix64),
                 :150-163 (sample_semantic: semantic constraint + RAS),
                 :139-145 (sample_codebook: repetition penalty + nucleus),
                 :168-180 (apply_repetition_penalty), :186-240 (logits_to_probs),
                 :249-263 (multinomial1);
  CosyVoice2 LM  crates/syrinx-lm/src/cv2/sampling.rs:13-22 (log_softmax_vec),
                 :48-60 (multinomial1), :64-87 (nucleus_sampling), :91-95
                 (random_sampling), :104-124 (ras_sampling).
Float types follow the reference: f32 logits and probabilities, f64 sums, exponentials
and uniforms where the reference computes in f64.  An f32 exponential (Rust's f32::exp)
is taken as the correctly rounded value, exp in f64 rounded to f32 (numpy's own float32
exp is a faster, less accurate routine).  Only tests/ use this module.
"""
from __future__ import annotations

import numpy as np

M64 = (1 << 64) - 1


class SplitMix64:
    """state += 0x9E3779B97F4A7C15; z = state; two xor-shift-multiply rounds; z ^ (z >> 31)."""

    def __init__(self, seed: int):
        self.state = seed & M64

    def next_u64(self) -> int:
        self.state = (self.state + 0x9E3779B97F4A7C15) & M64
        z = self.state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
        return z ^ (z >> 31)

    def next_f64(self) -> float:
        return float(self.next_u64() >> 11) * (1.0 / float(1 << 53))


def seq_sum_f64(v) -> float:
    """Left-to-right f64 sum (np.cumsum adds in order; np.sum would add pairwise)."""
    v = np.asarray(v, np.float64)
    return float(np.cumsum(v)[-1]) if v.size else 0.0


def multinomial1(probs, rng: SplitMix64) -> int:
    """Inverse CDF on one uniform: total and running sums in f64, index order."""
    acc = np.cumsum(np.asarray(probs, np.float32).astype(np.float64))
    total = float(acc[-1]) if acc.size else 0.0
    if total <= 0.0:
        return 0
    u = rng.next_f64() * total
    i = int(np.searchsorted(acc, u, side="right"))  # first i with u < acc[i]
    return min(i, len(acc) - 1)


def _desc_order(keys):
    """Indices sorted by key descending, ties by ascending index (a stable sort)."""
    k = np.asarray(keys, np.float32)
    return np.lexsort((np.arange(len(k)), -k.astype(np.float64)))


# ------------------------------------------------------------------ Fish (common/sampling.rs)
def apply_repetition_penalty(logits, recent, penalty: float):
    out = np.array(logits, np.float32, copy=True)
    if abs(np.float32(penalty) - np.float32(1.0)) < np.finfo(np.float32).eps:
        return out
    pen = np.float32(penalty)
    for i in recent:
        if 0 <= int(i) < len(out):
            l = out[int(i)]
            out[int(i)] = (l / pen) if l > 0 else (l * pen)
    return out


def logits_to_probs(logits, temperature: float, top_p: float, top_k: int):
    x = np.asarray(logits, np.float32)
    n = len(x)
    order = _desc_order(x)
    mx = x[order[0]] if n else np.float32(0.0)
    exps = np.exp((x[order] - mx).astype(np.float64))
    total = seq_sum_f64(exps)
    k_cap = n if top_k == 0 else top_k
    keep = np.zeros(n, bool)
    cum = 0.0
    for rank, i in enumerate(order):
        if rank == 0:
            keep[i] = True
        elif cum <= float(np.float32(top_p)) and rank < k_cap:
            keep[i] = True
        else:
            break
        cum += float(exps[rank]) / total
    t = max(np.float32(temperature), np.float32(1e-5))
    kept = np.nonzero(keep)[0]
    scaled = (x[kept] / t).astype(np.float32)
    kmax = scaled.max()
    probs = np.zeros(n, np.float32)
    e = np.exp((scaled - kmax).astype(np.float64))
    psum = seq_sum_f64(e)
    probs[kept] = e.astype(np.float32)
    if psum > 0.0:
        probs[kept] = (probs[kept].astype(np.float64) / psum).astype(np.float32)
    return probs


class FishSampler:
    def __init__(self, seed: int, temperature=1.0, top_p=0.9, top_k=30, repetition_penalty=1.1, ras_win_size=10,
                 ras_high_temp=1.0, ras_high_top_p=0.9):
        self.rng = SplitMix64(seed)
        self.temperature, self.top_p, self.top_k = temperature, top_p, top_k
        self.repetition_penalty = repetition_penalty
        self.ras_win_size, self.ras_high_temp, self.ras_high_top_p = ras_win_size, ras_high_temp, ras_high_top_p

    def sample_codebook(self, logits, recent=()):
        work = apply_repetition_penalty(logits, recent, self.repetition_penalty)
        return multinomial1(logits_to_probs(work, self.temperature, self.top_p, self.top_k), self.rng)

    def sample_semantic(self, logits, window, begin: int, end: int, stop: int):
        c = np.array(logits, np.float32, copy=True)
        ids = np.arange(len(c))
        c[~(((ids >= begin) & (ids <= end)) | (ids == stop))] = -np.inf
        normal = multinomial1(logits_to_probs(c, self.temperature, self.top_p, self.top_k), self.rng)
        high = multinomial1(logits_to_probs(c, self.ras_high_temp, self.ras_high_top_p, self.top_k), self.rng)
        in_window = any(int(t) == normal for t in window)
        return high if (in_window and begin <= normal <= end) else normal


# ------------------------------------------------------------------ CosyVoice2 (cv2/sampling.rs)
def log_softmax_vec(logits):
    v = np.asarray(logits, np.float32)
    m = v.max()
    s = seq_sum_f64(np.exp((v - m).astype(np.float64)))
    lse = float(m) + float(np.log(s))
    return (v.astype(np.float64) - lse).astype(np.float32)


def exp_f32(x):
    """f32 exp, correctly rounded: exp in f64, then rounded to f32."""
    return np.exp(np.asarray(x, np.float32).astype(np.float64)).astype(np.float32)


def nucleus_sampling(logp, top_p: float, top_k: int, rng: SplitMix64) -> int:
    probs = exp_f32(logp)
    order = _desc_order(probs)
    cum = np.float32(0.0)
    cand_idx, cand_prob = [], []
    for i in order:
        if cum < np.float32(top_p) and len(cand_prob) < top_k:
            cum = np.float32(cum + probs[i])
            cand_prob.append(probs[i])
            cand_idx.append(int(i))
        else:
            break
    return cand_idx[multinomial1(np.array(cand_prob, np.float32), rng)]


def random_sampling(logp, rng: SplitMix64) -> int:
    return multinomial1(exp_f32(logp), rng)


def ras_sampling(logits, decoded, rng: SplitMix64, ignore_eos: bool, eos_begin: int, eos_end: int, top_p=0.8,
                 top_k=25, win=10, tau_r=0.1) -> int:
    """log_softmax of the raw logits, the stop ids [eos_begin, eos_end) masked when
    ignore_eos, nucleus draw; a draw repeated >= win * tau_r times among the last win
    decoded tokens is replaced by a draw from the full distribution."""
    logp = log_softmax_vec(logits)
    if ignore_eos:
        logp[eos_begin:eos_end] = -np.inf
    top = nucleus_sampling(logp, top_p, top_k, rng)
    recent = list(decoded)[max(0, len(decoded) - win):]
    rep = sum(1 for t in recent if int(t) == top)
    if np.float32(rep) >= np.float32(win) * np.float32(tau_r):
        return random_sampling(logp, rng)
    return top
