"""Host mirror of the reference's seeded token samplers, drawing on the device (libsxq).

* ``FishSampler`` -- crates/syrinx-fish/src/common/sampling.rs ``Sampler``:
  ``sample_semantic(logits, constraint)`` (:150-163, the driver's RAS window kept on the
  device, common/dualar.rs:188-205) and ``sample_codebook(logits, recent)`` (:139-145).
* ``RasSampler`` -- crates/syrinx-lm/src/cv2/sampling.rs ``ras_sampling`` after
  ``log_softmax_vec`` with the generate loop's token history
  (crates/syrinx-lm/src/cv2/generate.rs:150-161).

Both hold one SplitMix64 state per stream on the device, seeded like the reference, and
write the drawn ids into a device tensor (for example the ids of the next decode step), so
a decode loop never copies logits to the host.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from ._lib import check, lib


class FishSamplingParams(ctypes.Structure):
    _fields_ = [
        ("temperature", ctypes.c_float), ("top_p", ctypes.c_float), ("top_k", ctypes.c_int32),
        ("repetition_penalty", ctypes.c_float), ("ras_win_size", ctypes.c_int32),
        ("ras_high_temp", ctypes.c_float), ("ras_high_top_p", ctypes.c_float),
        ("semantic_begin", ctypes.c_int32), ("semantic_end", ctypes.c_int32), ("stop_id", ctypes.c_int32),
    ]


@dataclass
class SamplingParams:
    """The reference's SamplingParams (common/sampling.rs:42-76), defaults included."""
    temperature: float = 1.0
    top_p: float = 0.9
    top_k: int = 30
    repetition_penalty: float = 1.1
    ras_win_size: int = 10
    ras_high_temp: float = 1.0
    ras_high_top_p: float = 0.9


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _rng_states(seeds, device):
    """SplitMix64 states as 64-bit words (held in an int64 tensor, two's complement)."""
    vals = [(int(s) & ((1 << 64) - 1)) for s in seeds]
    return torch.tensor([v - (1 << 64) if v >= 1 << 63 else v for v in vals], dtype=torch.int64, device=device)


def _dev(device: torch.device) -> int:
    return device.index if device.index is not None else torch.cuda.current_device()


class FishSampler:
    """Per-stream seeded Fish samplers: stream i seeded `seeds[i]` (drive_batch seeds
    sample i with seed + i, common/dualar.rs:246-260)."""

    def __init__(self, seeds, params: SamplingParams = None, semantic=(0, -1, -1), device="cuda:0"):
        self.device = torch.device(device)
        self.n = len(seeds)
        self.params = params or SamplingParams()
        self.rng = _rng_states(seeds, self.device)
        w = max(1, self.params.ras_win_size)
        self.window = torch.zeros((self.n, w), dtype=torch.int32, device=self.device)
        self.window_len = torch.zeros(self.n, dtype=torch.int32, device=self.device)
        self.semantic = semantic  # (begin, end, stop id)

    def _c(self):
        p = self.params
        b, e, stop = self.semantic
        return FishSamplingParams(p.temperature, p.top_p, p.top_k, p.repetition_penalty, p.ras_win_size,
                                  p.ras_high_temp, p.ras_high_top_p, b, e, stop)

    def sample_semantic(self, logits: torch.Tensor, out: torch.Tensor = None, out_stride: int = 1,
                        active: torch.Tensor = None):
        """logits [n, vocab] f32 (device) -> ids [n] int32; with `out` the ids go to
        out[i * out_stride] instead (e.g. column 0 of the next step's frames).  `active`
        int32 [n] (device): streams at 0 draw nothing; a stop draw sets a stream's flag to 0."""
        logits = logits.reshape(self.n, -1)
        if out is None:
            out = torch.empty(self.n, dtype=torch.int32, device=self.device)
        c = self._c()
        check(lib().sxq_sample_semantic(_dev(self.device), _p(logits), logits.stride(0), self.n, logits.shape[1],
                                        ctypes.byref(c), _p(self.rng), _p(self.window), _p(self.window_len),
                                        _p(active), _p(out), out_stride,
                                        torch.cuda.current_stream(self.device).cuda_stream))
        return out

    def sample_codebook(self, logits: torch.Tensor, recent: torch.Tensor = None, out: torch.Tensor = None,
                        out_stride: int = 1, active: torch.Tensor = None):
        logits = logits.reshape(self.n, -1)
        if out is None:
            out = torch.empty(self.n, dtype=torch.int32, device=self.device)
        n_recent = 0 if recent is None else recent.shape[1]
        c = self._c()
        check(lib().sxq_sample_codebook(_dev(self.device), _p(logits), logits.stride(0), self.n, logits.shape[1],
                                        ctypes.byref(c), _p(self.rng), _p(recent), n_recent, _p(active), _p(out),
                                        out_stride, torch.cuda.current_stream(self.device).cuda_stream))
        return out


class RasSampler:
    """CosyVoice ras_sampling per stream (top_p 0.8, top_k 25, window 10, tau_r 0.1 as the
    reference pins them), the stop ids [eos_begin, eos_end) (6561..6564 for CosyVoice2)."""

    def __init__(self, seeds, eos=(6561, 6564), top_p=0.8, top_k=25, win=10, tau_r=0.1, device="cuda:0"):
        self.device = torch.device(device)
        self.n = len(seeds)
        self.rng = _rng_states(seeds, self.device)
        self.decoded = torch.zeros((self.n, max(1, win)), dtype=torch.int32, device=self.device)
        self.decoded_len = torch.zeros(self.n, dtype=torch.int32, device=self.device)
        self.eos, self.top_p, self.top_k, self.win, self.tau_r = eos, top_p, top_k, win, tau_r

    def sample(self, logits: torch.Tensor, ignore_eos: bool, out: torch.Tensor = None, out_stride: int = 1):
        """logits [n, vocab] f32 (device; overwritten with log-probabilities) -> ids [n]."""
        logits = logits.reshape(self.n, -1)
        if out is None:
            out = torch.empty(self.n, dtype=torch.int32, device=self.device)
        check(lib().sxq_sample_ras(_dev(self.device), _p(logits), logits.stride(0), self.n, logits.shape[1],
                                   int(bool(ignore_eos)), self.eos[0], self.eos[1], self.top_p, self.top_k, self.win,
                                   self.tau_r, _p(self.rng), _p(self.decoded), _p(self.decoded_len), _p(out),
                                   out_stride, torch.cuda.current_stream(self.device).cuda_stream))
        return out
