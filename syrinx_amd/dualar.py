"""The Fish dual-AR generation loop over the device engines (common/dualar.rs).

``drive`` (crates/syrinx-fish/src/common/dualar.rs:163-238) and ``drive_batch``
(:240-360) with the s2 backend's pieces on the GPU: the slow AR prefill and steps
(``SlowAr``), the semantic draw with its RAS window (``FishSampler.sample_semantic``),
the frame expansion (``FastAr.expand_batch``, its nine residual draws from the same
sampler) and the feedback of the full frame ``[semantic, code 0 .. code 9]`` into the next
slow step.  Every token stays on the device: the frame a slow step consumes is the buffer
the samplers wrote, and a stream that draws the stop id is frozen by the samplers'
``active`` flags (no further draws, an inert zero frame), so the host only reads one flag
per stream and frame to know when all streams have stopped.  That read overlaps the next
slow step, which is enqueued first (its output is unused when every stream has stopped).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

from .decoder import FastAr, SlowAr
from .sampling import FishSampler, SamplingParams


@dataclass
class DriveParams:
    """DriveParams (common/dualar.rs:136-161), defaults included."""
    max_new_frames: int = 2048
    seed: int = 42
    sampling: SamplingParams = field(default_factory=SamplingParams)


def drive(slow: SlowAr, fast: FastAr, prompt, stop_id: int, params: DriveParams = None) -> torch.Tensor:
    """drive (dualar.rs:163-238): prompt [1 + num_codebooks, T] -> the [num_codebooks, T_gen]
    code matrix (int32, on the device).  Sample i of drive_batch reproduces drive seeded
    seed + i (the reference's own contract, dualar.rs:244-252), so one prompt is a batch of one."""
    return drive_batch(slow, fast, [prompt], stop_id, params)[0]


def drive_batch(slow: SlowAr, fast: FastAr, prompts, stop_id: int, params: DriveParams = None):
    """drive_batch (dualar.rs:240-360): one [num_codebooks, T_i] matrix per prompt, each cut
    at its own stop.  The semantic constraint is the slow engine's semantic range plus
    stop_id (the tokenizer's <|im_end|> id, FishConfig::stop_token_id)."""
    params = params or DriveParams()
    c = slow.cfg
    n_cb = c.n_codebooks
    n = len(prompts)
    if n == 0:
        return []
    if n > min(c.max_batch, fast.cfg.max_batch):
        raise ValueError(f"drive_batch: {n} prompts exceed the engines' max_batch")
    if fast.cfg.max_seq < n_cb:
        raise ValueError("drive_batch: the fast engine's cache is shorter than a frame")
    if slow.hidden_dim != fast.cfg.dim:
        raise ValueError(f"drive_batch: the slow AR hands over {slow.hidden_dim}-wide hiddens, the fast AR is "
                         f"{fast.cfg.dim} wide (a narrower fast AR needs fast_project_in)")
    dev = slow.device
    stop = int(stop_id)
    sampler = FishSampler([params.seed + i for i in range(n)], params.sampling, semantic=(c.semantic_begin,
                          c.semantic_end, stop), device=dev)
    prompts = [torch.as_tensor(p, dtype=torch.int32).reshape(1 + n_cb, -1) for p in prompts]
    tmax = max(int(p.shape[1]) for p in prompts)

    slow.reset(n)
    logits0, hidden0 = slow.prefill_batch(prompts)
    frames, flags = generate_frames(slow, fast, sampler, logits0, hidden0, params.max_new_frames, tmax)
    f = torch.stack(frames)      # [T, n, 1 + n_cb]
    a = torch.stack(flags)       # [T, n]: the frame of step t counts for stream i when still active
    out = []
    for i in range(n):
        keep = a[:, i] != 0
        out.append(f[keep, i, 1:].t().contiguous())
    return out


def generate_frames(slow: SlowAr, fast: FastAr, sampler: FishSampler, logits0, hidden0, max_new_frames: int,
                    pos: int, active: torch.Tensor = None, frame: torch.Tensor = None):
    """The frame loop of drive_batch (dualar.rs:286-346) from a prefilled slow cache whose
    last step gave logits0 [n, vocab] and hidden0 [n, 1, dim]; pos is the longest stream's
    cache length.  Returns the frames [n, 1 + n_cb] of every pass and the streams' active
    flags after each pass's semantic draw (device tensors; the host has synchronised).
    `active` / `frame` may be passed to keep their buffers (and the captured expansion)
    across calls."""
    c = slow.cfg
    n_cb = c.n_codebooks
    n = logits0.shape[0]
    dev = slow.device
    # fixed buffers: the expansion graph is captured on their addresses
    logits = logits0.contiguous()
    hidden = hidden0.reshape(n, slow.hidden_dim).contiguous()
    nxt = torch.empty(n, dtype=torch.int32, device=dev)
    if frame is None:
        frame = torch.zeros((n, 1 + n_cb), dtype=torch.int32, device=dev)
    if active is None:
        active = torch.ones(n, dtype=torch.int32, device=dev)
    frames, flags = [], []
    flag_host = torch.empty(n, dtype=torch.int32, pin_memory=True)
    done = torch.cuda.Event()
    for _ in range(max_new_frames):
        # 1. each active stream's semantic draw (a stop freezes the stream); 2. the frame
        sampler.sample_semantic(logits, out=frame[:, 0], out_stride=1 + n_cb, active=active)
        fast.expand_batch(hidden, frame[:, 0], sampler, active=active, codes=frame[:, 1:], n_codes=n_cb)
        frames.append(frame.clone())
        flags.append(active.clone())
        flag_host.copy_(active, non_blocking=True)
        done.record()
        if len(frames) >= max_new_frames or pos + 1 >= c.max_seq:
            break
        # 4. feed the frame back (enqueued before the host looks at the flags)
        slow.slow_step_batch(frame, out=(logits, nxt, hidden))
        pos += 1
        done.synchronize()
        if not bool(flag_host.any()):
            break
    torch.cuda.current_stream(dev).synchronize()
    return frames, flags
