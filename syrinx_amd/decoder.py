"""Host mirror of the decode-step callers of QMatMul, over libsxq's sxq_lm_* C-ABI.

``DecoderLM`` is one Qwen2/Qwen3-style decoder whose every projection is a libsxq
QMatMul and whose whole token step (embedding, layers, head, argmax) runs on the GPU,
optionally as a replayed HIP graph.  Two presets mirror the reference's models:

* ``fish_s2_slow_ar_config`` -- the Fish s2-pro slow AR (Qwen3-4B shape), whose
  ``slow_step(frame, pos)`` is crates/syrinx-fish/src/s2/slow_ar.rs:259-271 and whose
  batched form ``slow_step_batch`` is :456-499;
* ``cosyvoice2_lm_config`` -- the CosyVoice2 Qwen2-0.5B LM, whose
  ``forward_logits_cached(embeds, cache)`` is crates/syrinx-lm/src/cv2/mod.rs:283-286.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, fields

import torch

from ._lib import check, lib
from .quantized import GgmlDType, QMatMul

LM_GRAPH = 1
LM_EXACT = 2       # prefill: Q4_K projections through Candle's integer vec-dot (bit-identical)
LM_ALL_LOGITS = 4  # prefill: logits / hidden for every prompt token
WQKV, WQ, WK, WV, WO, W1, W3, W2, HEAD = range(9)
ATTN_NORM, FFN_NORM, Q_NORM, K_NORM, BQ, BK, BV, FINAL_NORM, HEAD_BIAS, EMBED, CODEBOOK_EMBED, BO = range(12)


class LmConfig(ctypes.Structure):
    _fields_ = [
        ("n_layers", ctypes.c_int32), ("dim", ctypes.c_int32), ("n_heads", ctypes.c_int32),
        ("n_kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32), ("intermediate", ctypes.c_int32),
        ("vocab", ctypes.c_int32), ("embed_rows", ctypes.c_int32), ("max_seq", ctypes.c_int32),
        ("max_batch", ctypes.c_int32), ("weight_dtype", ctypes.c_int32), ("norm_eps", ctypes.c_float),
        ("rope_theta", ctypes.c_float), ("rope_interleaved", ctypes.c_int32), ("qk_norm", ctypes.c_int32),
        ("qkv_bias", ctypes.c_int32), ("head_bias", ctypes.c_int32), ("tied_embedding", ctypes.c_int32),
        ("n_codebooks", ctypes.c_int32), ("codebook_size", ctypes.c_int32), ("semantic_begin", ctypes.c_int32),
        ("semantic_end", ctypes.c_int32), ("o_bias", ctypes.c_int32),
    ]


@dataclass
class DecoderConfig:
    n_layers: int
    dim: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    intermediate: int
    vocab: int
    max_seq: int
    max_batch: int = 1
    weight_dtype: int = int(GgmlDType.Q4K)
    norm_eps: float = 1e-6
    rope_theta: float = 1e6
    rope_interleaved: int = 1
    qk_norm: int = 1
    qkv_bias: int = 0
    head_bias: int = 0
    tied_embedding: int = 1
    embed_rows: int = 0
    n_codebooks: int = 0
    codebook_size: int = 0
    semantic_begin: int = 0
    semantic_end: int = -1
    o_bias: int = 0

    def to_c(self) -> LmConfig:
        c = LmConfig()
        for f in fields(self):
            setattr(c, f.name, getattr(self, f.name))
        return c


def fish_s2_slow_ar_config(n_layers=36, max_seq=1280, max_batch=1, dtype=GgmlDType.Q4K, n_codebooks=10,
                           **kw) -> DecoderConfig:
    """Qwen3-4B slow AR of Fish s2-pro (crates/syrinx-fish/src/common/config.rs:194-251):
    36 layers, dim 2560, 32/8 heads of 128, SwiGLU 9728, eps 1e-6, RoPE base 1e6
    interleaved, QK-RMSNorm, no qkv/o bias, head tied to the 155776-row embedding, MCF
    over 10 codebooks of 4096 (semantic ids 151678..155773)."""
    base = dict(n_layers=n_layers, dim=2560, n_heads=32, n_kv_heads=8, head_dim=128, intermediate=9728,
                vocab=155776, max_seq=max_seq, max_batch=max_batch, weight_dtype=int(dtype), norm_eps=1e-6,
                rope_theta=1e6, rope_interleaved=1, qk_norm=1, qkv_bias=0, head_bias=0, tied_embedding=1,
                n_codebooks=n_codebooks, codebook_size=4096 if n_codebooks else 0, semantic_begin=151678,
                semantic_end=155773)
    base.update(kw)
    return DecoderConfig(**base)


def cosyvoice2_lm_config(n_layers=24, max_seq=1024, max_batch=1, dtype=GgmlDType.Q8_0, **kw) -> DecoderConfig:
    """CosyVoice2 Qwen2-0.5B LM (crates/syrinx-lm/src/cv2/mod.rs:36-56): 24 layers, hidden
    896, 14/2 heads of 64, SwiGLU 4864, eps 1e-6, RoPE theta 1e6 rotate-half, q/k/v
    biases, llm_decoder head [6564 x 896] with bias, speech embedding table."""
    base = dict(n_layers=n_layers, dim=896, n_heads=14, n_kv_heads=2, head_dim=64, intermediate=4864,
                vocab=6564, max_seq=max_seq, max_batch=max_batch, weight_dtype=int(dtype), norm_eps=1e-6,
                rope_theta=1e6, rope_interleaved=0, qk_norm=0, qkv_bias=1, head_bias=1, tied_embedding=0,
                embed_rows=6564 + 3)
    base.update(kw)
    return DecoderConfig(**base)


def cosyvoice3_lm_config(n_layers=24, max_seq=1024, max_batch=1, dtype=GgmlDType.Q8_0, **kw) -> DecoderConfig:
    """CosyVoice3 LM (crates/syrinx-lm/src/cv3/mod.rs:44-68, lm.rs:143-147): the CosyVoice2
    Qwen2-0.5B body with a bias-free llm_decoder [6761 x 896] (6561 speech ids + 200
    control ids) and a 6761-row speech_embedding, which also holds the sos / task_id rows."""
    base = dict(head_bias=0, vocab=6761, embed_rows=6761)
    base.update(kw)
    return cosyvoice2_lm_config(n_layers=n_layers, max_seq=max_seq, max_batch=max_batch, dtype=dtype, **base)


def fish_s2_fast_ar_config(n_layers=4, num_codebooks=10, residual_size=4096, max_batch=1, dtype=GgmlDType.Q4K,
                           **kw) -> DecoderConfig:
    """The s2-pro fast AR (the audio decoder, crates/syrinx-fish/src/s2/fast_ar.rs:1-66):
    4 layers of the slow block's geometry (dim 2560, 32/8 heads of 128, SwiGLU 9728, eps
    1e-6) with no QK-norm and no qkv/o bias, interleaved RoPE (base 1e6) over the codebook
    axis, a local cache of num_codebooks positions, the shared fast_embeddings table
    [residual_size, 2560] as its input and fast_output [residual_size, 2560] as its head."""
    base = dict(n_layers=n_layers, dim=2560, n_heads=32, n_kv_heads=8, head_dim=128, intermediate=9728,
                vocab=residual_size, max_seq=num_codebooks, max_batch=max_batch, weight_dtype=int(dtype),
                norm_eps=1e-6, rope_theta=1e6, rope_interleaved=1, qk_norm=0, qkv_bias=0, head_bias=0,
                tied_embedding=0, embed_rows=residual_size)
    base.update(kw)
    return DecoderConfig(**base)


class DecoderLM:
    """A decode-step engine (sxq_lm) on one GPU."""

    def __init__(self, cfg: DecoderConfig, device="cuda:0"):
        self.cfg = cfg
        self.device = torch.device(device)
        self._h = ctypes.c_void_p()
        self._c = cfg.to_c()
        check(lib().sxq_lm_create(self._dev(), ctypes.byref(self._c), ctypes.byref(self._h)))
        self.ids_per = 1 + cfg.n_codebooks

    def _dev(self) -> int:
        return self.device.index if self.device.index is not None else torch.cuda.current_device()

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            try:
                lib().sxq_lm_destroy(h)
            except Exception:
                pass
            self._h = None

    # -- weights ----------------------------------------------------------------------
    def set_linear(self, layer: int, which: int, qmm: QMatMul) -> None:
        check(lib().sxq_lm_set_linear(self._h, layer, which, ctypes.c_void_p(qmm.handle())))

    def set_vector(self, layer: int, which: int, data: torch.Tensor) -> None:
        t = data.detach().to(device=self.device, dtype=torch.float32).contiguous()
        torch.cuda.current_stream(self.device).synchronize()
        check(lib().sxq_lm_set_vector(self._h, layer, which, ctypes.c_void_p(t.data_ptr()), t.numel(), 1))

    def set_embed_quantized(self, qe) -> None:
        """Hold the input table (EMBED) as a QEmbed: steps and prefill gather-dequantize it."""
        torch.cuda.current_stream(self.device).synchronize()
        check(lib().sxq_lm_set_embed_quantized(self._h, qe.scheme, ctypes.c_void_p(qe.q.data_ptr()),
                                                ctypes.c_void_p(qe.scale.data_ptr())))

    def init_random(self, seed: int = 0, std: float = 0.02) -> None:
        check(lib().sxq_lm_init_random(self._h, seed, std))

    def kv_fill_random(self, lengths, seed: int = 0) -> None:
        arr = (ctypes.c_int32 * len(lengths))(*lengths)
        check(lib().sxq_lm_kv_fill_random(self._h, arr, len(lengths), seed))

    def set_lengths(self, lengths) -> None:
        arr = (ctypes.c_int32 * len(lengths))(*lengths)
        check(lib().sxq_lm_set_lengths(self._h, arr, len(lengths)))

    def lengths(self, n=None):
        n = n or self.cfg.max_batch
        arr = (ctypes.c_int32 * n)()
        check(lib().sxq_lm_get_lengths(self._h, arr, n))
        return list(arr)

    def reset(self, n=None) -> None:
        """SlowAr::reset (slow_ar.rs:79-81): empty the caches of streams 0..n-1, ordered on
        the current stream."""
        check(lib().sxq_lm_reset(self._h, n or self.cfg.max_batch, torch.cuda.current_stream(self.device).cuda_stream))

    def weight_bytes(self):
        lb, hb = ctypes.c_size_t(), ctypes.c_size_t()
        check(lib().sxq_lm_weight_bytes(self._h, ctypes.byref(lb), ctypes.byref(hb)))
        return int(lb.value), int(hb.value)

    PATH_ATTN, PATH_ATTN_WO, PATH_SWIGLU = 1, 2, 4

    def paths(self) -> int:
        """The fused launches a one-stream step runs (tests): PATH_* bits."""
        p = ctypes.c_uint()
        check(lib().sxq_lm_paths(self._h, ctypes.byref(p)))
        return int(p.value)

    # -- step ---------------------------------------------------------------------------
    def step(self, ids: torch.Tensor = None, embeds: torch.Tensor = None, n: int = None, graph: bool = False,
             want_logits: bool = True, want_hidden: bool = False, out=None):
        """One token for n streams.  ids int32 [n, 1 + n_codebooks] (or [n]) or embeds
        f32 [n, dim]; None for both reuses the previous argmax.  Returns (logits, next_ids),
        or (logits, next_ids, hidden) with want_hidden (the post-final-RMSNorm state).
        out = (logits, next_ids, hidden) writes into those device tensors instead (fixed
        buffers for a loop whose later launches are captured on their addresses)."""
        if ids is not None:
            ids = ids.to(device=self.device, dtype=torch.int32).reshape(-1, self.ids_per).contiguous()
            n = ids.shape[0]
        if embeds is not None:
            embeds = embeds.to(device=self.device, dtype=torch.float32).reshape(-1, self.cfg.dim).contiguous()
            n = embeds.shape[0]
        if n is None:
            raise ValueError("step: give ids, embeds or n")
        if out is not None:
            logits, nxt, hidden = out
            for t, w in ((logits, self.cfg.vocab), (hidden, self.cfg.dim)):
                if t is not None and (t.dtype != torch.float32 or not t.is_contiguous() or t.numel() != n * w):
                    raise ValueError("step: out buffers must be contiguous f32 of n rows")
            want_hidden = True
        else:
            logits = torch.empty((n, self.cfg.vocab), dtype=torch.float32, device=self.device) if want_logits else None
            nxt = torch.empty((n,), dtype=torch.int32, device=self.device)
            hidden = torch.empty((n, self.cfg.dim), dtype=torch.float32, device=self.device) if want_hidden else None
        P = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None  # noqa: E731
        check(lib().sxq_lm_step(self._h, n, P(ids), P(embeds), P(logits), P(hidden), P(nxt), LM_GRAPH if graph else 0,
                                torch.cuda.current_stream(self.device).cuda_stream))
        return (logits, nxt, hidden) if want_hidden else (logits, nxt)

    def prefill(self, prompts=None, embeds=None, exact: bool = False, all_logits: bool = False, trace: bool = False):
        """Prompt prefill of streams 0..n-1 (sxq_lm_prefill): prompts is a list (one entry
        per stream) of int32 token frames [T_s, 1 + n_codebooks] (or [T_s]), or embeds a
        list of f32 [T_s, dim].  Each stream's tokens go at its current length, which then
        advances by T_s.  Returns (logits, next_ids, hidden): logits [n, vocab] and hidden
        [n, dim] of each stream's last token, or [sum T_s, ...] with all_logits; with
        trace=True a fourth item, the trace of every intermediate (as trace())."""
        c = self.cfg
        if (prompts is None) == (embeds is None):
            raise ValueError("prefill: give prompts or embeds")
        rows = prompts if prompts is not None else embeds
        n = len(rows)
        if prompts is not None:
            mats = [torch.as_tensor(p, dtype=torch.int32).reshape(-1, self.ids_per) for p in prompts]
        else:
            mats = [torch.as_tensor(e, dtype=torch.float32).reshape(-1, c.dim) for e in embeds]
        counts = [int(m.shape[0]) for m in mats]
        T = sum(counts)
        data = torch.cat(mats).to(self.device).contiguous()
        out_rows = T if all_logits else n
        logits = torch.empty((out_rows, c.vocab), dtype=torch.float32, device=self.device)
        hidden = torch.empty((out_rows, c.dim), dtype=torch.float32, device=self.device)
        nxt = torch.empty((n,), dtype=torch.int32, device=self.device)
        tr = None
        if trace:
            sz = ctypes.c_size_t()
            check(lib().sxq_lm_prefill_trace_floats(self._h, T, ctypes.byref(sz)))
            tr = torch.zeros(int(sz.value), dtype=torch.float32, device=self.device)
        P = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None  # noqa: E731
        cnt = (ctypes.c_int32 * n)(*counts)
        flags = (LM_EXACT if exact else 0) | (LM_ALL_LOGITS if all_logits else 0)
        check(lib().sxq_lm_prefill(self._h, n, cnt, P(data) if prompts is not None else None,
                                   P(data) if embeds is not None else None, P(logits), P(hidden), P(nxt), flags,
                                   P(tr), tr.numel() if tr is not None else 0,
                                   torch.cuda.current_stream(self.device).cuda_stream))
        if trace:
            return logits, nxt, hidden, self._parse_trace(tr.cpu().numpy(), T, out_rows)
        return logits, nxt, hidden

    TRACE_SEGMENTS = ("hn_attn", "qkv", "q", "ctx", "h_mid", "hn_ffn", "gu", "act", "h_out")

    def enable_trace(self, on: bool = True) -> None:
        """Record every f32 intermediate of each following step (tests)."""
        if not on:
            check(lib().sxq_lm_set_trace(self._h, None, 0))
            self._trace = None
            return
        sz = ctypes.c_size_t()
        check(lib().sxq_lm_trace_floats(self._h, self.cfg.max_batch, ctypes.byref(sz)))
        self._trace = torch.zeros(int(sz.value), dtype=torch.float32, device=self.device)
        check(lib().sxq_lm_set_trace(self._h, ctypes.c_void_p(self._trace.data_ptr()), int(sz.value)))

    def trace(self, n: int) -> dict:
        """The last traced step of n streams: {'embed': [n, dim], 'final_hn': [n, dim],
        'layers': [{segment: [n, size]} per layer]} as numpy arrays."""
        return self._parse_trace(self._trace.cpu().numpy(), n, n)

    def _parse_trace(self, t, n: int, n_final: int) -> dict:
        c = self.cfg
        qkv_n = (c.n_heads + 2 * c.n_kv_heads) * c.head_dim
        ctx = c.n_heads * c.head_dim
        sizes = dict(hn_attn=c.dim, qkv=qkv_n, q=ctx, ctx=ctx, h_mid=c.dim, hn_ffn=c.dim, gu=2 * c.intermediate,
                     act=c.intermediate, h_out=c.dim)
        off = 0

        def take(size):
            nonlocal off
            a = t[off: off + n * size].reshape(n, size)
            off += n * size
            return a

        out = {"embed": take(c.dim), "layers": []}
        for _ in range(c.n_layers):
            out["layers"].append({seg: take(sizes[seg]) for seg in self.TRACE_SEGMENTS})
        out["final_hn"] = t[off: off + n_final * c.dim].reshape(n_final, c.dim)
        return out

    def read_state(self, which: int, n: int = 1) -> torch.Tensor:
        """A step buffer (tests): 0 residual after the last layer, 1 logits, 2 last qkv,
        3 last gate|up, 4 last post-RoPE queries, 5 the silu(g)*u row of the fused one-row
        gate|up GEMV (zero until it runs)."""
        c = self.cfg
        per = {0: c.dim, 1: c.vocab, 2: (c.n_heads + 2 * c.n_kv_heads) * c.head_dim, 3: 2 * c.intermediate,
               4: c.n_heads * c.head_dim, 5: c.intermediate}[which]
        out = torch.empty((n, per), dtype=torch.float32, device=self.device)
        check(lib().sxq_lm_read_state(self._h, which, n, ctypes.c_void_p(out.data_ptr()),
                                      torch.cuda.current_stream(self.device).cuda_stream))
        return out

    def read_kv(self, layer: int, stream: int, kv_head: int, pos0: int, count: int):
        hd = self.cfg.head_dim
        k = torch.empty((count, hd), dtype=torch.float32, device=self.device)
        v = torch.empty_like(k)
        check(lib().sxq_lm_read_kv(self._h, layer, stream, kv_head, pos0, count, ctypes.c_void_p(k.data_ptr()),
                                   ctypes.c_void_p(v.data_ptr()), torch.cuda.current_stream(self.device).cuda_stream))
        return k, v


class SlowAr(DecoderLM):
    """Fish s2 slow AR decode (crates/syrinx-fish/src/s2/slow_ar.rs)."""

    project_in = None       # fast_project_in QMatMul [fast_dim, dim] (a narrower fast AR), or None
    project_in_bias = None  # its bias (device f32 [fast_dim]), or None

    def set_project_in(self, qmm: QMatMul, bias: torch.Tensor = None) -> None:
        """A checkpoint's fast_project_in (slow_ar.rs:230-243): every hidden this engine
        returns for the fast AR is then linear(normed, fast_project_in.weight[, .bias]),
        a QMatMul forward on the device, instead of the post-norm hidden itself."""
        if qmm.shape[1] != self.cfg.dim:
            raise ValueError(f"fast_project_in takes {qmm.shape[1]} inputs, the slow AR's hidden has {self.cfg.dim}")
        self.project_in = qmm
        self.project_in_bias = None if bias is None else bias.detach().to(self.device, torch.float32).contiguous()

    @property
    def hidden_dim(self) -> int:
        """Width of the hidden handed to the fast AR (fast_dim with a project_in)."""
        return self.cfg.dim if self.project_in is None else self.project_in.shape[0]

    def _fast_hidden(self, raw: torch.Tensor, out: torch.Tensor = None) -> torch.Tensor:
        """raw [n, dim] post-norm hidden -> the fast AR's hidden [n, hidden_dim] (into out)."""
        if self.project_in is None:
            return raw if out is None else out
        y = self.project_in.forward(raw.reshape(-1, self.cfg.dim), self.project_in_bias)
        if out is None:
            return y
        out.view(-1, self.hidden_dim).copy_(y)
        return out

    def slow_step(self, frame, pos: int = None, graph: bool = True):
        """frame: [1 + num_codebooks] ids of the previous frame; pos must equal the cache
        length (slow_ar.rs:259-271).  Returns (semantic_logits [vocab], hidden [1, 1, dim]),
        as SlowAr::slow_step does; the greedy argmax of the logits is kept on the device
        and read with last_argmax()."""
        if pos is not None and pos != self.lengths(1)[0]:
            raise ValueError(f"slow_step pos {pos} must equal the current cache length {self.lengths(1)[0]}")
        ids = torch.as_tensor(frame, dtype=torch.int32).reshape(1, -1)
        logits, nxt, hidden = self.step(ids=ids, graph=graph, want_hidden=True)
        self._last_argmax = nxt
        return logits[0], self._fast_hidden(hidden).reshape(1, 1, -1)

    def slow_step_batch(self, frames, graph: bool = True, out=None):
        """frames: [n, 1 + num_codebooks]; ragged cache lengths need no left padding
        (slow_ar.rs:456-499).  Returns (semantic_logits [n, vocab], hidden [n, 1, hidden_dim]);
        out = (logits, next_ids, hidden) as for step() (hidden [n, hidden_dim])."""
        hid_out = None
        if out is not None and self.project_in is not None:  # the step writes the raw hidden first
            raw = torch.empty((out[0].shape[0], self.cfg.dim), dtype=torch.float32, device=self.device)
            out, hid_out = (out[0], out[1], raw), out[2]
        logits, nxt, hidden = self.step(ids=torch.as_tensor(frames, dtype=torch.int32), graph=graph, want_hidden=True,
                                        out=out)
        self._last_argmax = nxt
        return logits, self._fast_hidden(hidden, hid_out).reshape(-1, 1, self.hidden_dim)

    def prefill(self, prompt, graph: bool = False):
        """SlowAr::prefill (slow_ar.rs:250-256): prompt [1 + num_codebooks, T] (rows =
        semantic ids then codebooks) into the cache at its current length.  Returns
        (semantic_logits [vocab], hidden [1, 1, dim]) of the last prompt position."""
        p = torch.as_tensor(prompt, dtype=torch.int32).reshape(self.ids_per, -1).t().contiguous()
        logits, nxt, hidden = super().prefill(prompts=[p])
        self._last_argmax = nxt
        return logits[0], self._fast_hidden(hidden).reshape(1, 1, -1)

    def prefill_batch(self, prompts):
        """SlowAr::prefill_batch (slow_ar.rs:404-454): ragged prompts [1 + num_codebooks,
        T_i], one per stream, without left padding.  Returns (logits [n, vocab], hidden
        [n, 1, dim]) of every stream's last prompt position."""
        ps = [torch.as_tensor(p, dtype=torch.int32).reshape(self.ids_per, -1).t().contiguous() for p in prompts]
        logits, nxt, hidden = super().prefill(prompts=ps)
        self._last_argmax = nxt
        return logits, self._fast_hidden(hidden).reshape(len(ps), 1, -1)

    def last_argmax(self) -> torch.Tensor:
        """Greedy argmax ids [n] of the last step's logits (device int32)."""
        return self._last_argmax


class Qwen2Lm(DecoderLM):
    """CosyVoice2 LM cached decode (crates/syrinx-lm/src/cv2/mod.rs:255-286)."""

    def forward_logits_cached(self, embeds: torch.Tensor, graph: bool = True):
        """embeds [b, t_new, 896] -> logits [b, t_new, 6564] for the new positions of every
        stream (cv2/mod.rs:283-286): one decode step for t_new = 1, the prompt prefill with
        every position's logits otherwise."""
        b, t = embeds.shape[0], embeds.shape[1] if embeds.dim() == 3 else 1
        if t == 1:
            logits, _ = self.step(embeds=embeds.reshape(b, -1), graph=graph)
            return logits.reshape(b, 1, -1)
        logits, _, _ = self.prefill(embeds=[embeds[i].reshape(t, -1) for i in range(b)], all_logits=True)
        return logits.reshape(b, t, -1)


class FastAr(DecoderLM):
    """Fish s2 fast AR (crates/syrinx-fish/src/s2/fast_ar.rs:28-224) over the decode engine:
    the per-frame expansion of one slow hidden into num_codebooks codes runs on the device,
    drawing each residual code with the driver's FishSampler (sxq_fish_fast_expand)."""

    def first_code(self, semantic_token: int, semantic_begin: int) -> int:
        """FastAr::first_code (fast_ar.rs:105-110): clamp(tok - begin, 0, residual - 1),
        saturating at 0."""
        return min(max(int(semantic_token) - int(semantic_begin), 0), self.cfg.vocab - 1)

    def expand_batch(self, hidden: torch.Tensor, semantic: torch.Tensor, sampler, active: torch.Tensor = None,
                     codes: torch.Tensor = None, graph: bool = True, n_codes: int = None):
        """FastAr::expand_batch (fast_ar.rs:170-224).  hidden f32 [n, 1, dim] (device), the
        sampled semantic ids (device int32: [n], or a column view such as frames[:, 0] of a
        [n, 1 + n_codes] ids frame), `sampler` a FishSampler of n streams (its rng advances
        by one draw per residual code of each active stream), `active` int32 [n] or None.
        Writes and returns codes [n, n_codes] (or the given strided view, e.g. frames[:, 1:])
        with codes[:, 0] = first_code(semantic)."""
        n_codes = n_codes or self.cfg.max_seq
        hidden = hidden.reshape(-1, self.cfg.dim)
        n = hidden.shape[0]
        if hidden.dtype != torch.float32 or not hidden.is_contiguous() or hidden.device != self.device:
            raise ValueError("expand_batch: hidden must be contiguous f32 on the engine's device")
        if semantic.dtype != torch.int32 or semantic.device != self.device or semantic.shape[0] != n:
            raise ValueError("expand_batch: semantic must be int32 [n] on the engine's device")
        if codes is None:
            codes = torch.empty((n, n_codes), dtype=torch.int32, device=self.device)
        if codes.dtype != torch.int32 or codes.shape[0] != n or codes.shape[-1] < n_codes or codes.stride(-1) != 1:
            raise ValueError("expand_batch: codes must be int32 [n, >= n_codes] with unit column stride")
        if sampler.n != n:
            raise ValueError(f"expand_batch: the sampler holds {sampler.n} streams, not {n}")
        c = sampler._c()
        P = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None  # noqa: E731
        check(lib().sxq_fish_fast_expand(self._h, n, P(hidden), P(semantic), semantic.stride(0), P(active),
                                         ctypes.byref(c), P(sampler.rng), n_codes, P(codes), codes.stride(0),
                                         LM_GRAPH if graph else 0, torch.cuda.current_stream(self.device).cuda_stream))
        return codes

    def expand(self, hidden: torch.Tensor, first_code: int, sampler, graph: bool = True):
        """FastAr::expand (fast_ar.rs:116-160) for one frame: returns the num_codebooks
        codes (a host list, index 0 == first_code)."""
        sem = torch.tensor([int(first_code) + sampler.semantic[0]], dtype=torch.int32, device=self.device)
        return self.expand_batch(hidden, sem, sampler, graph=graph)[0].tolist()

