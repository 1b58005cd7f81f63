"""CosyVoice speech-token generation over the device decode engine.

``CosyVoiceLm`` mirrors the two autoregressive loops of the reference's CosyVoice LMs:

* ``Qwen2Lm::generate`` (crates/syrinx-lm/src/cv2/generate.rs:136-163): the step-0 input
  ``[llm_embedding[sos], embed_tokens(text), llm_embedding[task_id], speech_embedding(prompt)]``
  (``build_lm_input``, :89-101), one cached prefill, then per token ``log_softmax`` ->
  ``ras_sampling`` (EOS masked while ``i < min_len``) -> stop on ``STOP_TOKENS``
  (6561..6563) -> feed the token's ``speech_embedding`` row back;
* ``Cv3Lm::generate`` / ``generate_instruct`` (crates/syrinx-lm/src/cv3/generate.rs:14-101):
  the same loop with ``sos`` / ``task_id`` taken from ``speech_embedding`` (rows 6561 / 6563,
  crates/syrinx-lm/src/cv3/lm.rs:81-92), a bias-free 6761-row head and every control id
  ``>= 6561`` a stop (also the ``min_len`` mask).

Everything a token touches stays on the GPU: the sampler (``RasSampler``, its SplitMix64
state and the decoded-token window on the device) writes the drawn id straight into the
buffer the next decode step reads, and the step embeds it from the engine's own
speech-embedding table.  The host reads one 4-byte id per token to decide when to stop,
and that read overlaps the next step, which is enqueued first (after a stop its output is
discarded).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .decoder import Qwen2Lm
from .embedding import QEmbed
from .sampling import RasSampler


@dataclass(frozen=True)
class CvVariant:
    """The constants one CosyVoice LM generation loop uses."""
    name: str
    sos: int                # row of the sos embedding (in llm_embedding for CosyVoice2, speech_embedding for 3)
    task_id: int            # row of the task_id embedding (same table as sos)
    sos_task_table: str     # "llm" or "speech"
    stop_begin: int         # stop ids: [stop_begin, stop_end) -- also the ids masked while i < min_len
    stop_end: int


# cv2/mod.rs:47-56 (SOS 0, TASK_ID 1 of llm_embedding; STOP_TOKENS 6561..6563; SPEECH_VOCAB 6564)
COSYVOICE2 = CvVariant("cosyvoice2", 0, 1, "llm", 6561, 6564)
# cv3/mod.rs:49-56 (SOS 6561, TASK_ID 6563 of speech_embedding; every id >= 6561 of the 6761 stops)
COSYVOICE3 = CvVariant("cosyvoice3", 6561, 6563, "speech", 6561, 6761)


def _rows(table, ids) -> torch.Tensor:
    """embed_rows (cv2/generate.rs:22-67): a dense f32 table's rows, or a QEmbed's rows
    dequantized on gather."""
    if isinstance(table, QEmbed):
        return table.rows(ids)
    idx = torch.as_tensor(list(ids), dtype=torch.int64, device=table.device)
    return table.index_select(0, idx).to(torch.float32)


class CosyVoiceLm:
    """A CosyVoice LM (Qwen2Lm engine + the embedding tables its prompt is built from).

    lm              the decode engine; its input table (SXQ_LM_EMBED, dense or a QEmbed via
                    set_embed_quantized) must be `speech_embed`, which every fed-back token
                    gathers from
    text_embed      llm.model.model.embed_tokens.weight: f32 [rows, dim] tensor or QEmbed
    speech_embed    speech_embedding.weight, likewise
    llm_embed       llm_embedding.weight (CosyVoice2's sos / task_id rows), or None for CosyVoice3
    """

    def __init__(self, lm: Qwen2Lm, text_embed, speech_embed, llm_embed=None, variant: CvVariant = COSYVOICE2):
        if variant.sos_task_table == "llm" and llm_embed is None:
            raise ValueError(f"{variant.name}: sos / task_id come from llm_embedding, which is missing")
        if lm.cfg.vocab < variant.stop_end:
            raise ValueError(f"{variant.name}: the head has {lm.cfg.vocab} outputs, the stop ids reach {variant.stop_end}")
        if lm.cfg.max_batch < 1:
            raise ValueError("the engine needs a stream")
        self.lm, self.text, self.speech, self.llm, self.v = lm, text_embed, speech_embed, llm_embed, variant

    def _sos_task(self, row: int) -> torch.Tensor:
        return _rows(self.llm if self.v.sos_task_table == "llm" else self.speech, [row])

    def build_lm_input(self, text_token, prompt_speech_token=()) -> torch.Tensor:
        """Qwen2Lm::build_lm_input (cv2/generate.rs:89-101) / Cv3Lm::build_lm_input
        (cv3/lm.rs:81-92): [sos, embed_tokens(text), task_id, speech_embedding(prompt)] ->
        f32 [T0, dim] on the device (the prompt-speech segment omitted when empty)."""
        parts = [self._sos_task(self.v.sos), _rows(self.text, text_token), self._sos_task(self.v.task_id)]
        if len(prompt_speech_token):
            parts.append(_rows(self.speech, prompt_speech_token))
        return torch.cat(parts, 0).contiguous()

    def build_lm_input_instruct(self, instruct_token, text_token) -> torch.Tensor:
        """Cv3Lm::build_lm_input_instruct (cv3/lm.rs:93-132): [sos, embed_tokens(instruct),
        embed_tokens(text), task_id], no prompt-speech segment."""
        return torch.cat([self._sos_task(self.v.sos), _rows(self.text, instruct_token), _rows(self.text, text_token),
                          self._sos_task(self.v.task_id)], 0).contiguous()

    def generate(self, text_token, prompt_speech_token, min_len: int, max_len: int, seed: int,
                 graph: bool = True, sampler: RasSampler = None):
        """Qwen2Lm::generate / Cv3Lm::generate: the generated speech-token ids (stop
        excluded), the cache starting empty.  `sampler` (one stream) may be passed to keep
        its rng and window for inspection; it is seeded `seed` otherwise."""
        return self.generate_from(self.build_lm_input(text_token, prompt_speech_token), min_len, max_len, seed,
                                  graph, sampler)

    def generate_instruct(self, instruct_token, text_token, min_len: int, max_len: int, seed: int,
                          graph: bool = True, sampler: RasSampler = None):
        """Cv3Lm::generate_instruct (cv3/generate.rs:14-44)."""
        return self.generate_from(self.build_lm_input_instruct(instruct_token, text_token), min_len, max_len, seed,
                                  graph, sampler)

    def generate_from(self, lm_input0: torch.Tensor, min_len: int, max_len: int, seed: int, graph: bool = True,
                      sampler: RasSampler = None):
        """The loop of both generate functions from an assembled step-0 input [T0, dim]."""
        lm, v = self.lm, self.v
        dev = lm.device
        if lm_input0.shape[0] + max_len > lm.cfg.max_seq + 1:
            raise ValueError(f"generate: {lm_input0.shape[0]} prompt rows + {max_len} tokens exceed the cache "
                             f"({lm.cfg.max_seq} positions)")
        smp = sampler or RasSampler([seed], eos=(v.stop_begin, v.stop_end), device=dev)
        if smp.n != 1 or tuple(smp.eos) != (v.stop_begin, v.stop_end):
            raise ValueError("generate: the sampler must hold one stream with this variant's stop ids")
        lm.reset(1)
        logits, _, _ = lm.prefill(embeds=[lm_input0])   # step-0 last-position logits [1, vocab]
        tok = torch.zeros((1, 1), dtype=torch.int32, device=dev)
        nxt = torch.empty(1, dtype=torch.int32, device=dev)
        host = torch.empty(1, dtype=torch.int32, pin_memory=True)
        done = torch.cuda.Event()
        out = []
        for i in range(max_len):
            smp.sample(logits, ignore_eos=i < min_len, out=tok.view(-1))
            host.copy_(tok.view(-1), non_blocking=True)
            done.record()
            if i + 1 < max_len:  # the next step, enqueued before the host looks at the token
                lm.step(ids=tok, graph=graph, out=(logits, nxt, None))
            done.synchronize()
            t = int(host[0])
            if v.stop_begin <= t < v.stop_end:
                break
            out.append(t)
        torch.cuda.current_stream(dev).synchronize()
        return out


__all__ = ["CosyVoiceLm", "CvVariant", "COSYVOICE2", "COSYVOICE3"]
