"""Per-row quantized embedding tables (libsxq sxq_embed_*), the reference's QEmbed.

``QEmbed.quantize`` is quantize_embed (crates/syrinx-lm/src/cv2/quant.rs:38-89) and
``QEmbed.rows`` is the dequant-on-gather of Qwen2Lm::embed_rows
(crates/syrinx-lm/src/cv2/generate.rs:22-67); both run on the GPU.  int4 (two codes per
byte) is the reference's DEFAULT_EMBED_SCHEME; int8 is the fallback for odd widths.
"""
from __future__ import annotations

import ctypes

import torch

from ._lib import check, lib

INT4, INT8 = 4, 8
DEFAULT_EMBED_SCHEME = INT4


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _dev(device: torch.device) -> int:
    return device.index if device.index is not None else torch.cuda.current_device()


class QEmbed:
    """An [rows, h] table held as per-row int8 / int4 codes plus one f32 scale per row."""

    def __init__(self, q: torch.Tensor, scale: torch.Tensor, h: int, scheme: int):
        self.q, self.scale, self.h, self.scheme = q, scale, int(h), int(scheme)

    @property
    def rows_count(self) -> int:
        return int(self.scale.shape[0])

    @property
    def bytes(self) -> int:
        """Realized storage (codes + f32 scales), as QEmbed::bytes counts it."""
        return self.q.numel() + self.scale.numel() * 4

    @classmethod
    def quantize(cls, table: torch.Tensor, scheme: int = DEFAULT_EMBED_SCHEME) -> "QEmbed":
        if table.dim() != 2:
            raise ValueError(f"QEmbed.quantize: a [rows, h] table, got shape {tuple(table.shape)}")
        t = table.to(dtype=torch.float32).contiguous()
        if not t.is_cuda:
            raise ValueError("QEmbed.quantize: the table must be on the GPU")
        v, h = t.shape
        eff = ctypes.c_int()
        check(lib().sxq_embed_scheme(int(scheme), h, ctypes.byref(eff)))
        q = torch.empty((v, h // 2 if eff.value == INT4 else h), dtype=torch.uint8, device=t.device)
        scale = torch.empty(v, dtype=torch.float32, device=t.device)
        check(lib().sxq_embed_quantize(_dev(t.device), eff.value, _p(t), v, h, _p(q), _p(scale),
                                       torch.cuda.current_stream(t.device).cuda_stream))
        return cls(q, scale, h, eff.value)

    def rows(self, ids) -> torch.Tensor:
        """embed_rows: f32 [n, h] for token ids (dequantized on gather)."""
        ids = torch.as_tensor(ids, dtype=torch.int32).to(self.q.device).reshape(-1).contiguous()
        out = torch.empty((ids.numel(), self.h), dtype=torch.float32, device=self.q.device)
        check(lib().sxq_embed_gather(_dev(self.q.device), self.scheme, _p(self.q), _p(self.scale), self.rows_count,
                                     self.h, _p(ids), ids.numel(), _p(out),
                                     torch.cuda.current_stream(self.q.device).cuda_stream))
        return out
