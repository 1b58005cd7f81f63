"""CPU oracle of the per-row int8 / int4 embedding tables (test infrastructure only:
tests/ import it as the checker).

Restates on numpy:
  quantize_embed        crates/syrinx-lm/src/cv2/quant.rs:38-47 (int4 needs an even width,
                        else int8)
  quantize_embed_int8   crates/syrinx-lm/src/cv2/quant.rs:50-61
  quantize_embed_int4   crates/syrinx-lm/src/cv2/quant.rs:66-89
  embed_rows            crates/syrinx-lm/src/cv2/generate.rs:22-67 (dequant-on-gather)
The float steps are those of candle-core 0.8 (third-party, absent from the reference
tree) on f32 tensors: `t / 127.0` and `t + 1e-12` with a scalar are its affine map
t * m + a with m = (1 / 127) and a = 1e-12 each rounded to f32, evaluated as a product
and then a sum, each rounded to f32; `broadcast_div` is an f32 division; `round()` is
Rust's f32::round (halves away from zero); the dequantized element is one f32 product.
"""
from __future__ import annotations

import numpy as np

INT4, INT8 = 4, 8


def effective_scheme(scheme: int, h: int) -> int:
    return INT8 if scheme == INT4 and h % 2 else scheme


def round_half_away(x: np.ndarray) -> np.ndarray:
    """f32::round: the nearest integer, halves away from zero (numpy's round is half-even)."""
    x = np.asarray(x, np.float32)
    return (np.sign(x) * np.floor(np.abs(x).astype(np.float64) + 0.5)).astype(np.float32)


def row_scales(table: np.ndarray, qmax: int) -> np.ndarray:
    t = np.asarray(table, np.float32)
    amax = np.abs(t).max(axis=1).astype(np.float32)
    m = np.float32(1.0 / qmax)
    return (amax * m).astype(np.float32) + np.float32(1e-12)


def quantize(table: np.ndarray, scheme: int):
    """-> (codes uint8 [V, H] or [V, H/2], scale f32 [V], effective scheme)."""
    t = np.asarray(table, np.float32)
    v, h = t.shape
    scheme = effective_scheme(scheme, h)
    qmax = 127 if scheme == INT8 else 7
    s = row_scales(t, qmax)
    q = np.clip(round_half_away((t / s[:, None]).astype(np.float32)), -qmax, qmax).astype(np.int32)
    if scheme == INT8:
        return (q + 128).astype(np.uint8), s, scheme
    lo = (q[:, 0::2] + 8) & 15
    hi = (q[:, 1::2] + 8) & 15
    return (lo | (hi << 4)).astype(np.uint8), s, scheme


def gather(codes: np.ndarray, scale: np.ndarray, scheme: int, h: int, ids) -> np.ndarray:
    ids = np.asarray(ids, np.int64)
    out = np.zeros((len(ids), h), np.float32)
    for i, r in enumerate(ids):
        if not 0 <= r < len(scale):
            continue
        if scheme == INT8:
            c = codes[r].astype(np.int32) - 128
        else:
            c = np.empty(h, np.int32)
            c[0::2] = (codes[r] & 15).astype(np.int32) - 8
            c[1::2] = (codes[r] >> 4).astype(np.int32) - 8
        out[i] = c.astype(np.float32) * np.float32(scale[r])
    return out
