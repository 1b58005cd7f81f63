"""ctypes binding of the CPU oracle (oracle/sxq_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by ``__graft_entry__.smoke()`` and by
``bench.py``'s cpu_baseline leg, to check results (or as the timed CPU baseline).  The
product package ``syrinx_amd`` never imports it.

The C file restates candle-core 0.8's quantized CPU path (third-party, absent from
the reference tree), as called from crates/syrinx-lm/src/cv2/load.rs:101-104 and
crates/syrinx-lm/src/cv2/mod.rs:195-211 of the reference.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle_sxq.so")

F32, F16, Q4_0, Q8_0, Q4K, Q8K = 0, 1, 2, 8, 12, 15
BLOCK = {Q4_0: 32, Q8_0: 32, Q4K: 256, Q8K: 256}
TYPE_SIZE = {Q4_0: 18, Q8_0: 34, Q4K: 144, Q8K: 292}
VEC_DOT = {Q4_0: Q8_0, Q8_0: Q8_0, Q4K: Q8K}

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library not built: {LIB_PATH} (run `make -C oracle`)")
        L = ctypes.CDLL(LIB_PATH)
        P, I64, I, D = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_double
        L.ora_type_size.restype = ctypes.c_size_t
        L.ora_type_size.argtypes = [I]
        L.ora_block_size.restype = ctypes.c_size_t
        L.ora_block_size.argtypes = [I]
        L.ora_f32_to_f16.restype = ctypes.c_uint16
        L.ora_f32_to_f16.argtypes = [ctypes.c_float]
        L.ora_f16_to_f32.restype = ctypes.c_float
        L.ora_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.ora_quantize_row.restype = I
        L.ora_quantize_row.argtypes = [I, P, I64, P]
        L.ora_dequantize_row.restype = I
        L.ora_dequantize_row.argtypes = [I, P, I64, P]
        L.ora_make_qkx1_quants.restype = None
        L.ora_make_qkx1_quants.argtypes = [I, I, P, I, P, P]
        L.ora_vec_dot.restype = ctypes.c_float
        L.ora_vec_dot.argtypes = [I, I64, P, P]
        L.ora_matmul.restype = I
        L.ora_matmul.argtypes = [I, I64, I64, I64, P, P, P, I]
        L.ora_dot_f64.restype = D
        L.ora_dot_f64.argtypes = [I, I64, P, P]
        L.ora_rms_norm.restype = None
        L.ora_rms_norm.argtypes = [P, P, I64, D, P]
        L.ora_rope_tables_interleaved.restype = None
        L.ora_rope_tables_interleaved.argtypes = [I64, I64, D, P, P]
        L.ora_rope_tables_half.restype = None
        L.ora_rope_tables_half.argtypes = [I64, I64, ctypes.c_float, P, P]
        L.ora_rope_interleaved.restype = None
        L.ora_rope_interleaved.argtypes = [P, I64, I64, P, P]
        L.ora_rope_half.restype = None
        L.ora_rope_half.argtypes = [P, I64, I64, P, P]
        L.ora_softmax.restype = None
        L.ora_softmax.argtypes = [P, I64]
        L.ora_silu.restype = ctypes.c_float
        L.ora_silu.argtypes = [ctypes.c_float]
        L.ora_silu_mul.restype = None
        L.ora_silu_mul.argtypes = [P, P, I64, P]
        L.ora_attend_one.restype = None
        L.ora_attend_one.argtypes = [P, P, P, I64, I64, P]
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def row_bytes(dtype: int, k: int) -> int:
    return (k // BLOCK[dtype]) * TYPE_SIZE[dtype]


def f32_to_f16_bits(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    L = lib()
    return np.array([L.ora_f32_to_f16(float(v)) for v in x], dtype=np.uint16)


def f16_bits_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16).ravel()
    L = lib()
    return np.array([L.ora_f16_to_f32(int(v)) for v in h], dtype=np.float32)


def quantize(dtype: int, x: np.ndarray) -> np.ndarray:
    """T::from_float row by row: f32 [rows, k] -> uint8 [rows, row_bytes]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.ndim == 1:
        x = x[None, :]
    rows, k = x.shape
    out = np.zeros((rows, row_bytes(dtype, k)), dtype=np.uint8)
    L = lib()
    for r in range(rows):
        rc = L.ora_quantize_row(dtype, _p(x[r]), k, _p(out[r]))
        if rc != 0:
            raise ValueError(f"quantize: k={k} not a multiple of the block size")
    return out


def dequantize(dtype: int, blocks: np.ndarray, k: int) -> np.ndarray:
    """T::to_float row by row: uint8 [rows, row_bytes] -> f32 [rows, k]."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    if blocks.ndim == 1:
        blocks = blocks[None, :]
    rows = blocks.shape[0]
    out = np.zeros((rows, k), dtype=np.float32)
    L = lib()
    for r in range(rows):
        if L.ora_dequantize_row(dtype, _p(blocks[r]), k, _p(out[r])) != 0:
            raise ValueError("dequantize: bad k")
    return out


def vec_dot(dtype: int, k: int, w_row: np.ndarray, act_row: np.ndarray) -> float:
    w_row = np.ascontiguousarray(w_row, dtype=np.uint8)
    act_row = np.ascontiguousarray(act_row, dtype=np.uint8)
    return float(lib().ora_vec_dot(dtype, k, _p(w_row), _p(act_row)))


def matmul(dtype: int, x: np.ndarray, w_blocks: np.ndarray, threads: int = 0) -> np.ndarray:
    """k_quants::matmul: x f32 [m, k] times W (blocks [n, row_bytes]) transposed -> [m, n]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.ndim == 1:
        x = x[None, :]
    m, k = x.shape
    w_blocks = np.ascontiguousarray(w_blocks, dtype=np.uint8)
    n = w_blocks.shape[0]
    assert w_blocks.shape[1] == row_bytes(dtype, k)
    y = np.zeros((m, n), dtype=np.float32)
    if lib().ora_matmul(dtype, m, k, n, _p(x), _p(w_blocks), _p(y), threads) != 0:
        raise ValueError("matmul: bad dtype or k")
    return y


def quant_margin(vdt: int, x: np.ndarray) -> float:
    """How close activation quantization of x comes to a decision boundary.

    Returns the smallest distance (in quantization steps) of any scaled value
    |x * iscale| from a rounding tie (k + 0.5), and, for Q8_K, of the two largest
    magnitudes of a block from each other (which one is "max" sets the sign of the
    scale).  Two f32 inputs that differ by a relative 1e-6 can only quantize
    differently where this margin is below ~1e-4."""
    x = np.asarray(x, np.float32).reshape(-1)
    bs = BLOCK[vdt]
    b = x.reshape(-1, bs)
    a = np.abs(b)
    if vdt == Q8K:
        idx = a.argmax(axis=1)
        mx = b[np.arange(len(b)), idx]
        ok = a.max(axis=1) > 0
        if not ok.any():
            return 1.0
        iscale = (np.float32(-128.0) / mx[ok]).astype(np.float32)
        v = (iscale[:, None] * b[ok]).astype(np.float32)
        top2 = np.sort(a[ok], axis=1)[:, -2:]
        tie = float((128.0 * (top2[:, 1] - top2[:, 0]) / top2[:, 1]).min())
    else:
        amax = a.max(axis=1)
        d = (amax / np.float32(127.0)).astype(np.float32)
        ok = d != 0
        if not ok.any():
            return 1.0
        inv = (np.float32(1.0) / d[ok]).astype(np.float32)
        v = (b[ok] * inv[:, None]).astype(np.float32)
        tie = 1.0
    av = np.abs(v.astype(np.float64))
    frac = av - np.floor(av)
    return float(min(np.abs(frac - 0.5).min(), tie))


def dot_f64(dtype: int, w_row: np.ndarray, x: np.ndarray) -> float:
    w_row = np.ascontiguousarray(w_row, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    return float(lib().ora_dot_f64(dtype, x.shape[-1], _p(w_row), _p(x)))


def make_qkx1_quants(nmax: int, ntry: int, x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32)
    s = np.zeros(1, np.float32)
    m = np.zeros(1, np.float32)
    lib().ora_make_qkx1_quants(nmax, ntry, _p(x), x.size, _p(s), _p(m))
    return float(s[0]), float(m[0])


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    y = np.empty_like(x)
    lib().ora_rms_norm(_p(x), _p(w), x.size, eps, _p(y))
    return y


def rope_tables_interleaved(seq_len: int, head_dim: int, base: float):
    c = np.zeros((seq_len, head_dim // 2), np.float32)
    s = np.zeros_like(c)
    lib().ora_rope_tables_interleaved(seq_len, head_dim, base, _p(c), _p(s))
    return c, s


def rope_tables_half(seq_len: int, head_dim: int, theta: float):
    c = np.zeros((seq_len, head_dim // 2), np.float32)
    s = np.zeros_like(c)
    lib().ora_rope_tables_half(seq_len, head_dim, theta, _p(c), _p(s))
    return c, s


def rope_interleaved(x: np.ndarray, cos_row: np.ndarray, sin_row: np.ndarray) -> np.ndarray:
    x = np.array(x, dtype=np.float32, order="C", copy=True)
    n_heads, hd = x.shape
    lib().ora_rope_interleaved(_p(x), n_heads, hd, _p(np.ascontiguousarray(cos_row, np.float32)),
                               _p(np.ascontiguousarray(sin_row, np.float32)))
    return x


def rope_half(x: np.ndarray, cos_row: np.ndarray, sin_row: np.ndarray) -> np.ndarray:
    x = np.array(x, dtype=np.float32, order="C", copy=True)
    n_heads, hd = x.shape
    lib().ora_rope_half(_p(x), n_heads, hd, _p(np.ascontiguousarray(cos_row, np.float32)),
                        _p(np.ascontiguousarray(sin_row, np.float32)))
    return x


def softmax(x: np.ndarray) -> np.ndarray:
    x = np.array(x, dtype=np.float32, order="C", copy=True)
    lib().ora_softmax(_p(x), x.size)
    return x


def silu(x: np.ndarray) -> np.ndarray:
    L = lib()
    x = np.asarray(x, dtype=np.float32)
    return np.array([L.ora_silu(float(v)) for v in x.ravel()], np.float32).reshape(x.shape)


def silu_mul(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    out = np.empty_like(g)
    lib().ora_silu_mul(_p(g), _p(u), g.size, _p(out))
    return out


def attend_one(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray) -> np.ndarray:
    q = np.ascontiguousarray(q, np.float32)
    k_cache = np.ascontiguousarray(k_cache, np.float32)
    v_cache = np.ascontiguousarray(v_cache, np.float32)
    L, hd = k_cache.shape
    out = np.zeros(hd, np.float32)
    lib().ora_attend_one(_p(q), _p(k_cache), _p(v_cache), L, hd, _p(out))
    return out
