"""Loader for libsxq.so (the C-ABI declared in include/sxq.h).

There is no CPU fallback: if the library is missing, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsxq.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "sxq.h")

OK, ERR_INVALID, ERR_DTYPE, ERR_BLOCK_ALIGN, ERR_SHAPE, ERR_NOT_CONTIGUOUS, ERR_DEVICE, ERR_OOM = range(8)
STATUS_NAMES = {
    ERR_INVALID: "INVALID",
    ERR_DTYPE: "DTYPE",
    ERR_BLOCK_ALIGN: "BLOCK_ALIGN",
    ERR_SHAPE: "SHAPE",
    ERR_NOT_CONTIGUOUS: "NOT_CONTIGUOUS",
    ERR_DEVICE: "DEVICE",
    ERR_OOM: "OOM",
}
HOST_PTRS = 1
BIT_EXACT = 2  # SXQ_BIT_EXACT
BF16_INPUT = 4  # SXQ_BF16_INPUT
DEVICE_PTRS = 0


class SxqError(RuntimeError):
    """A failed libsxq call: `code` is the sxq_status, the message is sxq_last_error()."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[{STATUS_NAMES.get(code, code)}] {msg}")
        self.code = code
        self.msg = msg


_lib = None

_P, _I, _I64, _SZ, _U, _U64, _F = (ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t,
                                   ctypes.c_uint, ctypes.c_uint64, ctypes.c_float)
_SIGS = {
    "sxq_last_error": (ctypes.c_char_p, []),
    "sxq_version": (ctypes.c_char_p, []),
    "sxq_block_size": (_SZ, [_I]),
    "sxq_type_size": (_SZ, [_I]),
    "sxq_device_count": (_I, [_P]),
    "sxq_quantize_rows": (_I, [_I, _I, _P, _I64, _I64, _P, _P]),
    "sxq_dequantize_rows": (_I, [_I, _I, _P, _I64, _I64, _P, _P]),
    "sxq_act_quantize": (_I, [_I, _I, _P, _I64, _I64, _P, _P]),
    "sxq_qmm_create": (_I, [_I, _I, _I64, _I64, _P, _SZ, _I, _P]),
    "sxq_qmm_forward": (_I, [_P, _P, _P, _I, _P, _P, _P, _U, _P]),
    "sxq_qmm_workspace_size": (_I, [_P, _I64, _U, _P]),
    "sxq_qmm_forward_ws": (_I, [_P, _P, _P, _I, _P, _P, _P, _U, _P, _SZ, _P]),
    "sxq_qmm_forward_noalloc": (_I, [_P, _P, _P, _I, _P, _P, _P, _U, _P]),
    "sxq_qmm_info": (_I, [_P, _P, _P, _P, _P]),
    "sxq_qmm_dequantize": (_I, [_P, _P, _P]),
    "sxq_qmm_export": (_I, [_P, _P, _P]),
    "sxq_qmm_destroy": (_I, [_P]),
    "sxq_fill_normal": (_I, [_I, _P, _I64, _U64, _F, _F, _P]),
    "sxq_lm_create": (_I, [_I, _P, _P]),
    "sxq_lm_set_linear": (_I, [_P, _I, _I, _P]),
    "sxq_lm_set_vector": (_I, [_P, _I, _I, _P, _I64, _I]),
    "sxq_lm_init_random": (_I, [_P, _U64, _F]),
    "sxq_lm_kv_fill_random": (_I, [_P, _P, _I, _U64]),
    "sxq_lm_set_lengths": (_I, [_P, _P, _I]),
    "sxq_lm_get_lengths": (_I, [_P, _P, _I]),
    "sxq_lm_reset": (_I, [_P, _I, _P]),
    "sxq_lm_set_embed_quantized": (_I, [_P, _I, _P, _P]),
    "sxq_embed_scheme": (_I, [_I, _I64, _P]),
    "sxq_embed_quantize": (_I, [_I, _I, _P, _I64, _I64, _P, _P, _P]),
    "sxq_embed_gather": (_I, [_I, _I, _P, _P, _I64, _I64, _P, _I, _P, _P]),
    "sxq_lm_step": (_I, [_P, _I, _P, _P, _P, _P, _P, _U, _P]),
    "sxq_lm_read_kv": (_I, [_P, _I, _I, _I, _I, _I, _P, _P, _P]),
    "sxq_lm_prefill": (_I, [_P, _I, _P, _P, _P, _P, _P, _P, _U, _P, _SZ, _P]),
    "sxq_lm_prefill_trace_floats": (_I, [_P, _I64, _P]),
    "sxq_lm_gemv_pass": (_I, [_P, _I, _I, _P]),
    "sxq_sample_semantic": (_I, [_I, _P, _I64, _I, _I, _P, _P, _P, _P, _P, _P, _I, _P]),
    "sxq_sample_codebook": (_I, [_I, _P, _I64, _I, _I, _P, _P, _P, _I, _P, _P, _I, _P]),
    "sxq_fish_fast_expand": (_I, [_P, _I, _P, _P, _I, _P, _P, _P, _I, _P, _I, _I, _P]),
    "sxq_sample_ras": (_I, [_I, _P, _I64, _I, _I, _I, _I, _I, _F, _I, _I, _F, _P, _P, _P, _P, _I, _P]),
    "sxq_lm_read_state": (_I, [_P, _I, _I, _P, _P]),
    "sxq_lm_trace_floats": (_I, [_P, _I, _P]),
    "sxq_lm_set_trace": (_I, [_P, _P, _SZ]),
    "sxq_lm_weight_bytes": (_I, [_P, _P, _P]),
    "sxq_lm_paths": (_I, [_P, _P]),
    "sxq_lm_destroy": (_I, [_P]),
}


def lib() -> ctypes.CDLL:
    """Load libsxq.so once (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"libsxq.so is not built ({LIB_PATH}); run `python -m syrinx_amd.build`. "
                "There is no CPU fallback for the quantized path.")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(code: int) -> None:
    if code != OK:
        raise SxqError(code, lib().sxq_last_error().decode(errors="replace"))


def header_functions() -> list:
    """Names of the functions include/sxq.h declares."""
    with open(HEADER) as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sxq_[a-z0-9_]+)\s*\(", text)))
