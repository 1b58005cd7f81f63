"""syrinx_amd -- MI355X (gfx950) quantized-linear hot path of syrinx.

The product is the C-ABI library ``libsxq.so`` (include/sxq.h) built from
``syrinx_amd/csrc``.  This package is its host-side mirror of candle-core's quantized
API (``GgmlDType``, ``QTensor``, ``QMatMul``) as syrinx calls it.
"""
from ._lib import SxqError, lib  # noqa: F401
from .quantized import GgmlDType, QMatMul, QTensor  # noqa: F401

__all__ = ["GgmlDType", "QTensor", "QMatMul", "SxqError", "lib"]
