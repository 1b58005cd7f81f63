"""Host mirror of candle-core 0.8's quantized API over libsxq (device tensors via torch).

Names, argument meaning and error text follow what the reference calls:

* ``QTensor.quantize(t, GgmlDType.X)``  -- crates/syrinx-lm/src/cv2/load.rs:102
* ``QTensor.storage_size_in_bytes()``   -- crates/syrinx-lm/src/cv2/load.rs:103
* ``QMatMul.from_qtensor(qt)``           -- crates/syrinx-lm/src/cv2/load.rs:104
* ``QMatMul.forward(xs)`` (Module)       -- crates/syrinx-lm/src/cv2/mod.rs:197
* ``QTensor.dequantize(device)``         -- crates/syrinx-vocoder/src/cv2/mod.rs:172
* ``GgmlDType.block_size()``             -- crates/syrinx-lm/src/cv2/load.rs:101

Quantized weights (Q4_0, Q8_0, Q4K) run on the hand-written gfx950 kernels; there is
no CPU fallback.  As in Candle, an F32/F16 QTensor, or the environment switches
``CANDLE_DEQUANTIZE_ALL`` / ``CANDLE_DEQUANTIZE_ALL_F16``, make ``from_qtensor``
hold a dense weight instead (``QMatMul::Tensor`` / ``QMatMul::TensorF16``).
"""
from __future__ import annotations

import ctypes
import enum
import os
from typing import Sequence

import torch

from ._lib import BF16_INPUT, BIT_EXACT, HOST_PTRS, SxqError, check, lib


class GgmlDType(enum.IntEnum):
    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q8_0 = 8
    Q4K = 12
    Q8K = 15

    def block_size(self) -> int:
        return int(lib().sxq_block_size(int(self)))

    def type_size(self) -> int:
        return int(lib().sxq_type_size(int(self)))

    def vec_dot_type(self) -> "GgmlDType":
        return {GgmlDType.Q4_0: GgmlDType.Q8_0, GgmlDType.Q8_0: GgmlDType.Q8_0,
                GgmlDType.Q4K: GgmlDType.Q8K}[self]


QUANTIZED = (GgmlDType.Q4_0, GgmlDType.Q8_0, GgmlDType.Q4K, GgmlDType.Q8K)


def _stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _dev_index(device: torch.device) -> int:
    return device.index if device.index is not None else torch.cuda.current_device()


def _ptr(t: torch.Tensor):
    return ctypes.c_void_p(t.data_ptr())


def _env_on(name: str) -> bool:
    return os.environ.get(name, "") not in ("", "0", "false", "False")


class QTensor:
    """GGML block storage of a tensor: canonical block bytes on a GPU (or f32/f16 dense)."""

    def __init__(self, data: torch.Tensor, shape: Sequence[int], dtype: GgmlDType):
        self._data = data
        self._shape = tuple(int(s) for s in shape)
        self._dtype = GgmlDType(dtype)

    # -- construction ---------------------------------------------------------------
    @staticmethod
    def quantize(src: torch.Tensor, dtype: GgmlDType, device=None) -> "QTensor":
        """QTensor::quantize: checks the block alignment of the last dim, runs from_float."""
        dtype = GgmlDType(dtype)
        shape = tuple(src.shape)
        if len(shape) == 0:
            raise SxqError(1, f"scalar tensor cannot be quantized {list(shape)}")
        bs = dtype.block_size()
        if shape[-1] % bs != 0:
            raise SxqError(3, f"quantized tensor must have their last dim divisible by block size {list(shape)} {bs}")
        dev = torch.device(device) if device is not None else (src.device if src.is_cuda else torch.device("cuda"))
        x = src.detach().to(device=dev, dtype=torch.float32).contiguous()
        if dtype == GgmlDType.F32:
            return QTensor(x, shape, dtype)
        if dtype == GgmlDType.F16:
            return QTensor(x.to(torch.float16), shape, dtype)
        k = shape[-1]
        rows = x.numel() // k if k else 0
        out = torch.empty(rows * (k // bs) * dtype.type_size(), dtype=torch.uint8, device=dev)
        check(lib().sxq_quantize_rows(_dev_index(dev), int(dtype), _ptr(x), rows, k, _ptr(out), _stream_ptr(dev)))
        return QTensor(out, shape, dtype)

    @staticmethod
    def from_blocks(blocks, shape: Sequence[int], dtype: GgmlDType, device="cuda") -> "QTensor":
        """Wrap canonical GGML block bytes (numpy / bytes / torch uint8) as a QTensor."""
        dtype = GgmlDType(dtype)
        if isinstance(blocks, (bytes, bytearray)):
            blocks = torch.frombuffer(bytearray(blocks), dtype=torch.uint8)
        elif not isinstance(blocks, torch.Tensor):
            blocks = torch.from_numpy(blocks.reshape(-1).view("uint8").copy())
        data = blocks.reshape(-1).to(device=device, dtype=torch.uint8).contiguous()
        shape = tuple(int(s) for s in shape)
        numel = 1
        for s in shape:
            numel *= s
        want = numel // dtype.block_size() * dtype.type_size()
        if shape[-1] % dtype.block_size() or data.numel() != want:
            raise SxqError(4, f"{data.numel()} bytes do not hold a {list(shape)} {dtype.name} tensor ({want})")
        return QTensor(data, shape, dtype)

    # -- accessors ------------------------------------------------------------------
    def dtype(self) -> GgmlDType:
        return self._dtype

    @property
    def shape(self):
        return self._shape

    def device(self) -> torch.device:
        return self._data.device

    def data(self) -> torch.Tensor:
        """The canonical block bytes (uint8, device)."""
        return self._data

    def storage_size_in_bytes(self) -> int:
        return self._data.numel() * self._data.element_size()

    def dequantize(self, device=None) -> torch.Tensor:
        """QTensor::dequantize: f32 tensor of the original shape (Candle's to_float)."""
        if self._dtype in (GgmlDType.F32, GgmlDType.F16):
            out = self._data.to(torch.float32).reshape(self._shape)
        else:
            dev = self._data.device
            k = self._shape[-1]
            rows = self.numel() // k
            out = torch.empty(self._shape, dtype=torch.float32, device=dev)
            check(lib().sxq_dequantize_rows(_dev_index(dev), int(self._dtype), _ptr(self._data), rows, k, _ptr(out),
                                            _stream_ptr(dev)))
        return out if device is None else out.to(device)

    def numel(self) -> int:
        n = 1
        for s in self._shape:
            n *= s
        return n


class QMatMul:
    """candle_core::quantized::QMatMul: ``forward(xs) = xs @ W^T`` for a [n, k] weight."""

    def __init__(self):
        self._h = None
        self._dense = None
        self._dense_f16 = False
        self._shape = None
        self._dtype = None
        self._device = None

    @staticmethod
    def from_qtensor(qt: QTensor) -> "QMatMul":
        if len(qt.shape) != 2:
            raise SxqError(4, f"QMatMul expects a 2-D weight, got {list(qt.shape)}")
        m = QMatMul()
        m._shape = qt.shape
        m._dtype = qt.dtype()
        m._device = qt.device()
        dense = qt.dtype() in (GgmlDType.F32, GgmlDType.F16) or _env_on("CANDLE_DEQUANTIZE_ALL")
        if dense:
            m._dense = qt.dequantize()
        elif _env_on("CANDLE_DEQUANTIZE_ALL_F16"):
            m._dense = qt.dequantize().to(torch.float16)
            m._dense_f16 = True
        else:
            if qt.dtype() == GgmlDType.Q8K:
                raise SxqError(2, "Q8K is an activation format; QMatMul weights are Q4_0, Q8_0 or Q4K")
            h = ctypes.c_void_p()
            n, k = qt.shape
            data = qt.data()
            torch.cuda.current_stream(data.device).synchronize()
            check(lib().sxq_qmm_create(_dev_index(data.device), int(qt.dtype()), n, k, _ptr(data), data.numel(), 1,
                                       ctypes.byref(h)))
            m._h = h
        return m

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            try:
                lib().sxq_qmm_destroy(h)
            except Exception:
                pass
            self._h = None

    @property
    def shape(self):
        return self._shape

    def dtype(self) -> GgmlDType:
        return self._dtype

    def storage_size_in_bytes(self) -> int:
        if self._h is None:
            return self._dense.numel() * self._dense.element_size()
        sz = ctypes.c_size_t()
        check(lib().sxq_qmm_info(self._h, None, None, None, ctypes.byref(sz)))
        return int(sz.value)

    def handle(self) -> int:
        """The sxq_qmm* pointer (for callers that drive the C-ABI directly)."""
        return self._h.value if self._h is not None else 0

    def forward(self, xs: torch.Tensor, bias: torch.Tensor = None, exact: bool = False) -> torch.Tensor:
        """Module::forward.  f32, contiguous, last dim == k, rank >= 2 (Candle's checks);
        bf16 input (the Fish GPU path's activations) is also taken and widened to f32
        exactly on the device (SXQ_BF16_INPUT).  The output is f32.

        Outputs equal Candle's CPU vec-dot bit for bit, except that a Q4_K weight applied
        to 64 or more rows runs the f16 MFMA prefill GEMM (error below
        2^-10 * sum |w x| per output); exact=True keeps the bit-identical path there too."""
        n, k = self._shape
        if self._dense is not None:
            w = self._dense
            if self._dense_f16:
                y = (xs.to(torch.float16) @ w.t()).to(xs.dtype)
            else:
                y = xs.to(w.dtype) @ w.t()
            return y if bias is None else y + bias
        if xs.dtype not in (torch.float32, torch.bfloat16):
            raise SxqError(2, f"unsupported dtype {xs.dtype} for op qmatmul (f32 or bf16)")
        if not xs.is_cuda:
            raise SxqError(6, "QMatMul input must be on the GPU holding the weight")
        shape = (ctypes.c_int64 * xs.dim())(*xs.shape)
        strides = (ctypes.c_int64 * xs.dim())(*xs.stride())
        out_shape = tuple(xs.shape[:-1]) + (n,)
        y = torch.empty(out_shape, dtype=torch.float32, device=xs.device)
        if bias is not None:
            bias = bias.to(device=xs.device, dtype=torch.float32).contiguous()
            if bias.numel() != n:
                raise SxqError(4, f"bias of {bias.numel()} elements for {n} outputs")
        flags = (BIT_EXACT if exact else 0) | (BF16_INPUT if xs.dtype == torch.bfloat16 else 0)
        bptr = _ptr(bias) if bias is not None else None
        if torch.cuda.is_current_stream_capturing():
            # Under graph capture the forward takes a workspace of its own from torch's
            # graph memory pool: replays never share the library's eager workspace with
            # other calls.  The workspace lives as long as the captured output y (as a
            # graph's own intermediates do), so a caller that re-captures and drops the old
            # outputs releases the old workspaces with them.
            need = ctypes.c_size_t()
            check(lib().sxq_qmm_workspace_size(self._h, xs.numel() // k, flags, ctypes.byref(need)))
            ws = torch.empty(max(int(need.value), 1), dtype=torch.uint8, device=xs.device)
            check(lib().sxq_qmm_forward_ws(self._h, _ptr(xs), shape, xs.dim(), strides, _ptr(y), bptr, flags,
                                           _ptr(ws), ws.numel(), _stream_ptr(xs.device)))
            y._sxq_graph_workspace = ws
        else:
            check(lib().sxq_qmm_forward(self._h, _ptr(xs), shape, xs.dim(), strides, _ptr(y), bptr, flags,
                                        _stream_ptr(xs.device)))
        return y

    __call__ = forward

    def dequantize(self) -> torch.Tensor:
        if self._dense is not None:
            return self._dense.to(torch.float32)
        n, k = self._shape
        out = torch.empty((n, k), dtype=torch.float32, device=self._device)
        check(lib().sxq_qmm_dequantize(self._h, _ptr(out), _stream_ptr(self._device)))
        return out

    def export_blocks(self) -> torch.Tensor:
        """The weight as canonical GGML block bytes (uint8, device)."""
        out = torch.empty(self.storage_size_in_bytes(), dtype=torch.uint8, device=self._device)
        check(lib().sxq_qmm_export(self._h, _ptr(out), _stream_ptr(self._device)))
        return out


def qmatmul_host(qmm: QMatMul, x_np, bias_np=None, exact: bool = False):
    """forward() with host (numpy) buffers through SXQ_HOST_PTRS: the FFI path a Rust
    caller without device tensors would use."""
    import numpy as np

    x = np.ascontiguousarray(x_np, dtype=np.float32)
    n, k = qmm.shape
    y = np.empty(x.shape[:-1] + (n,), np.float32)
    shape = (ctypes.c_int64 * x.ndim)(*x.shape)
    b = None
    if bias_np is not None:
        bias_np = np.ascontiguousarray(bias_np, dtype=np.float32)
        b = bias_np.ctypes.data_as(ctypes.c_void_p)
    check(lib().sxq_qmm_forward(qmm._h, x.ctypes.data_as(ctypes.c_void_p), shape, x.ndim, None,
                                y.ctypes.data_as(ctypes.c_void_p), b, HOST_PTRS | (BIT_EXACT if exact else 0), None))
    return y
