"""GGUF files: the quantized on-disk format for this path's weights.

A reader and a writer with candle-core 0.8's ``quantized::gguf_file`` interface
(``Content::read``, ``Content::tensor``, ``gguf_file::write``), which Candle's quantized
models load their QTensors through.  The block bytes a GGUF file holds are the GGML
blocks ``QTensor`` carries (Q4_0, Q8_0, Q4_K, ...), so a tensor read from a file is
wrapped as a QTensor without conversion and becomes a ``QMatMul`` like one made by
``QTensor.quantize``; the writer stores QTensors (quantized on the GPU by Candle's
``from_float``) so a checkpoint can be quantized once and loaded many times.

Layout (GGUF v3; v1 and v2 are read too -- v1 has 32-bit counts and lengths):
    u32 magic "GGUF" | u32 version | u64 n_tensors | u64 n_kv
    n_kv x (string key, u32 value type, value)
    n_tensors x (string name, u32 n_dims, u64 dims[n_dims] innermost first, u32 ggml type,
                 u64 offset into the data section)
    zero padding to `general.alignment` (default 32), then the data section, every
    tensor at its offset (a multiple of the alignment).
Strings are a u64 byte count and UTF-8 bytes; arrays a u32 element type, a u64 count and
the elements; everything little-endian.  A tensor's dims are its shape reversed (a
[N, K] weight is stored with dims (K, N)), as Candle reads and writes them.

Reference: the reference builds its QTensors by quantizing at load
(crates/syrinx-lm/src/cv2/load.rs:101-104; crates/syrinx-fish/src/s2/load.rs:32-51);
these files hold exactly those QTensors.
"""
from __future__ import annotations

import enum
import os
import struct
from dataclasses import dataclass
from typing import BinaryIO, Iterable, Sequence

import numpy as np
import torch

from ._lib import SxqError
from .quantized import GgmlDType, QTensor

GGUF_MAGIC = 0x46554747  # b"GGUF" read as a little-endian u32
DEFAULT_ALIGNMENT = 32

# (block size, bytes per block) of every GGML tensor type, for the byte extent of a
# tensor; the ones QTensor can hold are GgmlDType's.
GGML_TYPE_SIZES = {
    0: (1, 4),       # F32
    1: (1, 2),       # F16
    2: (32, 18),     # Q4_0
    3: (32, 20),     # Q4_1
    6: (32, 22),     # Q5_0
    7: (32, 24),     # Q5_1
    8: (32, 34),     # Q8_0
    9: (32, 36),     # Q8_1
    10: (256, 84),   # Q2_K
    11: (256, 110),  # Q3_K
    12: (256, 144),  # Q4_K
    13: (256, 176),  # Q5_K
    14: (256, 210),  # Q6_K
    15: (256, 292),  # Q8_K
    24: (1, 1),      # I8
    25: (1, 2),      # I16
    26: (1, 4),      # I32
    27: (1, 8),      # I64
    28: (1, 8),      # F64
    30: (1, 2),      # BF16
}


class ValueType(enum.IntEnum):
    U8 = 0
    I8 = 1
    U16 = 2
    I16 = 3
    U32 = 4
    I32 = 5
    F32 = 6
    BOOL = 7
    STRING = 8
    ARRAY = 9
    U64 = 10
    I64 = 11
    F64 = 12


_SCALAR = {ValueType.U8: "<B", ValueType.I8: "<b", ValueType.U16: "<H", ValueType.I16: "<h",
           ValueType.U32: "<I", ValueType.I32: "<i", ValueType.F32: "<f", ValueType.BOOL: "<?",
           ValueType.U64: "<Q", ValueType.I64: "<q", ValueType.F64: "<d"}


@dataclass(frozen=True)
class Value:
    """A typed metadata value (Candle's gguf_file::Value): `kind`, and `value` -- a Python
    scalar, a str, or for ARRAY a tuple (element kind, tuple of element values)."""
    kind: ValueType
    value: object

    @staticmethod
    def of(v) -> "Value":
        """A Value from a Python value: str -> STRING, bool -> BOOL, int -> U32 when it fits
        (else I64), float -> F32, list/tuple -> ARRAY of the first element's kind."""
        if isinstance(v, Value):
            return v
        if isinstance(v, str):
            return Value(ValueType.STRING, v)
        if isinstance(v, bool):
            return Value(ValueType.BOOL, v)
        if isinstance(v, int):
            return Value(ValueType.U32 if 0 <= v < 2 ** 32 else ValueType.I64, v)
        if isinstance(v, float):
            return Value(ValueType.F32, v)
        if isinstance(v, (list, tuple)):
            items = [Value.of(x) for x in v]
            kind = items[0].kind if items else ValueType.U32
            if any(x.kind != kind for x in items):
                raise SxqError(1, "gguf: array elements of different types")
            return Value(ValueType.ARRAY, (kind, tuple(x.value for x in items)))
        raise SxqError(1, f"gguf: no metadata type for {type(v).__name__}")

    def to_u32(self) -> int:
        if self.kind != ValueType.U32:
            raise SxqError(1, f"gguf: not a u32 {self.kind.name}")
        return int(self.value)

    def to_string(self) -> str:
        if self.kind != ValueType.STRING:
            raise SxqError(1, f"gguf: not a string {self.kind.name}")
        return str(self.value)


@dataclass(frozen=True)
class TensorInfo:
    """Candle's gguf_file::TensorInfo: type, shape (outermost first), data-section offset."""
    ggml_dtype: int
    shape: tuple
    offset: int

    def nbytes(self) -> int:
        bs, ts = GGML_TYPE_SIZES[self.ggml_dtype]
        n = 1
        for s in self.shape:
            n *= s
        return n // bs * ts


class _Reader:
    def __init__(self, buf, pos: int = 0, wide: bool = True):
        self.buf, self.pos, self.wide = buf, pos, wide

    def take(self, n: int) -> bytes:
        if self.pos + n > len(self.buf):
            raise SxqError(1, f"gguf: truncated file (need {n} bytes at {self.pos}, have {len(self.buf) - self.pos})")
        b = bytes(self.buf[self.pos:self.pos + n])
        self.pos += n
        return b

    def scalar(self, fmt: str):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def count(self) -> int:  # u64 from v2 on, u32 in v1
        return self.scalar("<Q" if self.wide else "<I")

    def string(self) -> str:
        return self.take(self.count()).decode("utf-8")

    def value(self, kind: ValueType):
        if kind == ValueType.STRING:
            return self.string()
        if kind == ValueType.ARRAY:
            ek = ValueType(self.scalar("<I"))
            n = self.count()
            return ek, tuple(self.value(ek) for _ in range(n))
        if kind not in _SCALAR:
            raise SxqError(1, f"gguf: unknown value type {int(kind)}")
        v = self.scalar(_SCALAR[kind])
        if kind == ValueType.BOOL and not isinstance(v, bool):
            v = bool(v)
        return v


class Content:
    """A parsed GGUF file (Candle's gguf_file::Content): metadata, tensor infos, and the
    start of the data section; tensors are read from the file on demand."""

    def __init__(self, version: int, metadata: dict, tensor_infos: dict, tensor_data_offset: int, path: str = None,
                 buf=None):
        self.version = version
        self.metadata = metadata
        self.tensor_infos = tensor_infos
        self.tensor_data_offset = tensor_data_offset
        self._path = path
        self._buf = buf

    @staticmethod
    def read(src) -> "Content":
        """Parse a file path, bytes, or a binary file object (read whole)."""
        path = None
        if isinstance(src, (str, os.PathLike)):
            path = os.fspath(src)
            buf = np.memmap(path, dtype=np.uint8, mode="r")
        elif isinstance(src, (bytes, bytearray, memoryview)):
            buf = np.frombuffer(bytes(src), dtype=np.uint8)
        else:
            buf = np.frombuffer(src.read(), dtype=np.uint8)
        r = _Reader(buf)
        magic = r.scalar("<I")
        if magic != GGUF_MAGIC:
            raise SxqError(1, f"gguf: unknown magic 0x{magic:08x}")
        version = r.scalar("<I")
        if version not in (1, 2, 3):
            raise SxqError(1, f"gguf: unsupported version {version}")
        r.wide = version >= 2
        n_tensors = r.count()
        n_kv = r.count()
        metadata = {}
        for _ in range(n_kv):
            key = r.string()
            kind = ValueType(r.scalar("<I"))
            metadata[key] = Value(kind, r.value(kind))
        infos = {}
        for _ in range(n_tensors):
            name = r.string()
            nd = r.scalar("<I")
            dims = [r.count() for _ in range(nd)]
            t = r.scalar("<I")
            off = r.scalar("<Q")
            if t not in GGML_TYPE_SIZES:
                raise SxqError(2, f"gguf: tensor {name}: unknown ggml type {t}")
            infos[name] = TensorInfo(t, tuple(int(d) for d in reversed(dims)), int(off))
        align = metadata["general.alignment"].to_u32() if "general.alignment" in metadata else DEFAULT_ALIGNMENT
        if align <= 0 or align & (align - 1):
            raise SxqError(1, f"gguf: alignment {align} is not a power of two")
        data0 = (r.pos + align - 1) // align * align
        for name, ti in infos.items():
            if ti.offset % align:
                raise SxqError(1, f"gguf: tensor {name} at offset {ti.offset}, not a multiple of {align}")
            bs = GGML_TYPE_SIZES[ti.ggml_dtype][0]
            if ti.shape and ti.shape[-1] % bs:
                raise SxqError(3, f"gguf: tensor {name} {list(ti.shape)}: last dim not a multiple of {bs}")
            if data0 + ti.offset + ti.nbytes() > len(buf):
                raise SxqError(1, f"gguf: tensor {name} runs past the end of the file")
        return Content(version, metadata, infos, data0, path, buf)

    def tensor_bytes(self, name: str) -> np.ndarray:
        """The tensor's stored bytes (a read-only view of the file)."""
        if name not in self.tensor_infos:
            raise SxqError(1, f"gguf: no tensor {name}")
        ti = self.tensor_infos[name]
        a = self.tensor_data_offset + ti.offset
        return self._buf[a:a + ti.nbytes()]

    def tensor(self, name: str, device="cuda") -> QTensor:
        """Content::tensor: the tensor as a QTensor on `device` (F32, F16, Q4_0, Q8_0, Q4_K,
        Q8_K; other GGML types have no kernels here and are refused)."""
        ti = self.tensor_infos.get(name)
        if ti is None:
            raise SxqError(1, f"gguf: no tensor {name}")
        try:
            dt = GgmlDType(ti.ggml_dtype)
        except ValueError:
            raise SxqError(2, f"gguf: tensor {name}: ggml type {ti.ggml_dtype} is not supported") from None
        raw = np.array(self.tensor_bytes(name))  # one host copy, off the file mapping
        if dt in (GgmlDType.F32, GgmlDType.F16):
            t = torch.from_numpy(raw.view(np.float32 if dt == GgmlDType.F32 else np.float16).reshape(ti.shape))
            return QTensor(t.to(device), ti.shape, dt)
        return QTensor.from_blocks(raw, ti.shape, dt, device=device)

    def dense(self, name: str, device="cuda") -> torch.Tensor:
        """An F32/F16 tensor as an f32 torch tensor (norm weights, embedding tables)."""
        qt = self.tensor(name, device)
        return qt.dequantize()


def _pack_value(v: Value, out: list) -> None:
    if v.kind == ValueType.STRING:
        b = str(v.value).encode("utf-8")
        out.append(struct.pack("<Q", len(b)) + b)
    elif v.kind == ValueType.ARRAY:
        ek, items = v.value
        out.append(struct.pack("<IQ", int(ek), len(items)))
        for x in items:
            _pack_value(Value(ValueType(ek), x), out)
    else:
        out.append(struct.pack(_SCALAR[v.kind], v.value))


def _stored(t) -> tuple:
    """(ggml type, shape, bytes) of a QTensor or a float torch tensor (stored as F32)."""
    if isinstance(t, QTensor):
        dt = t.dtype()
        if dt in (GgmlDType.F32, GgmlDType.F16):
            arr = t.data().detach().to("cpu").contiguous().numpy()
            return int(dt), t.shape, arr.tobytes()
        return int(dt), t.shape, t.data().detach().to("cpu").numpy().tobytes()
    if isinstance(t, torch.Tensor):
        if t.dtype == torch.float16:
            return 1, tuple(t.shape), t.detach().to("cpu").contiguous().numpy().tobytes()
        return 0, tuple(t.shape), t.detach().to(device="cpu", dtype=torch.float32).contiguous().numpy().tobytes()
    raise SxqError(1, f"gguf: cannot store {type(t).__name__}")


def write(f: BinaryIO, metadata: Iterable[tuple], tensors: Iterable[tuple], alignment: int = DEFAULT_ALIGNMENT) -> None:
    """gguf_file::write: version 3, the metadata (key, Value or Python value) pairs and the
    (name, QTensor or float torch tensor) pairs in order, each tensor at the next
    multiple of the alignment.  A `general.alignment` entry in the metadata must match
    `alignment`."""
    metadata = [(k, Value.of(v)) for k, v in metadata]
    for k, v in metadata:
        if k == "general.alignment" and v.to_u32() != alignment:
            raise SxqError(1, f"gguf: general.alignment {v.value} but writing with {alignment}")
    if alignment != DEFAULT_ALIGNMENT and not any(k == "general.alignment" for k, _ in metadata):
        metadata.append(("general.alignment", Value(ValueType.U32, alignment)))
    stored = [(name, *_stored(t)) for name, t in tensors]
    names = [s[0] for s in stored]
    if len(set(names)) != len(names):
        raise SxqError(1, "gguf: duplicate tensor names")
    head = [struct.pack("<IIQQ", GGUF_MAGIC, 3, len(stored), len(metadata))]
    for k, v in metadata:
        kb = k.encode("utf-8")
        head.append(struct.pack("<Q", len(kb)) + kb + struct.pack("<I", int(v.kind)))
        _pack_value(v, head)
    offset = 0
    offsets = []
    for name, t, shape, data in stored:
        nb = name.encode("utf-8")
        head.append(struct.pack("<Q", len(nb)) + nb + struct.pack("<I", len(shape)))
        head.append(b"".join(struct.pack("<Q", int(d)) for d in reversed(shape)))
        head.append(struct.pack("<IQ", t, offset))
        offsets.append(offset)
        offset += (len(data) + alignment - 1) // alignment * alignment
    hb = b"".join(head)
    f.write(hb)
    f.write(b"\0" * ((-len(hb)) % alignment))
    for (_, _, _, data), off in zip(stored, offsets):
        f.write(data)
        f.write(b"\0" * ((-len(data)) % alignment))


def save(path: str, metadata: Sequence[tuple], tensors: Sequence[tuple], alignment: int = DEFAULT_ALIGNMENT) -> None:
    with open(path, "wb") as f:
        write(f, metadata, tensors, alignment)


__all__ = ["Content", "TensorInfo", "Value", "ValueType", "write", "save", "GGUF_MAGIC", "GGML_TYPE_SIZES"]
