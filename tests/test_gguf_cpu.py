"""GGUF reader / writer (syrinx_amd/gguf.py) on the CPU.

The reader is checked against files laid out byte by byte here from the published GGUF
format (v3, and v1's 32-bit counts), not through the writer: magic, version, counts, every
metadata value type, tensor infos with dims innermost first, alignment padding and
offsets.  The writer is checked by reading its files back (bytes, shapes, types, metadata)
and against the same byte layout.  Block contents come from the oracle's from_float, so a
stored tensor is exactly what QTensor.quantize would hand to QMatMul.
"""
import io
import struct

import numpy as np
import pytest
import torch

import oracle
from syrinx_amd import GgmlDType, QTensor, SxqError
from syrinx_amd import gguf as G
from syrinx_amd.ingest import is_fish_projection


def _s(text: str, wide=True) -> bytes:
    b = text.encode("utf-8")
    return struct.pack("<Q" if wide else "<I", len(b)) + b


def _kv(key, kind, payload, wide=True):
    return _s(key, wide) + struct.pack("<I", kind) + payload


def _pad(n, a=32):
    return b"\0" * ((-n) % a)


def _blocks(dt, rows, k, seed):
    x = np.random.default_rng(seed).standard_normal((rows, k)).astype(np.float32) * 0.1
    return oracle.quantize(dt, x)


def _hand_built(version=3, alignment=None):
    """A GGUF file built field by field: a Q8_0 [3, 64] weight, an F32 [5] vector, a Q4_K
    [2, 256] weight, and one metadata entry of every value type."""
    wide = version >= 2
    q8 = _blocks(oracle.Q8_0, 3, 64, 1).tobytes()
    f32 = np.arange(5, dtype=np.float32) * 0.5 - 1.0
    q4k = _blocks(oracle.Q4K, 2, 256, 2).tobytes()
    cnt = (lambda n: struct.pack("<Q", n)) if wide else (lambda n: struct.pack("<I", n))
    kvs = [
        _kv("a.u8", 0, struct.pack("<B", 200), wide), _kv("a.i8", 1, struct.pack("<b", -7), wide),
        _kv("a.u16", 2, struct.pack("<H", 65000), wide), _kv("a.i16", 3, struct.pack("<h", -30000), wide),
        _kv("a.u32", 4, struct.pack("<I", 4000000000), wide), _kv("a.i32", 5, struct.pack("<i", -2000000000), wide),
        _kv("a.f32", 6, struct.pack("<f", 0.25), wide), _kv("a.bool", 7, struct.pack("<B", 1), wide),
        _kv("a.str", 8, _s("héllo", wide), wide),
        _kv("a.arr", 9, struct.pack("<I", 4) + cnt(3) + struct.pack("<III", 1, 2, 3), wide),
        _kv("a.strs", 9, struct.pack("<I", 8) + cnt(2) + _s("x", wide) + _s("yz", wide), wide),
        _kv("a.u64", 10, struct.pack("<Q", 2 ** 40), wide), _kv("a.i64", 11, struct.pack("<q", -(2 ** 40)), wide),
        _kv("a.f64", 12, struct.pack("<d", 1.0 / 3.0), wide),
    ]
    a = alignment or 32
    if alignment:
        kvs.append(_kv("general.alignment", 4, struct.pack("<I", alignment), wide))
    tensors = [("blk.0.w", 8, (64, 3), q8), ("blk.0.norm", 0, (5,), f32.tobytes()), ("blk.0.k", 12, (256, 2), q4k)]
    infos, data, off = [], b"", 0
    for name, t, dims, raw in tensors:
        infos.append(_s(name, wide) + struct.pack("<I", len(dims)) + b"".join(cnt(d) for d in dims) +
                     struct.pack("<IQ", t, off))
        data += raw + _pad(len(raw), a)
        off = len(data)
    head = struct.pack("<II", 0x46554747, version) + cnt(len(tensors)) + cnt(len(kvs)) + b"".join(kvs) + b"".join(infos)
    return head + _pad(len(head), a) + data, (q8, f32, q4k)


@pytest.mark.parametrize("version", [1, 2, 3])
def test_reads_a_hand_built_file(version):
    buf, (q8, f32, q4k) = _hand_built(version)
    c = G.Content.read(buf)
    assert c.version == version
    md = c.metadata
    assert (md["a.u8"].kind, md["a.u8"].value) == (G.ValueType.U8, 200)
    assert md["a.i8"].value == -7 and md["a.u16"].value == 65000 and md["a.i16"].value == -30000
    assert md["a.u32"].to_u32() == 4000000000 and md["a.i32"].value == -2000000000
    assert md["a.f32"].value == 0.25 and md["a.bool"].value is True and md["a.str"].to_string() == "héllo"
    assert md["a.arr"].value == (G.ValueType.U32, (1, 2, 3))
    assert md["a.strs"].value == (G.ValueType.STRING, ("x", "yz"))
    assert md["a.u64"].value == 2 ** 40 and md["a.i64"].value == -(2 ** 40) and md["a.f64"].value == 1.0 / 3.0
    ti = c.tensor_infos
    assert list(ti) == ["blk.0.w", "blk.0.norm", "blk.0.k"]
    assert (ti["blk.0.w"].ggml_dtype, ti["blk.0.w"].shape) == (8, (3, 64))  # dims reversed into the shape
    assert (ti["blk.0.norm"].ggml_dtype, ti["blk.0.norm"].shape) == (0, (5,))
    assert (ti["blk.0.k"].ggml_dtype, ti["blk.0.k"].shape) == (12, (2, 256))
    assert c.tensor_data_offset % 32 == 0
    assert bytes(c.tensor_bytes("blk.0.w")) == q8 and bytes(c.tensor_bytes("blk.0.k")) == q4k
    qt = c.tensor("blk.0.w", device="cpu")
    assert qt.dtype() == GgmlDType.Q8_0 and qt.shape == (3, 64) and qt.storage_size_in_bytes() == 3 * 2 * 34
    assert bytes(qt.data().numpy()) == q8
    v = c.dense("blk.0.norm", device="cpu")
    assert v.dtype == torch.float32 and np.array_equal(v.numpy(), f32)


def test_alignment_from_metadata():
    buf, (q8, _, q4k) = _hand_built(alignment=128)
    c = G.Content.read(buf)
    assert c.tensor_data_offset % 128 == 0
    assert c.tensor_infos["blk.0.norm"].offset == 256  # the 204-byte Q8_0 tensor padded to two 128-byte units
    assert bytes(c.tensor_bytes("blk.0.k")) == q4k


def test_write_read_round_trip(tmp_path):
    q4k = _blocks(oracle.Q4K, 4, 512, 3)
    q80 = _blocks(oracle.Q8_0, 5, 96, 4)
    q40 = _blocks(oracle.Q4_0, 2, 64, 5)
    vec = torch.linspace(-1, 1, 7)
    tensors = [("w.q4k", QTensor.from_blocks(q4k, (4, 512), GgmlDType.Q4K, device="cpu")),
               ("w.q8_0", QTensor.from_blocks(q80, (5, 96), GgmlDType.Q8_0, device="cpu")),
               ("w.q4_0", QTensor.from_blocks(q40, (2, 64), GgmlDType.Q4_0, device="cpu")),
               ("v", vec), ("h", vec.to(torch.float16))]
    meta = [("general.architecture", "fish-s2"), ("n", 36), ("eps", 1e-6), ("flag", False),
            ("ids", [3, 1, 4]), ("neg", -5), ("big", 2 ** 40)]
    path = tmp_path / "m.gguf"
    G.save(str(path), meta, tensors)
    c = G.Content.read(str(path))
    assert c.version == 3
    assert c.metadata["general.architecture"].to_string() == "fish-s2" and c.metadata["n"].to_u32() == 36
    assert c.metadata["eps"].kind == G.ValueType.F32 and c.metadata["flag"].value is False
    assert c.metadata["ids"].value == (G.ValueType.U32, (3, 1, 4))
    assert c.metadata["neg"].kind == G.ValueType.I64 and c.metadata["neg"].value == -5
    assert c.metadata["big"].value == 2 ** 40
    for name, raw, shape, dt in (("w.q4k", q4k, (4, 512), 12), ("w.q8_0", q80, (5, 96), 8), ("w.q4_0", q40, (2, 64), 2)):
        assert (c.tensor_infos[name].ggml_dtype, c.tensor_infos[name].shape) == (dt, shape)
        assert bytes(c.tensor_bytes(name)) == raw.tobytes()
    assert np.array_equal(c.dense("v", device="cpu").numpy(), vec.numpy())
    assert c.tensor_infos["h"].ggml_dtype == 1
    assert np.array_equal(c.dense("h", device="cpu").numpy(), vec.to(torch.float16).float().numpy())
    # the writer's layout is the format's: every offset aligned, data packed in order
    offs = [c.tensor_infos[n].offset for n, _ in tensors]
    assert offs == sorted(offs) and all(o % 32 == 0 for o in offs)
    size = c.tensor_data_offset + offs[-1] + c.tensor_infos["h"].nbytes()
    assert path.stat().st_size == size + (-size) % 32


def test_writer_bytes_match_the_layout():
    """The writer's bytes equal the field-by-field layout of the same content."""
    buf, (q8, f32, q4k) = _hand_built(version=3)
    c = G.Content.read(buf)
    f = io.BytesIO()
    G.write(f, [(k, v) for k, v in c.metadata.items()],
            [("blk.0.w", QTensor.from_blocks(np.frombuffer(q8, np.uint8), (3, 64), GgmlDType.Q8_0, device="cpu")),
             ("blk.0.norm", torch.from_numpy(f32)),
             ("blk.0.k", QTensor.from_blocks(np.frombuffer(q4k, np.uint8), (2, 256), GgmlDType.Q4K, device="cpu"))])
    assert f.getvalue() == buf


def test_custom_alignment_round_trip():
    f = io.BytesIO()
    G.write(f, [], [("a", torch.ones(3)), ("b", torch.zeros(70))], alignment=64)
    c = G.Content.read(f.getvalue())
    assert c.metadata["general.alignment"].to_u32() == 64
    assert c.tensor_data_offset % 64 == 0 and c.tensor_infos["b"].offset == 64


def test_errors():
    buf, _ = _hand_built()
    with pytest.raises(SxqError, match="magic"):
        G.Content.read(b"GGUX" + buf[4:])
    with pytest.raises(SxqError, match="version"):
        G.Content.read(buf[:4] + struct.pack("<I", 4) + buf[8:])
    with pytest.raises(SxqError, match="truncated|past the end"):
        G.Content.read(buf[:len(buf) - 40])
    with pytest.raises(SxqError, match="truncated"):
        G.Content.read(buf[:30])
    c = G.Content.read(buf)
    with pytest.raises(SxqError, match="no tensor"):
        c.tensor("missing", device="cpu")
    # a GGML type with no kernels here (Q6_K) is listed but refused as a QTensor
    f = io.BytesIO()
    f.write(struct.pack("<IIQQ", 0x46554747, 3, 1, 0) + _s("q6") + struct.pack("<IQQIQ", 2, 256, 1, 14, 0))
    f.write(_pad(f.tell()) + b"\0" * 210)
    c = G.Content.read(f.getvalue())
    assert c.tensor_infos["q6"].nbytes() == 210
    with pytest.raises(SxqError, match="not supported"):
        c.tensor("q6", device="cpu")
    with pytest.raises(SxqError, match="alignment"):
        G.write(io.BytesIO(), [("general.alignment", 64)], [], alignment=32)
    with pytest.raises(SxqError, match="duplicate"):
        G.write(io.BytesIO(), [], [("a", torch.ones(2)), ("a", torch.ones(2))])


def test_fish_projection_names():
    assert is_fish_projection("layers.3.attention.wqkv.weight") and is_fish_projection("fast_layers.0.feed_forward.w2.weight")
    assert is_fish_projection("output.weight") and is_fish_projection("fast_output.weight")
    assert is_fish_projection("fast_project_in.weight")
    # embeddings.weight stays a dense table: the token embedding gathers it (slow_ar.rs:117)
    for n in ("layers.3.attention_norm.weight", "codebook_embeddings.weight", "fast_embeddings.weight",
              "layers.0.attention.q_norm.weight", "norm.weight", "embeddings.weight", "layers.0.attention.wo.bias",
              "fast_project_in.bias"):
        assert not is_fish_projection(n)
