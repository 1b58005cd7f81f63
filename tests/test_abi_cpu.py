"""CPU-only checks of the C-ABI library: it loads, exports every symbol include/sxq.h
declares, and rejects bad arguments (with Candle's error text) before touching a GPU."""
import ctypes

import pytest

import syrinx_amd
from syrinx_amd import _lib


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    names = _lib.header_functions()
    assert len(names) >= 15
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_block_geometry_matches_ggml():
    L = _lib.lib()
    G = syrinx_amd.GgmlDType
    assert [L.sxq_block_size(int(d)) for d in (G.Q4_0, G.Q8_0, G.Q4K, G.Q8K)] == [32, 32, 256, 256]
    assert [L.sxq_type_size(int(d)) for d in (G.Q4_0, G.Q8_0, G.Q4K, G.Q8K)] == [18, 34, 144, 292]
    assert G.Q4K.block_size() == 256 and G.Q8_0.type_size() == 34
    assert L.sxq_block_size(99) == 0


def _create(dtype, n, k, nbytes, buf=None):
    L = _lib.lib()
    h = ctypes.c_void_p()
    rc = L.sxq_qmm_create(0, dtype, n, k, buf, nbytes, 0, ctypes.byref(h))
    return rc, L.sxq_last_error().decode(), h


def test_create_rejects_misaligned_k_with_candle_message():
    rc, msg, h = _create(12, 10, 896, 0)
    assert rc == _lib.ERR_BLOCK_ALIGN and not h.value
    assert msg == "quantized tensor must have their last dim divisible by block size [10, 896] 256"


def test_create_rejects_bad_dtype_and_size():
    assert _create(3, 10, 896, 0)[0] == _lib.ERR_DTYPE          # Q4_1: not on this path
    assert _create(15, 10, 256, 2920)[0] == _lib.ERR_DTYPE      # Q8K is an activation type
    rc, msg, _ = _create(8, 10, 896, 100)
    assert rc == _lib.ERR_SHAPE and "needs 9520" in msg
    assert _create(8, 0, 896, 0)[0] == _lib.ERR_INVALID
    buf = ctypes.create_string_buffer(9520)
    assert _create(8, 10, 896, 9520, None)[0] == _lib.ERR_INVALID  # null blocks
    del buf


def test_forward_argument_checks_need_no_gpu():
    L = _lib.lib()
    shape = (ctypes.c_int64 * 2)(1, 896)
    assert L.sxq_qmm_forward(None, None, shape, 2, None, None, None, 0, None) == _lib.ERR_INVALID
    assert L.sxq_qmm_destroy(None) == _lib.OK
    assert L.sxq_quantize_rows(0, 12, None, 4, 896, None, None) == _lib.ERR_BLOCK_ALIGN
    assert L.sxq_quantize_rows(0, 3, None, 4, 896, None, None) == _lib.ERR_DTYPE
    assert L.sxq_act_quantize(0, 12, None, 1, 256, None, None) == _lib.ERR_DTYPE


def test_workspace_entry_points_check_arguments_without_a_gpu():
    L = _lib.lib()
    shape = (ctypes.c_int64 * 2)(1, 896)
    sz = ctypes.c_size_t(123)
    assert L.sxq_qmm_workspace_size(None, 1, 0, ctypes.byref(sz)) == _lib.ERR_INVALID
    assert L.sxq_qmm_workspace_size(None, 1, 0, None) == _lib.ERR_INVALID
    assert L.sxq_qmm_forward_ws(None, None, shape, 2, None, None, None, 0, None, 0, None) == _lib.ERR_INVALID
    assert "null handle" in L.sxq_last_error().decode()


def test_fast_expand_and_reset_check_arguments_without_a_gpu():
    L = _lib.lib()
    assert L.sxq_fish_fast_expand(None, 1, None, None, 1, None, None, None, 10, None, 1, 0, None) == _lib.ERR_INVALID
    assert "null handle" in L.sxq_last_error().decode()
    assert L.sxq_lm_reset(None, 1, None) == _lib.ERR_INVALID


def test_embed_entry_points_check_arguments_without_a_gpu():
    L = _lib.lib()
    eff = ctypes.c_int()
    assert L.sxq_embed_scheme(4, 896, ctypes.byref(eff)) == _lib.OK and eff.value == 4
    assert L.sxq_embed_scheme(4, 81, ctypes.byref(eff)) == _lib.OK and eff.value == 8  # odd width: int8
    assert L.sxq_embed_scheme(5, 896, ctypes.byref(eff)) == _lib.ERR_INVALID
    assert L.sxq_embed_quantize(0, 4, None, 10, 81, None, None, None) == _lib.ERR_INVALID
    assert "odd" in L.sxq_last_error().decode()
    assert L.sxq_embed_gather(0, 8, None, None, 10, 16, None, 0, None, None) == _lib.OK  # nothing to gather
    assert L.sxq_lm_set_embed_quantized(None, 4, None, None) == _lib.ERR_INVALID


def test_python_mirror_rejects_misaligned_quantize():
    import torch
    with pytest.raises(syrinx_amd.SxqError) as e:
        syrinx_amd.QTensor.quantize(torch.zeros(4, 896), syrinx_amd.GgmlDType.Q4K)
    assert "divisible by block size [4, 896] 256" in str(e.value)
    with pytest.raises(syrinx_amd.SxqError):
        syrinx_amd.QTensor.quantize(torch.tensor(1.0), syrinx_amd.GgmlDType.Q8_0)
