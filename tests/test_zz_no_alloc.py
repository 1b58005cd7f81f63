"""sxq_qmm_forward_noalloc (the QMatMul forward whose workspace is the library's fixed
device scratch) against sxq_qmm_forward on the same inputs: bit-identical outputs on
two calls in a row, the second smaller than the first, for the decode GEMV, the
matrix-core GEMV and the prefill GEMM; sizes beyond the scratch are refused before any
GPU work."""
import ctypes

import numpy as np
import pytest
import torch

from syrinx_amd import GgmlDType, QMatMul, QTensor, SxqError, lib
from syrinx_amd._lib import check

pytestmark = pytest.mark.gpu

G = GgmlDType


@pytest.fixture(scope="module")
def cuda():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a ROCm GPU")
    return torch.device("cuda:0")


def _noalloc():
    return lib().sxq_qmm_forward_noalloc


def _call(fn, qmm, x, bias=None, flags=0):
    n = qmm.shape[0]
    y = torch.full(tuple(x.shape[:-1]) + (n,), float("nan"), dtype=torch.float32, device=x.device)
    shape = (ctypes.c_int64 * x.dim())(*x.shape)
    stream = ctypes.c_void_p(torch.cuda.current_stream(x.device).cuda_stream)
    check(fn(ctypes.c_void_p(qmm.handle()), ctypes.c_void_p(x.data_ptr()), shape, x.dim(), None,
             ctypes.c_void_p(y.data_ptr()), ctypes.c_void_p(bias.data_ptr()) if bias is not None else None, flags,
             stream))
    return y


def _bits_equal(a, b, what):
    a = a.cpu().numpy().view(np.uint32)
    b = b.cpu().numpy().view(np.uint32)
    assert np.array_equal(a, b), f"{what}: {(a != b).sum()} of {a.size} differ"


# (dtype, n, k, first m, second m): the second call smaller than the first
CASES = [
    (G.Q4K, 2560, 4096, 128, 3),   # prefill GEMM (split-K partials in the scratch), then the GEMV
    (G.Q4K, 6144, 2560, 16, 1),    # matrix-core GEMV, then the one-row GEMV
    (G.Q8_0, 4864, 896, 40, 5),    # Q8_0 GEMV in 16-row slabs, then four rows + one
    (G.Q4_0, 896, 4864, 7, 2),
]


@pytest.mark.parametrize("dt,n,k,m1,m2", CASES)
def test_noalloc_forward_equals_forward(cuda, dt, n, k, m1, m2):
    fn = _noalloc()
    g = torch.Generator(device=cuda).manual_seed(n + k)
    w = torch.randn(n, k, device=cuda, generator=g) * 0.02
    qmm = QMatMul.from_qtensor(QTensor.quantize(w, dt))
    bias = torch.randn(n, device=cuda, generator=g) * 0.02
    for m, with_bias in ((m1, False), (m2, True)):
        x = torch.randn(m, k, device=cuda, generator=g)
        b = bias if with_bias else None
        want = qmm.forward(x, bias=b)
        got = _call(fn, qmm, x, bias=b)
        torch.cuda.synchronize()
        _bits_equal(got, want, f"{dt.name} [{n}x{k}] m={m}")


def test_noalloc_in_a_captured_graph(cuda):
    """Under graph capture, with nothing allocated by the call: replays equal eager."""
    fn = _noalloc()
    n, k = 2560, 2560
    g = torch.Generator(device=cuda).manual_seed(5)
    qmm = QMatMul.from_qtensor(QTensor.quantize(torch.randn(n, k, device=cuda, generator=g) * 0.02, G.Q4K))
    x = torch.randn(1, k, device=cuda, generator=g)
    want = qmm.forward(x)
    s = torch.cuda.Stream(device=cuda)
    s.wait_stream(torch.cuda.current_stream(cuda))
    y = torch.empty((1, n), device=cuda)
    shape = (ctypes.c_int64 * 2)(1, k)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        check(fn(ctypes.c_void_p(qmm.handle()), ctypes.c_void_p(x.data_ptr()), shape, 2, None,
                 ctypes.c_void_p(y.data_ptr()), None, 0, ctypes.c_void_p(s.cuda_stream)))
    torch.cuda.synchronize()
    for _ in range(3):
        _ = torch.zeros(1000, device=cuda).sum().item()
        y.zero_()
        graph.replay()
        torch.cuda.synchronize()
        _bits_equal(y, want, "captured noalloc forward")


def test_noalloc_refuses_sizes_beyond_the_scratch(cuda):
    fn = _noalloc()
    n, k = 2560, 9728
    qmm = QMatMul.from_qtensor(QTensor.quantize(torch.zeros(n, k, device=cuda), G.Q4K))
    x = torch.zeros(4096, k, device=cuda)  # 80 MB of f16 staging alone
    with pytest.raises(SxqError) as e:
        _call(fn, qmm, x)
    assert "fixed scratch" in str(e.value)
