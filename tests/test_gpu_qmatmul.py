"""GPU parity of the quantized path against the CPU oracle (Candle's generic CPU path).

Bar: bit-exact.  Weight and activation blocks are byte-identical, dequantized weights
bit-identical, and QMatMul outputs bit-identical to Candle's generic vec-dot order,
for every row count of the decode GEMV -- integer and float steps replay Candle's order.
The prefill GEMM (Q4_K, >= 64 rows) rounds both operands to f16 for MFMA: it is held to
the rounding bound of that, against the f64 product of the exactly dequantized weight.
"""
import threading

import numpy as np
import pytest
import torch

from syrinx_amd import GgmlDType, QMatMul, QTensor, SxqError
from syrinx_amd.quantized import qmatmul_host

pytestmark = pytest.mark.gpu

G = GgmlDType


@pytest.fixture(scope="module")
def cuda():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a ROCm GPU (torch.cuda.is_available() is False)")
    return torch.device("cuda:0")


def _weights(n, k, seed, std=0.02):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * std).astype(np.float32)
    # edge rows: a zero row, a row of ties, a row with f16-subnormal scales, a large row
    if n >= 4:
        w[0] = 0.0
        w[1, :] = 0.5
        w[1, ::2] = -0.5
        w[2] *= 1e-4
        w[3] *= 1e4
    return w


def _acts(m, k, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(np.float32)
    if m >= 3:
        x[1] = 0.0             # all-zero activation row -> d = 0 blocks
        x[2, :64] = 3.0        # ties at the maximum magnitude
        x[2, 64:128] = -3.0
    return x


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _eq_bits(got, want):
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    assert got.shape == want.shape
    same = (_bits(got) == _bits(want)) | ((got == 0) & (want == 0))  # +0 == -0
    if not same.all():
        i = np.argwhere(~same)[:5]
        raise AssertionError(f"{(~same).sum()} of {same.size} differ; first {i.tolist()}: "
                             f"got {got[tuple(i[0])]!r} want {want[tuple(i[0])]!r}")


# ------------------------------------------------------------------ quantize / dequantize
@pytest.mark.parametrize("dt,k", [(G.Q8_0, 896), (G.Q4_0, 896), (G.Q4K, 2560), (G.Q8_0, 4864), (G.Q8K, 2560)])
def test_quantize_rows_bytes_match_oracle(cuda, ora, dt, k):
    w = _weights(48, k, 1)
    qt = QTensor.quantize(torch.from_numpy(w).to(cuda), dt)
    got = qt.data().cpu().numpy().reshape(48, -1)
    want = ora.quantize(int(dt), w)
    np.testing.assert_array_equal(got, want)
    assert qt.storage_size_in_bytes() == want.size


@pytest.mark.parametrize("dt,k", [(G.Q8_0, 896), (G.Q4_0, 896), (G.Q4K, 2560), (G.Q8K, 512)])
def test_dequantize_bit_exact(cuda, ora, dt, k):
    w = _weights(32, k, 2)
    blocks = ora.quantize(int(dt), w)
    qt = QTensor.from_blocks(blocks, (32, k), dt, device=cuda)
    _eq_bits(qt.dequantize().cpu().numpy(), ora.dequantize(int(dt), blocks, k))


def test_dequantize_q4k_arbitrary_bytes(cuda, ora):
    # random scale/min/nibble bytes (finite f16 d, dmin): exercises every 6-bit packing path
    rng = np.random.default_rng(3)
    blk = rng.integers(0, 256, size=(64, 144), dtype=np.uint8)
    d = (rng.standard_normal((64, 2)) * 0.01).astype(np.float16)
    blk[:, :4] = d.view(np.uint8).reshape(64, 4)
    qt = QTensor.from_blocks(blk, (64, 256), G.Q4K, device=cuda)
    _eq_bits(qt.dequantize().cpu().numpy(), ora.dequantize(ora.Q4K, blk, 256))


@pytest.mark.parametrize("vdt,k", [(G.Q8_0, 896), (G.Q8_0, 4864), (G.Q8K, 2560), (G.Q8K, 9728)])
def test_activation_blocks_bit_exact(cuda, ora, vdt, k):
    import ctypes
    from syrinx_amd._lib import check, lib
    x = _acts(5, k, 4)
    xt = torch.from_numpy(x).to(cuda)
    nbytes = 5 * (k // vdt.block_size()) * vdt.type_size()
    out = torch.zeros(nbytes, dtype=torch.uint8, device=cuda)
    check(lib().sxq_act_quantize(0, int(vdt), ctypes.c_void_p(xt.data_ptr()), 5, k, ctypes.c_void_p(out.data_ptr()),
                                 torch.cuda.current_stream().cuda_stream))
    np.testing.assert_array_equal(out.cpu().numpy().reshape(5, -1), ora.quantize(int(vdt), x))


# ------------------------------------------------------------------ QMatMul forward
CASES = [
    (G.Q8_0, 4864, 896, 1),    # Qwen2-0.5B MLP up-projection, one row
    (G.Q8_0, 896, 4864, 1),    # down-proj
    (G.Q8_0, 128, 896, 3),     # k/v proj, ragged rows
    (G.Q4_0, 896, 896, 2),     # the dtype the reference ships
    (G.Q4_0, 6564, 896, 1),    # CV2 head shape
    (G.Q4K, 6144, 2560, 1),    # Qwen3-4B fused wqkv
    (G.Q4K, 2560, 9728, 1),    # w2
    (G.Q4K, 2560, 4096, 16),   # wo, skinny batch of 16
    (G.Q4K, 1003, 2560, 5),    # n not a multiple of the 8-row group
    (G.Q4K, 9728, 2560, 17),   # two 16-row slabs
    (G.Q8_0, 2560, 9728, 4),   # Q8_0 at the Qwen3-4B shape
    # tall matrices; 16389 rows leave a partial last workgroup of rows
    (G.Q4K, 16389, 1024, 1),
    (G.Q4K, 16389, 1024, 2),
    (G.Q4K, 16389, 512, 3),
    (G.Q4K, 16384, 9728, 4),   # nb = 38 blocks per row, four activation rows
    (G.Q4K, 19456, 2560, 1),   # Qwen3-4B fused w1|w3
    (G.Q4K, 2560, 9728, 10),   # skinny batch in chunks of four rows: 4 + 4 + 2
    (G.Q8_0, 896, 4864, 7),    # Q8_0 in chunks: 4 + 3
    (G.Q4K, 7, 256, 12),       # matrix-core GEMV: fewer weight rows than a tile, one block
    (G.Q4K, 40, 1536, 16),     # matrix-core GEMV: 6 blocks = a full and a partial chunk
    # matrix-core GEMV with two 16-row tiles per workgroup (16384 rows and more)
    (G.Q4K, 19456, 2560, 16),  # Qwen3-4B fused w1|w3 at the 16-stream batch
    (G.Q4K, 16400, 512, 7),    # last workgroup: one live tile, the other clamped
    (G.Q4K, 16389, 1024, 5),   # last workgroup: five live rows
    # Q8_0 at the Qwen3-4B widths: tall matrices with a partial last workgroup
    (G.Q8_0, 16389, 2560, 1),
    (G.Q8_0, 19456, 2560, 1),  # Qwen3-4B fused w1|w3
    (G.Q8_0, 2560, 9728, 1),   # w2 (K = 9728: 304 blocks per row)
    (G.Q8_0, 16389, 2560, 3),
    # one activation row of Q8_0 / Q4_0 (the GEMV quantizes x in its prologue): the
    # smallest matrix, the widest row it takes (384 blocks), and a wider one (512 blocks:
    # the quantizer and the GEMV as two launches)
    (G.Q8_0, 1, 32, 1),
    (G.Q4_0, 77, 12288, 1),
    (G.Q8_0, 300, 16384, 1),
    (G.Q4K, 1, 256, 1),        # the smallest Q4_K matrix
]


@pytest.mark.parametrize("dt,n,k,m", CASES)
def test_qmatmul_bit_exact_vs_oracle(cuda, ora, dt, n, k, m):
    w = _weights(n, k, 10 + n % 7)
    x = _acts(m, k, 20 + m)
    blocks = ora.quantize(int(dt), w)
    qmm = QMatMul.from_qtensor(QTensor.from_blocks(blocks, (n, k), dt, device=cuda))
    y = qmm.forward(torch.from_numpy(x).to(cuda))
    torch.cuda.synchronize()
    _eq_bits(y.cpu().numpy(), ora.matmul(int(dt), x, blocks))


def test_bias_batch_shape_and_host_pointers(cuda, ora):
    n, k = 896, 896
    w = _weights(n, k, 5)
    b = (np.random.default_rng(6).standard_normal(n) * 0.02).astype(np.float32)
    x = _acts(6, k, 7).reshape(2, 3, k)
    blocks = ora.quantize(ora.Q8_0, w)
    qmm = QMatMul.from_qtensor(QTensor.from_blocks(blocks, (n, k), G.Q8_0, device=cuda))
    y = qmm.forward(torch.from_numpy(x).to(cuda), bias=torch.from_numpy(b).to(cuda)).cpu().numpy()
    assert y.shape == (2, 3, n)
    want = (ora.matmul(ora.Q8_0, x.reshape(6, k), blocks) + b[None, :]).astype(np.float32)  # f32 bias add
    _eq_bits(y.reshape(6, n), want)
    _eq_bits(qmatmul_host(qmm, x, b).reshape(6, n), want)


def test_bias_on_tall_q4k(cuda, ora):
    # bias epilogue on a tall Q4_K matrix, rows not a multiple of 8
    n, k = 16395, 512
    w = _weights(n, k, 31)
    b = (np.random.default_rng(32).standard_normal(n) * 0.02).astype(np.float32)
    x = _acts(2, k, 33)
    blocks = ora.quantize(ora.Q4K, w)
    qmm = QMatMul.from_qtensor(QTensor.from_blocks(blocks, (n, k), G.Q4K, device=cuda))
    y = qmm.forward(torch.from_numpy(x).to(cuda), bias=torch.from_numpy(b).to(cuda)).cpu().numpy()
    _eq_bits(y, (ora.matmul(ora.Q4K, x, blocks) + b[None, :]).astype(np.float32))


def test_bias_on_q4k_matrix_core_rows(cuda, ora):
    # 5..16 rows of Q4_K take the matrix-core GEMV: bias epilogue, ragged n, 9 rows
    n, k = 1003, 2560
    w = _weights(n, k, 34)
    b = (np.random.default_rng(35).standard_normal(n) * 0.02).astype(np.float32)
    x = _acts(9, k, 36)
    blocks = ora.quantize(ora.Q4K, w)
    qmm = QMatMul.from_qtensor(QTensor.from_blocks(blocks, (n, k), G.Q4K, device=cuda))
    y = qmm.forward(torch.from_numpy(x).to(cuda), bias=torch.from_numpy(b).to(cuda)).cpu().numpy()
    _eq_bits(y, (ora.matmul(ora.Q4K, x, blocks) + b[None, :]).astype(np.float32))


def test_export_and_dequantize_round_trip(cuda, ora):
    w = _weights(300, 2560, 8)
    blocks = ora.quantize(ora.Q4K, w)
    qmm = QMatMul.from_qtensor(QTensor.from_blocks(blocks, (300, 2560), G.Q4K, device=cuda))
    np.testing.assert_array_equal(qmm.export_blocks().cpu().numpy(), blocks.ravel())
    _eq_bits(qmm.dequantize().cpu().numpy(), ora.dequantize(ora.Q4K, blocks, 2560))
    assert qmm.storage_size_in_bytes() == blocks.size


def test_forward_error_behaviour(cuda):
    qmm = QMatMul.from_qtensor(QTensor.quantize(torch.randn(64, 512, device=cuda) * 0.02, G.Q8_0))
    with pytest.raises(SxqError) as e:
        qmm.forward(torch.randn(2, 256, device=cuda))
    assert "incompatible with [64, 512]" in str(e.value)
    with pytest.raises(SxqError) as e:
        qmm.forward(torch.randn(512, device=cuda))
    assert "only one dimension" in str(e.value)
    with pytest.raises(SxqError) as e:
        qmm.forward(torch.randn(512, 4, device=cuda).t())
    assert "not contiguous" in str(e.value)
    with pytest.raises(SxqError):
        qmm.forward(torch.randn(2, 512, device=cuda, dtype=torch.float16))
    y = qmm.forward(torch.zeros(0, 512, device=cuda))
    assert y.shape == (0, 64)


def test_concurrent_forward_on_one_handle(cuda, ora):
    # tests/real_lm_hammer.rs:48-83 shares one model across threads; forward is re-entrant.
    n, k = 2048, 2560
    w = _weights(n, k, 9)
    blocks = ora.quantize(ora.Q4K, w)
    qmm = QMatMul.from_qtensor(QTensor.from_blocks(blocks, (n, k), G.Q4K, device=cuda))
    xs = [_acts(1 + i % 3, k, 30 + i) for i in range(6)]
    want = [ora.matmul(ora.Q4K, x, blocks) for x in xs]
    out = [None] * len(xs)

    def run(i):
        s = torch.cuda.Stream(device=cuda)
        with torch.cuda.stream(s):
            for _ in range(3):
                y = qmm.forward(torch.from_numpy(xs[i]).to(cuda))
            s.synchronize()
            out[i] = y.cpu().numpy()

    th = [threading.Thread(target=run, args=(i,)) for i in range(len(xs))]
    for t in th:
        t.start()
    for t in th:
        t.join()
    for o, wnt in zip(out, want):
        _eq_bits(o, wnt)


@pytest.mark.parametrize("dt", [G.Q4K, G.Q8_0])
def test_full_size_tied_head(cuda, ora, dt):
    # The Qwen3-4B tied LM head [155776 x 2560] at full size, bit-exact on every row (Q8_0:
    # the 424 MB head of the Q8_0 decode configuration).
    n, k = 155776, 2560
    g = torch.Generator(device=cuda).manual_seed(11)
    w = torch.randn(n, k, device=cuda, generator=g) * 0.02
    qt = QTensor.quantize(w, dt)
    del w
    qmm = QMatMul.from_qtensor(qt)
    x = _acts(1, k, 12)
    y = qmm.forward(torch.from_numpy(x).to(cuda)).cpu().numpy()
    blocks = qt.data().cpu().numpy().reshape(n, -1)
    _eq_bits(y, ora.matmul(int(dt), x, blocks))


# ------------------------------------------------------------------ prefill GEMM (MFMA)
PREFILL = [
    (300, 512, 200),     # rows and outputs not multiples of the 128 x 128 tile, with bias
    (6144, 2560, 512),   # Qwen3-4B fused wqkv at a 512-token prompt
    (2560, 9728, 128),   # down projection, K = 9728 (38 blocks)
    # the other three projections of a Qwen3-4B layer at 512 tokens, each with the split
    # plan the default forward picks: wo and w2 split K six ways (40 tiles for 256 CUs),
    # the fused w1|w3 runs 256 whole tiles and splits the remaining 48 five ways
    (2560, 4096, 512),   # wo
    (19456, 2560, 512),  # w1|w3
    (2560, 9728, 512),   # w2
]


# Q8_0 / Q4_0 prompts: the int8 matrix-core GEMM, bit-identical to the oracle at every row
# count (dtype, weight rows n, k, prompt rows m, with bias)
PREFILL_Q80 = [
    (G.Q8_0, 4864, 896, 512, False),   # CosyVoice2 gate/up at a 512-token prompt
    (G.Q8_0, 896, 4864, 130, True),    # down projection, rows not a multiple of the 64-row tile
    (G.Q4_0, 896, 896, 128, True),     # the dtype the reference ships, exactly two row tiles
    (G.Q4_0, 1003, 896, 200, False),   # weight rows not a multiple of the 128-row tile
    (G.Q8_0, 6144, 2560, 160, False),  # Qwen3-4B wqkv, Q8_0
    (G.Q4_0, 6564, 896, 129, True),    # CosyVoice2 head shape, one row into the third tile
]


@pytest.mark.parametrize("dt,n,k,m,with_bias", PREFILL_Q80)
def test_prefill_gemm_q8_0_q4_0_bit_exact(cuda, ora, dt, n, k, m, with_bias):
    w = _weights(n, k, 80 + m)
    x = _acts(m, k, 81 + m)
    blocks = ora.quantize(int(dt), w)
    qmm = QMatMul.from_qtensor(QTensor.from_blocks(blocks, (n, k), dt, device=cuda))
    b = (np.random.default_rng(82).standard_normal(n) * 0.02).astype(np.float32) if with_bias else None
    y = qmm.forward(torch.from_numpy(x).to(cuda), bias=None if b is None else torch.from_numpy(b).to(cuda))
    want = ora.matmul(int(dt), x, blocks)
    if b is not None:
        want = (want + b[None, :]).astype(np.float32)
    _eq_bits(y.cpu().numpy(), want)


# The CosyVoice3 flow's DiT linears (crates/syrinx-acoustic/src/cv3/dit.rs, Q4_0 from
# crates/syrinx-acoustic/src/cv3/mod.rs:150-168, bias added after QMatMul::forward at
# :200-211) at M = CFG batch 2 x 250 mel frames, and their batch-row users at M = 2.
DIT = [
    (1024, 1024, 500),   # to_q / to_k / to_v / to_out.0 (dit.rs:241-267)
    (2048, 1024, 500),   # ff.0.0 (dit.rs:272)
    (1024, 2048, 500),   # ff.2
    (1024, 320, 500),    # input_embed.proj over [x, cond, mu, spks] (dit.rs:61-64)
    (80, 1024, 500),     # proj_out (dit.rs:79)
    (6144, 1024, 2),     # AdaLayerNormZero linear (dit.rs:196)
    (1024, 256, 2),      # time_mlp.0 (dit.rs:93)
]


@pytest.mark.parametrize("n,k,m", DIT)
def test_flow_dit_linears_bit_exact(cuda, ora, n, k, m):
    w = _weights(n, k, 90 + n)
    x = _acts(m, k, 91 + k)
    blocks = ora.quantize(ora.Q4_0, w)
    qmm = QMatMul.from_qtensor(QTensor.from_blocks(blocks, (n, k), G.Q4_0, device=cuda))
    b = (np.random.default_rng(92).standard_normal(n) * 0.02).astype(np.float32)
    y = qmm.forward(torch.from_numpy(x).to(cuda).reshape(2, m // 2, k), bias=torch.from_numpy(b).to(cuda))
    assert tuple(y.shape) == (2, m // 2, n)
    want = (ora.matmul(ora.Q4_0, x, blocks) + b[None, :]).astype(np.float32)
    _eq_bits(y.reshape(m, n).cpu().numpy(), want)


def _prefill_check(ora, x, blocks, k, y, b=None):
    wd = ora.dequantize(ora.Q4K, blocks, k).reshape(-1, k).astype(np.float64)  # Candle's to_float, exact
    y64 = x.astype(np.float64) @ wd.T + (0.0 if b is None else b.astype(np.float64))
    S = np.abs(x).astype(np.float64) @ np.abs(wd).T
    tol = (2.0 ** -10 + k * 2.0 ** -24) * S + 2.0 ** -24 * np.abs(x).sum(1, keepdims=True) + 1e-30
    err = np.abs(y - y64)
    assert (err <= tol).all(), f"{int((err > tol).sum())} outputs beyond the bound; worst ratio {float((err / tol).max()):.3g}"


@pytest.mark.parametrize("k", [512, 2560, 4096, 9728])
def test_one_pass_f16_conversion_equals_two_pass(cuda, ora, monkeypatch, k):
    """The prefill GEMM's x -> f16 (GEMM K order) conversion in one pass over the row gives
    the two-pass kernel's bits: the products of both are identical, for rows with and
    without the power-of-two scaling (values beyond f16's range)."""
    n, m = 384, 96
    blocks = ora.quantize(ora.Q4K, _weights(n, k, 70))
    qmm = QMatMul.from_qtensor(QTensor.from_blocks(blocks, (n, k), G.Q4K, device=cuda))
    x = _acts(m, k, 71)
    x[5] *= 1e5   # a row scaled by 2^-e before the rounding
    x[7, 3] = 7e4
    xt = torch.from_numpy(x).to(cuda)
    y1 = qmm.forward(xt).cpu().numpy()
    monkeypatch.setenv("SXQ_X2F16_TWO_PASS", "1")
    y2 = qmm.forward(xt).cpu().numpy()
    _eq_bits(y1, y2)


@pytest.mark.parametrize("splits", ["1", "3"])
def test_prefill_gemm_split_counts_agree(cuda, ora, monkeypatch, splits):
    """The same product with K unsplit and split unevenly across workgroups (4 blocks
    into 1 + 1 + 2): both within the f16 bound, and the split partials are added in a
    fixed order, so repeated calls give identical bits."""
    n, k, m = 600, 1024, 256
    w = _weights(n, k, 43)
    x = _acts(m, k, 44)
    blocks = ora.quantize(ora.Q4K, w)
    qmm = QMatMul.from_qtensor(QTensor.from_blocks(blocks, (n, k), G.Q4K, device=cuda))
    xt = torch.from_numpy(x).to(cuda)
    monkeypatch.setenv("SXQ_GEMM_SPLITS", splits)
    y1 = qmm.forward(xt).cpu().numpy()
    y2 = qmm.forward(xt).cpu().numpy()
    _eq_bits(y1, y2)
    _prefill_check(ora, x, blocks, k, y1.astype(np.float64))


@pytest.mark.parametrize("n,k,m", PREFILL)
def test_prefill_gemm_within_f16_rounding_bound(cuda, ora, n, k, m):
    w = _weights(n, k, 40 + n % 5)
    x = _acts(m, k, 41)
    b = (np.random.default_rng(42).standard_normal(n) * 0.02).astype(np.float32) if n == 300 else None
    blocks = ora.quantize(ora.Q4K, w)
    qmm = QMatMul.from_qtensor(QTensor.from_blocks(blocks, (n, k), G.Q4K, device=cuda))
    xt = torch.from_numpy(x).to(cuda)
    y = qmm.forward(xt, bias=None if b is None else torch.from_numpy(b).to(cuda)).cpu().numpy().astype(np.float64)
    wd = ora.dequantize(ora.Q4K, blocks, k).reshape(n, k).astype(np.float64)  # Candle's to_float, exact
    y64 = x.astype(np.float64) @ wd.T + (0.0 if b is None else b.astype(np.float64))
    # Bound: each operand rounded to f16 (relative 2^-11, or 2^-25 absolute in the
    # subnormal range), products and sums in f32.
    S = np.abs(x).astype(np.float64) @ np.abs(wd).T
    tol = (2.0 ** -10 + k * 2.0 ** -24) * S + 2.0 ** -24 * np.abs(x).sum(1, keepdims=True) + 1e-30
    err = np.abs(y - y64)
    assert (err <= tol).all(), f"{int((err > tol).sum())} outputs beyond the bound; worst ratio {float((err / tol).max()):.3g}"
    # typical error, relative to the output scale
    rel = float(np.sqrt(np.mean(err ** 2)) / np.sqrt(np.mean(y64 ** 2)))
    print(f"prefill GEMM [{n}x{k}] at {m} rows: rms rel err {rel:.2e}, worst/bound {float((err / tol).max()):.3f}")
    assert rel < 2e-3, rel
    # the split partials are added in a fixed order: a second call gives the same bits
    y2 = qmm.forward(xt, bias=None if b is None else torch.from_numpy(b).to(cuda)).cpu().numpy()
    _eq_bits(y2, y.astype(np.float32))
    # the exact path stays available and bit-identical for the same call
    if m <= 200:
        y_exact = qmm.forward(xt, bias=None if b is None else torch.from_numpy(b).to(cuda), exact=True).cpu().numpy()
        want = ora.matmul(ora.Q4K, x, blocks)
        if b is not None:
            want = (want + b[None, :]).astype(np.float32)
        _eq_bits(y_exact, want)


BF16_CASES = [  # (dtype, n, k, m): the GEMV, the 5..16-row matrix-core GEMV, both prefill GEMMs
    (G.Q4K, 2560, 2560, 1), (G.Q4K, 1003, 2560, 9), (G.Q4K, 2560, 4096, 128), (G.Q8_0, 896, 896, 3),
    (G.Q8_0, 4864, 896, 200), (G.Q4_0, 896, 896, 130),
]


@pytest.mark.parametrize("dt,n,k,m", BF16_CASES)
def test_bf16_input_equals_f32_input_of_the_same_values(cuda, ora, dt, n, k, m):
    """SXQ_BF16_INPUT: bf16 activations (the Fish GPU path's dtype) widen to f32 exactly, so
    the outputs are those of the f32 input holding the same values, bit for bit -- on
    device pointers, on host pointers and through the no-allocation entry point."""
    import ctypes
    from syrinx_amd._lib import BF16_INPUT, HOST_PTRS, check, lib
    w = _weights(n, k, 70 + m)
    blocks = ora.quantize(int(dt), w)
    qmm = QMatMul.from_qtensor(QTensor.from_blocks(blocks, (n, k), dt, device=cuda))
    xb = torch.from_numpy(_acts(m, k, 71 + m)).to(torch.bfloat16).to(cuda)
    want = qmm.forward(xb.float()).cpu().numpy()
    _eq_bits(qmm.forward(xb).cpu().numpy(), want)
    # host pointers: the bf16 bits from host memory
    xh = xb.cpu().view(torch.int16).numpy().copy()
    yh = np.empty((m, n), np.float32)
    shape = (ctypes.c_int64 * 2)(m, k)
    check(lib().sxq_qmm_forward(qmm._h, xh.ctypes.data_as(ctypes.c_void_p), shape, 2, None,
                                yh.ctypes.data_as(ctypes.c_void_p), None, HOST_PTRS | BF16_INPUT, None))
    _eq_bits(yh, want)
    # the fixed-scratch entry point
    y = torch.empty((m, n), dtype=torch.float32, device=cuda)
    check(lib().sxq_qmm_forward_noalloc(qmm._h, ctypes.c_void_p(xb.data_ptr()), shape, 2, None,
                                        ctypes.c_void_p(y.data_ptr()), None, BF16_INPUT,
                                        ctypes.c_void_p(torch.cuda.current_stream(cuda).cuda_stream)))
    _eq_bits(y.cpu().numpy(), want)


def test_bf16_input_captured_in_a_graph(cuda, ora):
    """A bf16 forward under graph capture takes its workspace (with the f32 copy of x)
    from the graph's pool; replays give the eager bits."""
    n, k, m = 2560, 2560, 3
    w = _weights(n, k, 80)
    qmm = QMatMul.from_qtensor(QTensor.from_blocks(ora.quantize(int(G.Q4K), w), (n, k), G.Q4K, device=cuda))
    x = torch.from_numpy(_acts(m, k, 81)).to(torch.bfloat16).to(cuda)
    want = qmm.forward(x).cpu().numpy()
    s = torch.cuda.Stream(device=cuda)
    s.wait_stream(torch.cuda.current_stream(cuda))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        y = qmm.forward(x)
    for _ in range(3):
        _ = torch.zeros(1000, device=cuda).sum().item()  # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        _eq_bits(y.cpu().numpy(), want)


def test_unsupported_input_dtype_is_refused(cuda, ora):
    qmm = QMatMul.from_qtensor(QTensor.from_blocks(ora.quantize(int(G.Q8_0), _weights(64, 64, 1)), (64, 64), G.Q8_0,
                                                   device=cuda))
    with pytest.raises(SxqError, match="unsupported dtype"):
        qmm.forward(torch.zeros((1, 64), dtype=torch.float16, device=cuda))


def test_forward_captured_in_a_graph(cuda, ora):
    # QMatMul.forward captured into a HIP graph (it takes a workspace of its own from the
    # graph's memory pool): GEMV, matrix-core GEMV and the split-K prefill GEMM, each
    # replayed several times with eager work between the replays
    cases = [(G.Q4K, 2560, 2560, 1), (G.Q4K, 1003, 2560, 9), (G.Q8_0, 896, 896, 3), (G.Q4K, 2560, 4096, 128)]
    for dt, n, k, m in cases:
        w = _weights(n, k, 40 + m)
        blocks = ora.quantize(ora.Q4K if dt == G.Q4K else ora.Q8_0, w)
        qmm = QMatMul.from_qtensor(QTensor.from_blocks(blocks, (n, k), dt, device=cuda))
        x = torch.from_numpy(_acts(m, k, 41 + m)).to(cuda)
        want = qmm.forward(x).cpu().numpy()
        s = torch.cuda.Stream(device=cuda)
        s.wait_stream(torch.cuda.current_stream(cuda))
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            y = qmm.forward(x)
        torch.cuda.synchronize()
        for rep in range(3):
            _ = torch.zeros(1000, device=cuda).sum().item()  # eager work between replays
            y.zero_()
            graph.replay()
            torch.cuda.synchronize()
            np.testing.assert_array_equal(y.cpu().numpy(), want, err_msg=f"{dt} m={m} replay {rep}")


def test_captured_workspaces_are_released_with_their_outputs(cuda, ora):
    """Each captured forward's workspace lives as long as its output: capturing the same
    QMatMul again and again (dropping the old graph and output) holds no more device
    memory than one capture does."""
    n, k, m = 2560, 4096, 128  # the prefill GEMM: a multi-MB workspace per capture
    blocks = ora.quantize(ora.Q4K, _weights(n, k, 66))
    qmm = QMatMul.from_qtensor(QTensor.from_blocks(blocks, (n, k), G.Q4K, device=cuda))
    x = torch.from_numpy(_acts(m, k, 67)).to(cuda)
    want = qmm.forward(x).cpu().numpy()
    torch.cuda.synchronize()
    held = []
    for rep in range(6):
        s = torch.cuda.Stream(device=cuda)
        s.wait_stream(torch.cuda.current_stream(cuda))
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            y = qmm.forward(x)
        graph.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(y.cpu().numpy(), want)
        del graph, y
        torch.cuda.synchronize()
        held.append(torch.cuda.memory_allocated(cuda))
    assert max(held[1:]) <= held[0], held


def test_captured_forward_survives_a_larger_eager_call(cuda, ora):
    """Capture a one-row forward, then run an eager 128-row prefill forward (which grows
    the library's shared workspace), then replay: the graph's workspace is its own, so
    the replay is untouched by the regrowth."""
    n, k = 2560, 4096
    w = _weights(n, k, 60)
    blocks = ora.quantize(ora.Q4K, w)
    qmm = QMatMul.from_qtensor(QTensor.from_blocks(blocks, (n, k), G.Q4K, device=cuda))
    x1 = torch.from_numpy(_acts(1, k, 61)).to(cuda)
    want1 = ora.matmul(ora.Q4K, x1.cpu().numpy(), blocks)
    s = torch.cuda.Stream(device=cuda)
    s.wait_stream(torch.cuda.current_stream(cuda))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        y1 = qmm.forward(x1)
    torch.cuda.synchronize()
    big = torch.from_numpy(_acts(128, k, 62)).to(cuda)
    for rep in range(2):
        y_big = qmm.forward(big)  # eager, larger workspace
        y1.zero_()
        graph.replay()
        torch.cuda.synchronize()
        _eq_bits(y1.cpu().numpy(), want1)
        _prefill_check(ora, big.cpu().numpy(), blocks, k, y_big.cpu().numpy().astype(np.float64))


def test_replays_overlapping_eager_forwards_on_another_stream(cuda, ora):
    """A captured forward replayed on one stream while eager forwards of the same
    QMatMul run on another stream: both stay bit-exact (the replay's workspace is not
    the one the eager calls share)."""
    n, k = 6144, 2560
    blocks = ora.quantize(ora.Q4K, _weights(n, k, 63))
    qmm = QMatMul.from_qtensor(QTensor.from_blocks(blocks, (n, k), G.Q4K, device=cuda))
    xg = torch.from_numpy(_acts(1, k, 64)).to(cuda)
    xe = torch.from_numpy(_acts(9, k, 65)).to(cuda)
    want_g = ora.matmul(ora.Q4K, xg.cpu().numpy(), blocks)
    want_e = ora.matmul(ora.Q4K, xe.cpu().numpy(), blocks)
    sg, se = torch.cuda.Stream(device=cuda), torch.cuda.Stream(device=cuda)
    sg.wait_stream(torch.cuda.current_stream(cuda))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=sg):
        yg = qmm.forward(xg)
    torch.cuda.synchronize()
    outs = []
    for _ in range(20):
        with torch.cuda.stream(sg):
            graph.replay()
        with torch.cuda.stream(se):
            outs.append(qmm.forward(xe))
    torch.cuda.synchronize()
    _eq_bits(yg.cpu().numpy(), want_g)
    for y in outs:
        _eq_bits(y.cpu().numpy(), want_e)


def test_shared_workspace_forward_is_refused_under_capture(cuda, ora):
    """The C-ABI forward that uses the library's shared workspace refuses a capturing
    stream (a replay could overlap later eager calls); the error names the
    caller-workspace entry point."""
    import ctypes
    from syrinx_amd import lib
    n, k = 256, 256
    qmm = QMatMul.from_qtensor(QTensor.from_blocks(ora.quantize(ora.Q4K, _weights(n, k, 66)), (n, k), G.Q4K,
                                                   device=cuda))
    x = torch.from_numpy(_acts(1, k, 67)).to(cuda)
    y = torch.empty((1, n), device=cuda)
    shape = (ctypes.c_int64 * 2)(1, k)
    s = torch.cuda.Stream(device=cuda)
    s.wait_stream(torch.cuda.current_stream(cuda))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        rc = lib().sxq_qmm_forward(ctypes.c_void_p(qmm.handle()), ctypes.c_void_p(x.data_ptr()), shape, 2, None,
                                   ctypes.c_void_p(y.data_ptr()), None, 0, ctypes.c_void_p(s.cuda_stream))
        msg = lib().sxq_last_error().decode()
    assert rc == 1 and "sxq_qmm_forward_ws" in msg, (rc, msg)


def test_prefill_gemm_stays_finite_beyond_f16_range(cuda, ora):
    """Rows with values beyond f16's range (65504) are scaled by a power of two before
    the f16 rounding and back after the f32 accumulation: every output stays finite and
    within the f16 bound, with the subnormal floor raised by the row's 2^e; rows that
    stay below 2^15 give the same bits as without such rows in the batch."""
    n, k, m = 640, 2560, 64
    blocks = ora.quantize(ora.Q4K, _weights(n, k, 70))
    qmm = QMatMul.from_qtensor(QTensor.from_blocks(blocks, (n, k), G.Q4K, device=cuda))
    rng = np.random.default_rng(71)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[1] *= 1e5                                   # every value of the row large
    x[2, 7] = 1e30                                # one huge outlier in a normal row
    x[3, :] = 65504.0
    x[3, 1::2] = -70000.0                         # beyond f16's largest finite value
    x[4, 100] = 32768.0                           # exactly at the scaling threshold
    x[5] *= 1e-3                                  # small values, unscaled
    y = qmm.forward(torch.from_numpy(x).to(cuda)).cpu().numpy().astype(np.float64)
    assert np.isfinite(y).all()
    wd = ora.dequantize(ora.Q4K, blocks, k).reshape(n, k).astype(np.float64)
    y64 = x.astype(np.float64) @ wd.T
    amax = np.abs(x).max(1)
    e = np.where(amax >= 32768.0, np.frexp(amax)[1] - 15, 0).astype(np.float64)
    S = np.abs(x).astype(np.float64) @ np.abs(wd).T
    tol = ((2.0 ** -10 + k * 2.0 ** -24) * S + 2.0 ** -24 * np.abs(x).sum(1, keepdims=True)
           + 2.0 ** (e[:, None] - 24) * np.abs(wd).sum(1)[None, :] + 1e-30)
    err = np.abs(y - y64)
    assert (err <= tol).all(), f"{int((err > tol).sum())} beyond the bound; worst ratio {float((err / tol).max()):.3g}"
    # rows below the threshold are unaffected by the scaled rows in the same batch
    plain = x.copy()
    plain[1:5] = 0.0
    y_plain = qmm.forward(torch.from_numpy(plain).to(cuda)).cpu().numpy()
    keep = [0] + list(range(5, m))
    _eq_bits(y[keep].astype(np.float32), y_plain[keep])


@pytest.mark.parametrize("mode", ["f32", "f16", "dequantize_all", "dequantize_all_f16"])
def test_dense_qmatmul_variants(cuda, ora, monkeypatch, mode):
    """Candle's dense QMatMul variants (QMatMul::from_arc): an F32 / F16 QTensor, or a
    quantized one under CANDLE_DEQUANTIZE_ALL (f32 weight = to_float) or
    CANDLE_DEQUANTIZE_ALL_F16 (f16 weight, the input cast to f16 and the product cast
    back).  The weight must be Candle's exactly; the product is a dense GEMM, within the
    rounding bound of its precision (cv2/load.rs:107-110 keeps unaligned 2-D weights f16)."""
    n, k, m = 300, 512, 7
    w = _weights(n, k, 95)
    x = _acts(m, k, 96)
    if mode == "f32":
        qt, wd, eps = QTensor.quantize(torch.from_numpy(w), G.F32, device=cuda), w.astype(np.float64), 2.0 ** -15
    elif mode == "f16":
        qt = QTensor.quantize(torch.from_numpy(w), G.F16, device=cuda)
        wd, eps = w.astype(np.float16).astype(np.float64), 2.0 ** -15
    else:
        blocks = ora.quantize(ora.Q4K, w)
        qt = QTensor.from_blocks(blocks, (n, k), G.Q4K, device=cuda)
        wd = ora.dequantize(ora.Q4K, blocks, k).reshape(n, k).astype(np.float64)
        eps = 2.0 ** -15  # f32 accumulation over k = 512 terms: below k * 2^-24 of sum |x w|
        monkeypatch.setenv("CANDLE_DEQUANTIZE_ALL" if mode == "dequantize_all" else "CANDLE_DEQUANTIZE_ALL_F16", "1")
        if mode == "dequantize_all_f16":
            wd, eps = wd.astype(np.float16).astype(np.float64), 2.0 ** -10  # plus the f16 output rounding
    qmm = QMatMul.from_qtensor(qt)
    assert qmm.handle() == 0  # a dense weight: no sxq_qmm behind it
    wt = qmm._dense.to(torch.float64).cpu().numpy()
    np.testing.assert_array_equal(wt, wd)
    y = qmm.forward(torch.from_numpy(x).to(cuda)).cpu().numpy().astype(np.float64)
    xr = x.astype(np.float16).astype(np.float64) if mode == "dequantize_all_f16" else x.astype(np.float64)
    ref = xr @ wd.T
    bound = eps * (np.abs(xr) @ np.abs(wd).T) + 1e-30
    assert (np.abs(y - ref) <= bound).all(), float((np.abs(y - ref) / bound).max())
