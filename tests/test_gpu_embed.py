"""The device per-row embedding quantizer and dequant-on-gather (libsxq sxq_embed_*,
the reference's quantize_embed / embed_rows, crates/syrinx-lm/src/cv2/quant.rs:38-89 and
crates/syrinx-lm/src/cv2/generate.rs:22-67) against the oracle (oracle/embed.py): codes
and scales byte-identical, gathered rows bit-identical; and an engine holding its input
table quantized gives the bits of one holding the dequantized table densely."""
import numpy as np
import pytest
import torch

import embed as E
from syrinx_amd import decoder as D
from syrinx_amd.embedding import INT4, INT8, QEmbed

from test_gpu_decoder import _build

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def cuda():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a ROCm GPU")
    return torch.device("cuda:0")


def _table(rng, v, h):
    t = (rng.standard_normal((v, h)) * 0.5).astype(np.float32)
    t[3] = 0.0                      # the zero row: scale 1e-12, codes 0
    t[5, 7] = 40.0                  # an outlier row
    t[6] = np.round(t[6] * 14) / 2  # exact halves: the rounding of ties
    return t


@pytest.mark.parametrize("scheme,v,h", [(INT4, 6567, 896), (INT8, 6567, 896), (INT4, 37, 81), (INT8, 300, 1024)])
def test_quantize_and_gather_bit_exact(cuda, scheme, v, h):
    rng = np.random.default_rng(v + h + scheme)
    t = _table(rng, v, h)
    qe = QEmbed.quantize(torch.from_numpy(t).to(cuda), scheme)
    wq, ws, wscheme = E.quantize(t, scheme)
    assert qe.scheme == wscheme and qe.h == h
    np.testing.assert_array_equal(qe.scale.cpu().numpy().view(np.uint32), ws.view(np.uint32))
    np.testing.assert_array_equal(qe.q.cpu().numpy(), wq)
    assert qe.bytes == wq.size + 4 * v
    ids = np.concatenate([rng.integers(0, v, 50), [0, v - 1, 3, 5, 6, -1, v]])
    got = qe.rows(torch.from_numpy(ids.astype(np.int32))).cpu().numpy()
    want = E.gather(wq, ws, wscheme, h, ids)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("scheme", [INT4, INT8])
def test_engine_with_quantized_table_equals_dense_dequantized(cuda, scheme):
    cfg = D.cosyvoice2_lm_config(n_layers=2, max_seq=64, max_batch=3, dtype=D.GgmlDType.Q8_0)
    dense, W = _build(cfg, cuda, 61, 3)
    quant, _ = _build(cfg, cuda, 61, 3)
    rows = cfg.embed_rows
    qe = QEmbed.quantize(torch.from_numpy(W["embed"]).to(cuda), scheme)
    deq = qe.rows(torch.arange(rows, dtype=torch.int32))
    dense.set_vector(-1, D.EMBED, deq)
    quant.set_embed_quantized(qe)
    rng = np.random.default_rng(62)
    prompts = [rng.integers(0, rows, T).astype(np.int32) for T in (4, 9, 2)]
    outs = []
    for lm in (dense, quant):
        lm.reset(3)
        lg, nxt, hid = lm.prefill(prompts=prompts)
        res = [lg.cpu().numpy(), hid.cpu().numpy()]
        for graph in (False, True, True):
            ids = torch.from_numpy(rng.integers(0, rows, 3).astype(np.int32))
            lg, _ = lm.step(ids=ids, graph=graph)
            res.append(lg.cpu().numpy())
        outs.append(res)
        rng = np.random.default_rng(62)
        prompts = [rng.integers(0, rows, T).astype(np.int32) for T in (4, 9, 2)]
    for a, b in zip(*outs):
        np.testing.assert_array_equal(a, b)
