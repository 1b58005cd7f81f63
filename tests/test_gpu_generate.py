"""GPU parity of the CosyVoice generation loops on the device (syrinx_amd.generate)
against the oracle of Qwen2Lm::generate (crates/syrinx-lm/src/cv2/generate.rs:136-163)
and Cv3Lm::generate / generate_instruct (crates/syrinx-lm/src/cv3/generate.rs:14-101).

As for the Fish drive loop: a draw is exact given its logits, so the device's tokens
are checked by replaying the engine's own steps on those tokens (the same kernels give
the same logits) and drawing with the oracle sampler (oracle/sampling.py) on them --
every token, the stop, and the final SplitMix64 state must agree exactly.  The replayed
logits are checked against the oracle decoder teacher-forced on the same step-0 input and
tokens, to the decode step's tolerance.  The models are random (two layers of the
Qwen2-0.5B shape, Q8_0); their control-id logits are raised so that the loops stop
within a few steps after min_len.
"""
import numpy as np
import pytest
import torch

import sampling as S
from syrinx_amd import GgmlDType, QMatMul, QTensor
from syrinx_amd import decoder as D
from syrinx_amd.embedding import QEmbed
from syrinx_amd.generate import COSYVOICE2, COSYVOICE3, CosyVoiceLm
from syrinx_amd.sampling import RasSampler

from test_gpu_decoder import _build, _check, _Tally

pytestmark = pytest.mark.gpu

TEXT_ROWS = 500


@pytest.fixture(scope="module")
def cuda():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a ROCm GPU")
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def model_oracle():
    import model
    return model


def _setup(variant, cuda, seed, n_layers=2, max_seq=96):
    make = D.cosyvoice2_lm_config if variant is COSYVOICE2 else D.cosyvoice3_lm_config
    cfg = make(n_layers=n_layers, max_seq=max_seq, dtype=GgmlDType.Q8_0)
    lm, W = _build(cfg, cuda, seed, 1, cls=D.Qwen2Lm)
    rng = np.random.default_rng(seed + 1)
    if variant is COSYVOICE2:  # the three stop ids' bias raised: each ~11 % of the mass
        b = W["head_bias"].copy()
        b[variant.stop_begin:variant.stop_end] += 7.0
        lm.set_vector(-1, D.HEAD_BIAS, torch.from_numpy(b))
        W["head_bias"] = b
    else:  # bias-free head: the 200 control rows scaled up instead
        w = (rng.standard_normal((cfg.vocab, cfg.dim)) * 0.02).astype(np.float32)
        w[variant.stop_begin:] *= 6.0
        qt = QTensor.quantize(torch.from_numpy(w).to(cuda), GgmlDType.Q8_0)
        lm.set_linear(-1, D.HEAD, QMatMul.from_qtensor(qt))
        W["head"] = qt.data().cpu().numpy().reshape(cfg.vocab, -1)
    text = torch.from_numpy((rng.standard_normal((TEXT_ROWS, cfg.dim)) * 0.5).astype(np.float32)).to(cuda)
    llm = torch.from_numpy((rng.standard_normal((2, cfg.dim)) * 0.5).astype(np.float32)).to(cuda)
    speech = torch.from_numpy(W["embed"]).to(cuda)
    cv = CosyVoiceLm(lm, text, speech, llm if variant is COSYVOICE2 else None, variant)
    return cv, cfg, W


def _replay(cv, lm_input0, toks):
    """The engine's logits for every sampled step of a generation over `toks`."""
    lm = cv.lm
    lm.reset(1)
    logits, _, _ = lm.prefill(embeds=[lm_input0])
    seen = [logits[0].cpu().numpy()]
    for t in toks:
        lg, _ = lm.step(ids=torch.tensor([[t]], dtype=torch.int32))
        seen.append(lg[0].cpu().numpy())
    return seen


def _check_loop(cv, lm_input0, toks, smp, seed, min_len, max_len):
    v = cv.v
    assert all(not (v.stop_begin <= t < v.stop_end) for t in toks)
    assert len(toks) <= max_len
    stopped = len(toks) < max_len
    assert len(toks) >= min_len or not stopped  # no stop is drawn while i < min_len
    seen = _replay(cv, lm_input0, toks)
    rng = S.SplitMix64(seed)
    out = []
    for i in range(len(toks) + (1 if stopped else 0)):
        top = S.ras_sampling(seen[i], out, rng, i < min_len, v.stop_begin, v.stop_end)
        if i == len(toks):
            assert v.stop_begin <= top < v.stop_end, (i, top)
            break
        assert top == toks[i], (i, top, toks[i])
        out.append(top)
    assert int(smp.rng.cpu().numpy()[0]) & ((1 << 64) - 1) == rng.state, "rng state"
    hist = smp.decoded.cpu().numpy()[0][: int(smp.decoded_len.cpu().numpy()[0])]
    assert list(hist) == toks[-len(hist):] if len(hist) else not toks
    return seen, stopped


@pytest.mark.parametrize("variant", [COSYVOICE2, COSYVOICE3], ids=["cv2", "cv3"])
@pytest.mark.parametrize("graph", [True, False])
def test_generate_matches_oracle(cuda, model_oracle, variant, graph):
    cv, cfg, W = _setup(variant, cuda, 61)
    text = [5, 17, 299, 3, 250, 41, 7]
    prompt = [12, 6000, 33, 1005]
    min_len, max_len, seed = 4, 30, 1234
    smp = RasSampler([seed], eos=(variant.stop_begin, variant.stop_end), device=cuda)
    toks = cv.generate(text, prompt, min_len, max_len, seed, graph=graph, sampler=smp)
    lm_input0 = cv.build_lm_input(text, prompt)
    assert lm_input0.shape == (1 + len(text) + 1 + len(prompt), cfg.dim)
    seen, stopped = _check_loop(cv, lm_input0, toks, smp, seed, min_len, max_len)
    assert stopped, "the raised control logits should stop the loop within max_len"
    # the step-0 input: sos, text rows, task_id, prompt-speech rows of the right tables
    e0 = lm_input0.cpu().numpy()
    sos_tab = cv.llm if variant is COSYVOICE2 else cv.speech
    np.testing.assert_array_equal(e0[0], sos_tab[variant.sos].cpu().numpy())
    np.testing.assert_array_equal(e0[1:1 + len(text)], cv.text[text].cpu().numpy())
    np.testing.assert_array_equal(e0[1 + len(text)], sos_tab[variant.task_id].cpu().numpy())
    np.testing.assert_array_equal(e0[2 + len(text):], W["embed"][prompt])
    # the replayed logits against the oracle decoder, teacher-forced on the same inputs
    orc = model_oracle.OracleDecoder(cfg, W, 1)
    tally = _Tally()
    for row in e0:
        lg = orc.step_one(0, embed=row)
    _check(seen[0], orc, lg, f"{variant.name} step 0 (prefill)", tally)
    for i, t in enumerate(toks):
        _check(seen[i + 1], orc, orc.step_one(0, frame=[t]), f"{variant.name} step {i + 1}", tally)
    tally.mostly_tight()


def test_generate_equals_oracle_loop_end_to_end(cuda, model_oracle):
    """The oracle's own loop (oracle/cv_generate.py: its model and its sampler) and the
    device loop on the same model and seed.  Both draw the same token from the same
    uniform whenever their logits agree to the tight bound; a step where the oracle model
    and the engine put an activation on different sides of a Q8 rounding tie may draw
    differently, and the sequences are compared up to the first such step."""
    import cv_generate as G
    from test_gpu_decoder import LOGIT_RTOL, _rel
    cv, cfg, W = _setup(COSYVOICE2, cuda, 62)
    text, prompt = [9, 8, 7, 6, 5], [100, 200]
    smp = RasSampler([99], eos=(6561, 6564), device=cuda)
    toks = cv.generate(text, prompt, 3, 20, 99, sampler=smp)
    orc = model_oracle.OracleDecoder(cfg, W, 1)
    want, rng, want_seen = G.generate(orc, cv.build_lm_input(text, prompt).cpu().numpy(), 3, 20, 99, 6561, 6564,
                                      stop=lambda t: t in (6561, 6562, 6563))
    got_seen = _replay(cv, cv.build_lm_input(text, prompt), toks)
    compared = 0
    for i in range(min(len(got_seen), len(want_seen))):
        if _rel(got_seen[i], want_seen[i]) > LOGIT_RTOL:
            break  # a Q8 tie flip: the draws may part from here
        compared += 1
        # step i drew toks[i] on the device (or the stop, at i == len(toks)), want[i] on the oracle
        g = toks[i] if i < len(toks) else "stop"
        w = want[i] if i < len(want) else "stop"
        assert g == w, (i, g, w)
    if compared == min(len(got_seen), len(want_seen)):  # no flip anywhere: the whole run agrees
        assert toks == want
        assert int(smp.rng.cpu().numpy()[0]) & ((1 << 64) - 1) == rng.state
    print(f"cv2 loop: {len(toks)} device tokens, {len(want)} oracle tokens, {compared} steps compared")
    assert compared >= 2


def test_generate_to_max_len_and_min_len_mask(cuda):
    """min_len = max_len masks every stop id on every step: exactly max_len tokens, none a
    control id (CosyVoice3: the whole 6561..6760 range masked, cv3/sampling.rs:123-138)."""
    cv, cfg, W = _setup(COSYVOICE3, cuda, 63)
    smp = RasSampler([5], eos=(6561, 6761), device=cuda)
    toks = cv.generate([1, 2, 3], [], 12, 12, 5, sampler=smp)
    assert len(toks) == 12 and all(t < 6561 for t in toks)
    _check_loop(cv, cv.build_lm_input([1, 2, 3], []), toks, smp, 5, 12, 12)


def test_generate_instruct_cv3(cuda):
    """Cv3Lm::generate_instruct: [sos, embed_tokens(instruct), embed_tokens(text), task_id]
    (cv3/lm.rs:93-132) and the same loop."""
    cv, cfg, W = _setup(COSYVOICE3, cuda, 64)
    instruct, text = [400, 401, 402], [10, 11, 12, 13]
    smp = RasSampler([8], eos=(6561, 6761), device=cuda)
    toks = cv.generate_instruct(instruct, text, 2, 25, 8, sampler=smp)
    e0 = cv.build_lm_input_instruct(instruct, text)
    assert e0.shape[0] == 1 + len(instruct) + len(text) + 1
    np.testing.assert_array_equal(e0[1:4].cpu().numpy(), cv.text[instruct].cpu().numpy())
    _check_loop(cv, e0, toks, smp, 8, 2, 25)


def test_generate_with_quantized_tables(cuda):
    """The quantized build's tables (per-row int4 QEmbeds, cv2/quant.rs:38-89): the prompt
    is gathered from them and every fed-back token from the engine's int4 speech table."""
    cv, cfg, W = _setup(COSYVOICE2, cuda, 65)
    qs = QEmbed.quantize(cv.speech, 4)
    cv.lm.set_embed_quantized(qs)
    cv = CosyVoiceLm(cv.lm, QEmbed.quantize(cv.text, 4), qs, QEmbed.quantize(cv.llm, 4), COSYVOICE2)
    smp = RasSampler([3], eos=(6561, 6564), device=cuda)
    toks = cv.generate([4, 5, 6], [7, 8], 2, 20, 3, sampler=smp)
    _check_loop(cv, cv.build_lm_input([4, 5, 6], [7, 8]), toks, smp, 3, 2, 20)


def test_generate_argument_errors(cuda):
    cv, cfg, W = _setup(COSYVOICE2, cuda, 66, n_layers=1, max_seq=16)
    with pytest.raises(ValueError, match="exceed the cache"):
        cv.generate(list(range(10)), [1, 2, 3], 0, 10, 1)
    with pytest.raises(ValueError, match="llm_embedding"):
        CosyVoiceLm(cv.lm, cv.text, cv.speech, None, COSYVOICE2)
