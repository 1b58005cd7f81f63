"""The device samplers (libsxq sxq_sample_*) against the oracle restatement of the
reference's samplers (oracle/sampling.py) on the same logits and seeds: every draw must
pick the same id, and the SplitMix64 states must advance identically (checked through
the ids of the following draws).  Plus the reference's distribution property (an
unbiased categorical draw), measured on the device."""
import numpy as np
import pytest
import torch

import sampling as S
from syrinx_amd.sampling import FishSampler, RasSampler, SamplingParams

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def cuda():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a ROCm GPU")
    return torch.device("cuda:0")


def _logits(rng, n, vocab, scale=3.0, ties=False):
    x = (rng.standard_normal((n, vocab)) * scale).astype(np.float32)
    if ties:  # blocks of equal values: the cut falls inside a tie, ordered by id
        x[:, ::7] = x[:, :1]
    return x


@pytest.mark.parametrize("ties", [False, True])
def test_semantic_draws_equal_oracle(cuda, ties):
    """Slow-AR semantic draws at the Qwen3-4B vocabulary (155776) with the s2 semantic
    range and stop id, RAS window on the device, 12 consecutive draws of 8 streams."""
    n, vocab = 8, 155776
    begin, end, stop = 151678, 155773, 151645
    params = SamplingParams()
    dev = FishSampler([42 + i for i in range(n)], params, (begin, end, stop), device=cuda)
    refs = [S.FishSampler(42 + i) for i in range(n)]
    windows = [[] for _ in range(n)]
    rng = np.random.default_rng(1)
    for step in range(12):
        x = _logits(rng, n, vocab, 1.0, ties)
        if step % 3 == 2:  # make repeats likely: peak a recent id so RAS triggers
            for i in range(n):
                if windows[i]:
                    x[i, windows[i][-1]] += 6.0
        got = dev.sample_semantic(torch.from_numpy(x).to(cuda)).cpu().numpy()
        for i in range(n):
            want = refs[i].sample_semantic(x[i], windows[i], begin, end, stop)
            assert got[i] == want, (step, i, got[i], want)
            if want != stop:
                windows[i].append(want)
                windows[i] = windows[i][-params.ras_win_size:]
    w = dev.window.cpu().numpy()
    L = dev.window_len.cpu().numpy()
    for i in range(n):
        assert list(w[i][:L[i]]) == windows[i]


def test_codebook_draws_with_repetition_penalty_equal_oracle(cuda):
    n, vocab = 16, 4096
    params = SamplingParams(temperature=0.8, top_p=0.7, top_k=40, repetition_penalty=1.3)
    dev = FishSampler([7 * i + 1 for i in range(n)], params, device=cuda)
    refs = [S.FishSampler(7 * i + 1, temperature=0.8, top_p=0.7, top_k=40, repetition_penalty=1.3) for i in range(n)]
    rng = np.random.default_rng(2)
    for step in range(10):
        x = _logits(rng, n, vocab, 2.0, ties=(step % 2 == 1))
        recent = rng.integers(0, vocab, (n, 6)).astype(np.int32)
        recent[:, 5] = recent[:, 4]  # a duplicate id is penalized twice
        got = dev.sample_codebook(torch.from_numpy(x).to(cuda), torch.from_numpy(recent).to(cuda)).cpu().numpy()
        for i in range(n):
            assert got[i] == refs[i].sample_codebook(x[i], list(recent[i])), (step, i)


# top_k 0 is unbounded (common/sampling.rs:50-52); caps above 64 keep more candidates than
# one wave sorts.  Flat logits keep thousands of ids under top_p, peaked ones a few (the
# staged wave path), ties put the cut inside a run of equal logits, top_p >= 1 keeps all.
WIDE = [
    # (top_k, top_p, logit scale, ties)
    (0, 0.9, 0.3, False),
    (0, 0.9, 0.3, True),
    (0, 0.7, 3.0, False),    # peaked: fewer than 64 kept
    (200, 0.9, 0.3, False),  # the cap binds before top_p
    (1000, 1.0, 0.5, True),  # top_p keeps everything, the cap cuts inside ties
    (0, 1.5, 0.5, False),    # every id kept
]


@pytest.mark.parametrize("top_k,top_p,scale,ties", WIDE)
def test_codebook_draws_unbounded_top_k_equal_oracle(cuda, top_k, top_p, scale, ties):
    n, vocab = 8, 4096
    params = SamplingParams(temperature=0.9, top_p=top_p, top_k=top_k, repetition_penalty=1.2)
    dev = FishSampler([31 * i + 5 for i in range(n)], params, device=cuda)
    refs = [S.FishSampler(31 * i + 5, temperature=0.9, top_p=top_p, top_k=top_k, repetition_penalty=1.2)
            for i in range(n)]
    rng = np.random.default_rng(11)
    for step in range(6):
        x = _logits(rng, n, vocab, scale, ties)
        recent = rng.integers(0, vocab, (n, 4)).astype(np.int32)
        got = dev.sample_codebook(torch.from_numpy(x).to(cuda), torch.from_numpy(recent).to(cuda)).cpu().numpy()
        for i in range(n):
            assert got[i] == refs[i].sample_codebook(x[i], list(recent[i])), (step, i)
    np.testing.assert_array_equal(dev.rng.cpu().numpy().astype(np.uint64),
                                  np.array([r.rng.state for r in refs], np.uint64))


@pytest.mark.parametrize("top_k,scale", [(0, 0.2), (0, 2.0), (500, 0.2)])
def test_semantic_draws_unbounded_top_k_equal_oracle(cuda, top_k, scale):
    """The slow-AR draw over the 155776-id vocabulary with the 4096-id semantic range: an
    unbounded (or 500) cap keeps ~3500 semantic ids of flat logits under top_p 0.9."""
    n, vocab = 4, 155776
    begin, end, stop = 151678, 155773, 151645
    params = SamplingParams(top_k=top_k)
    dev = FishSampler([9 + i for i in range(n)], params, (begin, end, stop), device=cuda)
    refs = [S.FishSampler(9 + i, top_k=top_k) for i in range(n)]
    windows = [[] for _ in range(n)]
    rng = np.random.default_rng(12)
    for step in range(6):
        x = _logits(rng, n, vocab, scale)
        if step % 2 == 1:
            for i in range(n):
                if windows[i]:
                    x[i, windows[i][-1]] += 3.0
        got = dev.sample_semantic(torch.from_numpy(x).to(cuda)).cpu().numpy()
        for i in range(n):
            want = refs[i].sample_semantic(x[i], windows[i], begin, end, stop)
            assert got[i] == want, (step, i, got[i], want)
            if want != stop:
                windows[i] = (windows[i] + [want])[-params.ras_win_size:]
    np.testing.assert_array_equal(dev.rng.cpu().numpy().astype(np.uint64),
                                  np.array([r.rng.state for r in refs], np.uint64))


@pytest.mark.parametrize("ignore_eos", [False, True])
def test_cosyvoice_ras_draws_equal_oracle(cuda, ignore_eos):
    """CosyVoice2 speech vocabulary (6564, stop ids 6561..6563): log_softmax, nucleus
    (top_p 0.8, top_k 25), the repetition fallback to the full distribution."""
    n, vocab = 12, 6564
    dev = RasSampler([100 + i for i in range(n)], device=cuda)
    refs = [S.SplitMix64(100 + i) for i in range(n)]
    hist = [[] for _ in range(n)]
    rng = np.random.default_rng(3)
    for step in range(15):
        x = _logits(rng, n, vocab, 2.0)
        x[:, 6561:6564] += 4.0 * (step % 4 == 0)
        if step % 2 == 1:
            for i in range(n):
                if hist[i]:
                    x[i, hist[i][-1]] += 8.0  # repeats: the fallback draw follows
        xt = torch.from_numpy(x).to(cuda)
        got = dev.sample(xt, ignore_eos).cpu().numpy()
        for i in range(n):
            want = S.ras_sampling(x[i], hist[i], refs[i], ignore_eos, 6561, 6564)
            assert got[i] == want, (step, i, got[i], want)
            if not 6561 <= want < 6564:
                hist[i] = (hist[i] + [want])[-10:]
        # the row now holds log_softmax (stop ids -inf when ignored)
        lp = xt.cpu().numpy()
        want_lp = S.log_softmax_vec(x[0])
        if ignore_eos:
            want_lp[6561:6564] = -np.inf
        np.testing.assert_allclose(lp[0], want_lp, rtol=0, atol=2e-6)


def test_device_draws_are_an_unbiased_categorical(cuda):
    """The reference's multinomial property (tests/real_cv3_multinomial.rs) on the device:
    4096 streams with different seeds draw from the same 5-way row."""
    n = 4096
    probs = np.array([0.05, 0.10, 0.20, 0.50, 0.15], np.float32)
    x = np.tile(np.log(probs)[None, :], (n, 1)).astype(np.float32)
    params = SamplingParams(temperature=1.0, top_p=1.0, top_k=5, repetition_penalty=1.0)
    counts = np.zeros(5)
    dev = FishSampler(list(range(1, n + 1)), params, device=cuda)
    for _ in range(10):
        got = dev.sample_codebook(torch.from_numpy(x).to(cuda)).cpu().numpy()
        counts += np.bincount(got, minlength=5)
    f = counts / counts.sum()
    assert np.abs(f - probs).max() < 1e-2, f


def test_active_flags_freeze_finished_streams(cuda):
    """drive_batch's `finished` on the device: a stream whose flag is 0 draws nothing (rng
    kept, token 0), a semantic draw of the stop id clears the stream's flag, and codebook
    draws read the flags without changing them."""
    n, vocab = 3, 300
    begin, end, stop = 100, 199, 250
    params = SamplingParams()
    dev = FishSampler([7, 8, 9], params, (begin, end, stop), device=cuda)
    x = np.full((n, vocab), -30.0, np.float32)
    x[0, stop] = 20.0   # stream 0 draws the stop id
    x[1, 120] = 20.0
    x[2, 150] = 20.0
    active = torch.tensor([1, 0, 1], dtype=torch.int32, device=cuda)
    rng0 = dev.rng.clone()
    got = dev.sample_semantic(torch.from_numpy(x).to(cuda), active=active).cpu().numpy()
    assert got.tolist() == [stop, 0, 150]
    assert active.cpu().tolist() == [0, 0, 1]
    adv = (dev.rng - rng0).cpu().tolist()
    assert adv[1] == 0 and adv[0] == adv[2] != 0  # two uniforms each for streams 0 and 2
    assert dev.window_len.cpu().tolist() == [0, 0, 1]  # a stop is not pushed into the window
    before = dev.rng.clone()
    y = np.zeros((n, 64), np.float32)
    y[:, 5] = 30.0
    codes = dev.sample_codebook(torch.from_numpy(y).to(cuda), active=active).cpu().numpy()
    assert codes.tolist() == [0, 0, 5]
    assert active.cpu().tolist() == [0, 0, 1]
    assert torch.equal(dev.rng[:2], before[:2]) and not torch.equal(dev.rng[2:], before[2:])
