"""GPU parity of the Fish s2 fast AR expansion (sxq_fish_fast_expand) and of the dual-AR
loop over the device engines (syrinx_amd.dualar), against the oracles of the reference's
FastAr::expand_batch (crates/syrinx-fish/src/s2/fast_ar.rs:170-224) and drive /
drive_batch (crates/syrinx-fish/src/common/dualar.rs:163-360).

Both levels of the decoder tests apply.  A draw is exact given its logits, so the token
sequence is checked by replaying the device's own steps (the same kernels on the same
inputs give the same logits) and drawing with the oracle sampler on those logits: every
code, semantic id, stop and rng state must then agree exactly.  The replayed logits are
checked against the oracle decoders, teacher-forced on the device's tokens, to the decode
step's tolerance.
"""
import numpy as np
import pytest
import torch

from syrinx_amd import decoder as D
from syrinx_amd import dualar as DA
from syrinx_amd.sampling import FishSampler, SamplingParams

from test_gpu_decoder import _build, _check, _Tally

pytestmark = pytest.mark.gpu

R = 128           # residual codebook size (fast vocab)
NCB = 6           # codes per frame
BEGIN = 200       # semantic ids BEGIN .. BEGIN + R - 1 of a 400-id slow vocab
GAMMA = 0x9E3779B97F4A7C15
PARAMS = SamplingParams(temperature=0.8, top_p=0.95, top_k=20, repetition_penalty=1.1, ras_win_size=3)


@pytest.fixture(scope="module")
def cuda():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a ROCm GPU")
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def model_oracle():
    import model
    return model


def _fast_cfg(max_batch):
    return D.fish_s2_fast_ar_config(n_layers=2, num_codebooks=NCB, residual_size=R, max_batch=max_batch, dim=256,
                                    n_heads=4, n_kv_heads=2, head_dim=64, intermediate=512)


def _slow_cfg(max_batch, dim=256):
    return D.fish_s2_slow_ar_config(n_layers=2, max_seq=40, max_batch=max_batch, vocab=400, dim=dim, n_heads=4,
                                    n_kv_heads=2, head_dim=64, intermediate=512, n_codebooks=NCB, codebook_size=R,
                                    semantic_begin=BEGIN, semantic_end=BEGIN + R - 1)


def _oracle_sampler(seed):
    import sampling as S
    p = PARAMS
    return S.FishSampler(seed, temperature=p.temperature, top_p=p.top_p, top_k=p.top_k,
                         repetition_penalty=p.repetition_penalty, ras_win_size=p.ras_win_size,
                         ras_high_temp=p.ras_high_temp, ras_high_top_p=p.ras_high_top_p)


def _u64(t):
    return [int(v) & ((1 << 64) - 1) for v in t.cpu().tolist()]


def _replay_fast(fast, hidden, first_codes, codes):
    """The device logits of positions 1..NCB-1 of one expansion, by plain steps."""
    fast.reset(hidden.shape[0])
    fast.step(embeds=hidden)
    out = []
    for cb in range(1, NCB):
        ids = torch.as_tensor(codes[:, cb - 1] if cb > 1 else first_codes, dtype=torch.int32)
        logits, _ = fast.step(ids=ids)
        out.append(logits.cpu().numpy())
    return out


def _oracle_fast_logits(model, cfg, W, hidden, codes):
    """Teacher-forced oracle logits of the same positions: [stream][cb - 1] -> (logits, margin)."""
    orc = model.OracleDecoder(cfg, W, 1)
    res = []
    for i in range(hidden.shape[0]):
        orc.reset(0)
        orc.step_one(0, embed=hidden[i])
        row = []
        for cb in range(1, NCB):
            lg = orc.step_one(0, frame=[int(codes[i, cb - 1])])
            row.append((lg, _Margin(orc.margin)))
        res.append(row)
    return res


class _Margin:
    def __init__(self, m):
        self.margin = m


@pytest.mark.parametrize("graph", [False, True])
def test_fast_expand_matches_replay_and_oracle(cuda, model_oracle, graph):
    n = 4
    cfg = _fast_cfg(n)
    fast, W = _build(cfg, cuda, 21, n, cls=D.FastAr)
    rng = np.random.default_rng(22)
    hidden_np = rng.standard_normal((n, cfg.dim)).astype(np.float32)
    hidden = torch.from_numpy(hidden_np).to(cuda)
    sem = torch.tensor([BEGIN + 7, BEGIN - 4, BEGIN + R + 9, BEGIN + 3], dtype=torch.int32, device=cuda)
    seeds = [101, 202, 303, 404]
    smp = FishSampler(seeds, PARAMS, semantic=(BEGIN, BEGIN + R - 1, 3), device=cuda)
    active = torch.tensor([1, 1, 1, 0], dtype=torch.int32, device=cuda)
    codes = fast.expand_batch(hidden, sem, smp, active=active, graph=graph).cpu().numpy()
    assert fast.lengths(n) == [NCB] * n
    # FastAr::first_code: clamp(tok - begin, 0, R - 1); a finished stream's codes are 0
    assert codes[:, 0].tolist() == [7, 0, R - 1, 0]
    assert (codes[3] == 0).all()
    assert _u64(smp.rng)[3] == 404  # no draw for the finished stream

    got = _replay_fast(fast, hidden, codes[:, 0], codes)
    for i in range(3):
        o = _oracle_sampler(seeds[i])
        want = [o.sample_codebook(got[cb - 1][i], []) for cb in range(1, NCB)]
        assert codes[i, 1:].tolist() == want, (i, codes[i], want)
        assert _u64(smp.rng)[i] == o.rng.state
    tally = _Tally()
    orc = _oracle_fast_logits(model_oracle, cfg, W, hidden_np, codes)
    for i in range(n):
        for cb in range(1, NCB):
            lg, m = orc[i][cb - 1]
            _check(got[cb - 1][i], m, lg, f"stream {i} codebook {cb}", tally)
    tally.mostly_tight()


def test_fast_expand_graph_replays_equal_eager(cuda):
    """The captured expansion, replayed on new hidden states with eager work and
    synchronisations between replays, gives the eager expansion's codes and rng states."""
    n = 2
    cfg = _fast_cfg(n)
    fast, _ = _build(cfg, cuda, 31, n, cls=D.FastAr)
    hidden = torch.empty((n, cfg.dim), device=cuda)
    sem = torch.tensor([BEGIN + 11, BEGIN + 90], dtype=torch.int32, device=cuda)
    sg = FishSampler([5, 6], PARAMS, semantic=(BEGIN, BEGIN + R - 1, 3), device=cuda)
    se = FishSampler([5, 6], PARAMS, semantic=(BEGIN, BEGIN + R - 1, 3), device=cuda)
    codes_g = torch.empty((n, NCB), dtype=torch.int32, device=cuda)
    gen = torch.Generator(device=cuda).manual_seed(32)
    for rep in range(4):
        hidden.copy_(torch.randn((n, cfg.dim), device=cuda, generator=gen))
        fast.expand_batch(hidden, sem, sg, codes=codes_g, graph=True)
        _ = torch.zeros(1000, device=cuda).sum().item()
        torch.cuda.synchronize()
        ce = fast.expand_batch(hidden, sem, se, graph=False)
        torch.cuda.synchronize()
        assert torch.equal(codes_g, ce), rep
        assert torch.equal(sg.rng, se.rng), rep


def test_fast_expand_argument_errors(cuda):
    cfg = _fast_cfg(2)
    fast = D.FastAr(cfg, device=cuda)
    smp = FishSampler([1, 2], PARAMS, device=cuda)
    h = torch.zeros((2, cfg.dim), device=cuda)
    sem = torch.zeros(2, dtype=torch.int32, device=cuda)
    with pytest.raises(RuntimeError, match="codes per frame"):
        fast.expand_batch(h, sem, smp, n_codes=NCB + 1)
    slow = D.DecoderLM(_slow_cfg(2), device=cuda)  # a frame-embedding engine is not a fast AR
    with pytest.raises(RuntimeError, match="dense table"):
        D.FastAr.expand_batch(slow, h, sem, smp, n_codes=NCB)


def _replay_drive(slow, fast, prompts, outs, n_frames):
    """Device logits / hiddens the drive saw, by plain steps on the drive's tokens."""
    n = len(prompts)
    slow.reset(n)
    logits, hidden = slow.prefill_batch(prompts)
    slow_logits, fast_logits, hid = [logits.cpu().numpy()], [], []
    for t in range(n_frames):
        frame = np.zeros((n, 1 + NCB), np.int32)
        for i in range(n):
            if t < outs[i].shape[1]:
                frame[i, 0] = outs[i][0, t] + BEGIN
                frame[i, 1:] = outs[i][:, t]
        h = hidden.reshape(n, -1).contiguous()
        hid.append(h.cpu().numpy())
        fast_logits.append(_replay_fast(fast, h, frame[:, 1], frame[:, 1:]))
        if t + 1 < n_frames:
            logits, hidden = slow.slow_step_batch(torch.from_numpy(frame))
            slow_logits.append(logits.cpu().numpy())
    return slow_logits, fast_logits, hid


# "project_in": a slow AR of width 512 over the 256-wide fast AR, joined by a Q4_K
# fast_project_in with bias (slow_ar.rs:230-243), as in the s2_pro() default geometry
# (a 1024-wide fast AR under the 2560-wide slow one, common/config.rs:213-226).
@pytest.mark.parametrize("variant", ["plain", "stop_from_run", "project_in"])
def test_drive_batch_matches_oracle_draws(cuda, model_oracle, variant):
    stop_from_run = variant == "stop_from_run"
    n, max_new = 2, 10
    scfg, fcfg = _slow_cfg(n, dim=512 if variant == "project_in" else 256), _fast_cfg(n)
    slow, WS = _build(scfg, cuda, 41, n, cls=D.SlowAr)
    fast, WF = _build(fcfg, cuda, 42, n, cls=D.FastAr)
    if variant == "project_in":
        from syrinx_amd import GgmlDType, QMatMul, QTensor
        rng_p = np.random.default_rng(44)
        wp = (rng_p.standard_normal((fcfg.dim, scfg.dim)) * 0.05).astype(np.float32)
        bp = (rng_p.standard_normal(fcfg.dim) * 0.02).astype(np.float32)
        qt = QTensor.quantize(torch.from_numpy(wp).to(cuda), GgmlDType.Q4K)
        slow.set_project_in(QMatMul.from_qtensor(qt), torch.from_numpy(bp))
        WS["project_in"] = qt.data().cpu().numpy().reshape(fcfg.dim, -1)
        WS["project_in_bias"] = bp
        assert slow.hidden_dim == fcfg.dim
    rng = np.random.default_rng(43)
    prompts = []
    for T in (5, 9):
        p = np.zeros((1 + NCB, T), np.int32)
        p[0] = rng.integers(0, scfg.vocab, T)
        p[1:] = rng.integers(0, R, (NCB, T))
        prompts.append(p)
    params = DA.DriveParams(max_new_frames=max_new, seed=77, sampling=PARAMS)
    if not stop_from_run:
        stop = 50  # outside the semantic range: the constraint's extra id
        outs = DA.drive_batch(slow, fast, prompts, stop, params)
    else:
        # stop ids inside the range keep the candidate set, so the draws of a run with
        # another such stop id agree up to it: stream 0 then stops at or before frame 2
        outs = DA.drive_batch(slow, fast, prompts, BEGIN + R - 1, params)
        assert outs[0].shape[1] >= 3
        stop = int(outs[0][0, 2].item()) + BEGIN
        outs = DA.drive_batch(slow, fast, prompts, stop, params)
        assert outs[0].shape[1] <= 2
    outs = [o.cpu().numpy() for o in outs]
    max_t = max(o.shape[1] for o in outs)
    n_iter = max_t + 1 if max_t < max_new else max_new  # loop passes, the last one all-stop or capped

    # sample i of the batch reproduces drive seeded seed + i (dualar.rs:244-252)
    for i in range(n):
        single = DA.drive(slow, fast, prompts[i], stop,
                          DA.DriveParams(max_new_frames=max_new, seed=77 + i, sampling=PARAMS)).cpu().numpy()
        np.testing.assert_array_equal(single, outs[i])

    sl, fl, hid = _replay_drive(slow, fast, prompts, outs, n_iter)
    for i in range(n):
        o = _oracle_sampler(77 + i)
        window = []
        T = outs[i].shape[1]
        for t in range(min(T + 1, n_iter)):
            sem = o.sample_semantic(sl[t][i], window, BEGIN, BEGIN + R - 1, stop)
            if t == T:  # the stream ended here: by a stop draw
                assert sem == stop, (i, t, sem)
                break
            assert sem == outs[i][0, t] + BEGIN, (i, t, sem)
            window = (window + [sem])[-PARAMS.ras_win_size:]
            for cb in range(1, NCB):
                assert o.sample_codebook(fl[t][cb - 1][i], []) == outs[i][cb, t], (i, t, cb)

    # the replayed logits against the oracle decoders, teacher-forced on the same tokens
    tally = _Tally()
    orc_slow = model_oracle.OracleDecoder(scfg, WS, n)
    for i in range(n):
        for tok in range(prompts[i].shape[1]):
            lg = orc_slow.step_one(i, frame=prompts[i][:, tok])
        _check(sl[0][i], orc_slow, lg, f"stream {i} prefill", tally)
        _check(hid[0][i], orc_slow, orc_slow.hidden, f"stream {i} prefill hidden")
        for t in range(1, n_iter):
            fr = np.zeros(1 + NCB, np.int32)
            if t - 1 < outs[i].shape[1]:
                fr[0] = outs[i][0, t - 1] + BEGIN
                fr[1:] = outs[i][:, t - 1]
            lg = orc_slow.step_one(i, frame=fr)
            _check(sl[t][i], orc_slow, lg, f"stream {i} frame {t}", tally)
            if t < outs[i].shape[1]:
                _check(hid[t][i], orc_slow, orc_slow.hidden, f"stream {i} frame {t} hidden")
    tally.mostly_tight()
