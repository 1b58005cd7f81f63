"""Checkpoint ingest on the GPU (syrinx_amd/ingest.py) from synthetic safetensors files in
the reference's layouts, checked against the oracle:

* CosyVoice2 Qwen2Lm::load_quantized (crates/syrinx-lm/src/cv2/load.rs:68-122): placement
  (lm_head dropped, embedding tables per-row int4, aligned 2-D Q4_0, the rest f16 / f32),
  the footprint arithmetic, bf16 / f16 sources cast to f32 before quantizing (a forward
  is bit-identical to the oracle's product with the oracle's blocks), and the wired engine's
  prompt + step logits against the oracle model of the same checkpoint.
* Fish s2 load_lm (crates/syrinx-fish/src/s2/load.rs:32-51) from two bf16 shards with an
  index: the slow and fast engines it builds against the oracle model, role by role as the
  reference's forward reads the names (s2/nn.rs, slow_ar.rs, fast_ar.rs).
"""
import json

import numpy as np
import pytest
import torch

import embed as E
from syrinx_amd import GgmlDType
from syrinx_amd import decoder as D
from syrinx_amd import ingest as I

from test_gpu_decoder import _check, _Tally

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def cuda():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a ROCm GPU")
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def model_oracle():
    import model
    return model


def _save(path, tensors):
    from safetensors.torch import save_file
    save_file({k: v.contiguous() for k, v in tensors.items()}, str(path))


def _rand(g, *shape, std=0.02, mean=0.0, dtype=torch.float32):
    return (mean + torch.randn(*shape, generator=g) * std).to(dtype)


def _f32(t):
    return t.to(torch.float32).numpy()


# ----------------------------------------------------------------------------- CosyVoice2
H, NH, NKV, HD, INTER, L, SPEECH, TEXT = 128, 2, 1, 64, 256, 2, 300, 500


def _cv2_checkpoint(path):
    g = torch.Generator().manual_seed(7)
    t = {}
    pre = "llm.model.model.layers"
    for l in range(L):
        p = f"{pre}.{l}"
        t[f"{p}.self_attn.q_proj.weight"] = _rand(g, NH * HD, H, dtype=torch.bfloat16)
        t[f"{p}.self_attn.k_proj.weight"] = _rand(g, NKV * HD, H, dtype=torch.bfloat16)
        t[f"{p}.self_attn.v_proj.weight"] = _rand(g, NKV * HD, H, dtype=torch.float16)
        t[f"{p}.self_attn.o_proj.weight"] = _rand(g, H, NH * HD)
        t[f"{p}.self_attn.q_proj.bias"] = _rand(g, NH * HD)
        t[f"{p}.self_attn.k_proj.bias"] = _rand(g, NKV * HD)
        t[f"{p}.self_attn.v_proj.bias"] = _rand(g, NKV * HD)
        t[f"{p}.mlp.gate_proj.weight"] = _rand(g, INTER, H, dtype=torch.bfloat16)
        t[f"{p}.mlp.up_proj.weight"] = _rand(g, INTER, H, dtype=torch.bfloat16)
        t[f"{p}.mlp.down_proj.weight"] = _rand(g, H, INTER, dtype=torch.bfloat16)
        t[f"{p}.input_layernorm.weight"] = _rand(g, H, std=0.1, mean=1.0)
        t[f"{p}.post_attention_layernorm.weight"] = _rand(g, H, std=0.1, mean=1.0)
    t["llm.model.model.norm.weight"] = _rand(g, H, std=0.1, mean=1.0)
    t["llm.model.model.embed_tokens.weight"] = _rand(g, TEXT, H, std=0.5, dtype=torch.float16)
    t["llm.model.lm_head.weight"] = _rand(g, TEXT, H)
    t["llm_embedding.weight"] = _rand(g, 2, H, std=0.5)
    t["speech_embedding.weight"] = _rand(g, SPEECH + 3, H, std=0.5, dtype=torch.bfloat16)
    t["llm_decoder.weight"] = _rand(g, SPEECH, H)
    t["llm_decoder.bias"] = _rand(g, SPEECH)
    t["odd.weight"] = _rand(g, 16, 80)      # 2-D, inner dim not a multiple of 32: dense f16
    _save(path, t)
    return t


def test_cv2_load_quantized_placement_and_footprint(cuda, tmp_path, ora):
    src = _cv2_checkpoint(tmp_path / "llm.safetensors")
    bag = I.load_cv2_quantized(str(tmp_path / "llm.safetensors"), device=cuda)
    assert not any("lm_head" in k for k in list(bag.qmm) + list(bag.w) + list(bag.qembed))
    assert set(bag.qembed) == set(I.CV2_EMBED_TABLES)
    assert all(e.scheme == E.INT4 for e in bag.qembed.values())
    assert bag.w["odd.weight"].dtype == torch.float16
    assert bag.w["llm_decoder.bias"].dtype == torch.float32
    aligned = [k for k, v in src.items() if v.dim() == 2 and v.shape[1] % 32 == 0 and I.cv2_policy(k, v.shape) == "qmm"]
    assert sorted(bag.qmm) == sorted(aligned)
    fp = bag.footprint()
    assert fp.n_quantized == len(aligned)
    assert fp.quant_bytes == sum(src[k].shape[0] * (src[k].shape[1] // 32) * 18 for k in aligned)
    assert fp.embed_bytes == sum(src[k].shape[0] * (src[k].shape[1] // 2 + 4) for k in I.CV2_EMBED_TABLES)
    assert fp.dense_bytes == sum(v.numel() * (2 if k == "odd.weight" else 4) for k, v in src.items()
                                 if I.cv2_policy(k, v.shape) in ("f16", "f32"))
    assert bag.dense_breakdown()[0][1] >= bag.dense_breakdown()[-1][1]
    # bf16 / f16 sources: cast to f32, then Candle's from_float (the oracle's bytes)
    rng = np.random.default_rng(3)
    for k in ("llm.model.model.layers.0.self_attn.q_proj.weight", "llm.model.model.layers.1.self_attn.v_proj.weight",
              "llm.model.model.layers.0.mlp.down_proj.weight"):
        w = _f32(src[k])
        x = rng.standard_normal((3, w.shape[1])).astype(np.float32)
        got = bag.qmm[k].forward(torch.from_numpy(x).to(cuda)).cpu().numpy()
        want = ora.matmul(ora.Q4_0, x, ora.quantize(ora.Q4_0, w))
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    # the embedding tables: the oracle's per-row int4 codes of the f32-cast table
    q, s, _ = E.quantize(_f32(src["speech_embedding.weight"]), E.INT4)
    np.testing.assert_array_equal(bag.qembed["speech_embedding.weight"].q.cpu().numpy(), q)
    np.testing.assert_array_equal(bag.qembed["speech_embedding.weight"].scale.cpu().numpy(), s)


def test_cv2_engine_from_checkpoint_matches_oracle(cuda, tmp_path, ora, model_oracle):
    src = _cv2_checkpoint(tmp_path / "llm.safetensors")
    bag = I.load_cv2_quantized(str(tmp_path / "llm.safetensors"), device=cuda)
    lm = I.cv2_engine(bag, max_seq=32, max_batch=1, device=cuda)
    c = lm.cfg
    assert (c.n_layers, c.dim, c.n_heads, c.n_kv_heads, c.intermediate, c.vocab, c.embed_rows) == (
        L, H, NH, NKV, INTER, SPEECH, SPEECH + 3)
    # the oracle model of the same checkpoint, by the reference's names (cv2/mod.rs:223-285,
    # cv2/attention.rs:15-33): gate_proj = w1, up_proj = w3, down_proj = w2
    pre = "llm.model.model.layers"
    qz = lambda k: ora.quantize(ora.Q4_0, _f32(src[k]))  # noqa: E731
    W = {}
    for l in range(L):
        p = f"{pre}.{l}"
        W[("wqkv", l)] = np.concatenate([qz(f"{p}.self_attn.{x}_proj.weight") for x in "qkv"])
        W[("bqkv", l)] = np.concatenate([_f32(src[f"{p}.self_attn.{x}_proj.bias"]) for x in "qkv"])
        W[("wo", l)] = qz(f"{p}.self_attn.o_proj.weight")
        W[("w1", l)] = qz(f"{p}.mlp.gate_proj.weight")
        W[("w3", l)] = qz(f"{p}.mlp.up_proj.weight")
        W[("w2", l)] = qz(f"{p}.mlp.down_proj.weight")
        W[("attn_norm", l)] = _f32(src[f"{p}.input_layernorm.weight"])
        W[("ffn_norm", l)] = _f32(src[f"{p}.post_attention_layernorm.weight"])
    W["head"] = qz("llm_decoder.weight")
    W["head_bias"] = _f32(src["llm_decoder.bias"])
    W["final_norm"] = _f32(src["llm.model.model.norm.weight"])
    q, s, sch = E.quantize(_f32(src["speech_embedding.weight"]), E.INT4)
    W["embed"] = E.gather(q, s, sch, H, np.arange(SPEECH + 3))
    orc = model_oracle.OracleDecoder(c, W, 1)
    prompt = np.array([5, 17, 299, 302, 0, 150], np.int32)
    lm.reset(1)
    lg, _, _ = lm.prefill(prompts=[prompt])
    for tok in prompt:
        want = orc.step_one(0, frame=[int(tok)])
    tally = _Tally()
    _check(lg[0].cpu().numpy(), orc, want, "cv2 prompt", tally)
    for tok in (42, 7):
        lg, _ = lm.step(ids=torch.tensor([tok], dtype=torch.int32))
        _check(lg[0].cpu().numpy(), orc, orc.step_one(0, frame=[tok]), f"cv2 step {tok}", tally)
    tally.mostly_tight()


# ----------------------------------------------------------------------------- Fish s2
FD, FNH, FNKV, FI, FV, R, NCB, BEGIN = 256, 4, 2, 512, 400, 128, 6, 200


SD_FULL = 512  # the "full" variant's slow width (its fast AR stays FD wide, joined by fast_project_in)


def _fish_checkpoint(d, variant="plain"):
    """A sharded s2 checkpoint.  "full": the slow stack also carries wqkv.bias and
    wo.bias, an untied text_model.lm_head, and a fast AR narrower than the slow AR
    behind fast_project_in (weight and bias) -- every variant the reference's loader
    detects from the tensors (slow_ar.rs:86-98, :213-243)."""
    g = torch.Generator().manual_seed(11)
    bf = torch.bfloat16
    full = variant == "full"
    SD = SD_FULL if full else FD
    t = {}
    for base, n, qk, D_ in (("text_model.model.layers", 2, True, SD), ("audio_decoder.layers", 2, False, FD)):
        for l in range(n):
            p = f"{base}.{l}"
            t[f"{p}.attention.wqkv.weight"] = _rand(g, (FNH + 2 * FNKV) * HD, D_, dtype=bf)
            t[f"{p}.attention.wo.weight"] = _rand(g, D_, FNH * HD, dtype=bf)
            t[f"{p}.feed_forward.w1.weight"] = _rand(g, FI, D_, dtype=bf)
            t[f"{p}.feed_forward.w3.weight"] = _rand(g, FI, D_, dtype=bf)
            t[f"{p}.feed_forward.w2.weight"] = _rand(g, D_, FI, dtype=bf)
            t[f"{p}.attention_norm.weight"] = _rand(g, D_, std=0.1, mean=1.0, dtype=bf)
            t[f"{p}.ffn_norm.weight"] = _rand(g, D_, std=0.1, mean=1.0, dtype=bf)
            if qk:
                t[f"{p}.attention.q_norm.weight"] = _rand(g, HD, std=0.1, mean=1.0, dtype=bf)
                t[f"{p}.attention.k_norm.weight"] = _rand(g, HD, std=0.1, mean=1.0, dtype=bf)
            if full and qk:
                t[f"{p}.attention.wqkv.bias"] = _rand(g, (FNH + 2 * FNKV) * HD, std=0.05, dtype=bf)
                t[f"{p}.attention.wo.bias"] = _rand(g, D_, std=0.05, dtype=bf)
    t["text_model.model.embeddings.weight"] = _rand(g, FV, SD, dtype=bf)
    t["text_model.model.norm.weight"] = _rand(g, SD, std=0.1, mean=1.0, dtype=bf)
    if full:
        t["text_model.lm_head.weight"] = _rand(g, FV, SD, dtype=bf)
        t["fast_project_in.weight"] = _rand(g, FD, SD, std=0.05, dtype=bf)
        t["fast_project_in.bias"] = _rand(g, FD, std=0.05, dtype=bf)
    t["audio_decoder.embeddings.weight"] = _rand(g, R, FD, std=0.5, dtype=bf)
    t["audio_decoder.codebook_embeddings.weight"] = _rand(g, NCB * R, SD, std=0.5, dtype=bf)
    t["audio_decoder.norm.weight"] = _rand(g, FD, std=0.1, mean=1.0, dtype=bf)
    t["audio_decoder.output.weight"] = _rand(g, R, FD, dtype=bf)
    t["audio_tower.conv.weight"] = _rand(g, 4, 4)  # multimodal encoders are dropped
    keys = sorted(t)
    shards = {"model-00001-of-00002.safetensors": keys[::2], "model-00002-of-00002.safetensors": keys[1::2]}
    for f, ks in shards.items():
        _save(d / f, {k: t[k] for k in ks})
    (d / "model.safetensors.index.json").write_text(json.dumps({"weight_map": {k: f for f, ks in shards.items()
                                                                                for k in ks}}))
    return t


@pytest.mark.parametrize("variant", ["plain", "full"])
def test_fish_engines_from_sharded_checkpoint_match_oracle(cuda, tmp_path, ora, model_oracle, variant):
    src = _fish_checkpoint(tmp_path, variant)
    full = variant == "full"
    SD = SD_FULL if full else FD
    w = I.load_fish_lm(str(tmp_path), device=cuda)
    assert "audio_tower.conv.weight" not in w and all(v.dtype == torch.float32 for v in w.values())
    slow, fast = I.fish_engines(w, n_codebooks=NCB, semantic_begin=BEGIN, semantic_end=BEGIN + R - 1, max_seq=16,
                                max_batch=1, dtype=GgmlDType.Q4K, device=cuda)
    assert (slow.cfg.n_layers, slow.cfg.dim, slow.cfg.n_heads, slow.cfg.n_kv_heads, slow.cfg.head_dim,
            slow.cfg.vocab, slow.cfg.codebook_size, slow.cfg.qk_norm) == (2, SD, FNH, FNKV, HD, FV, R, 1)
    assert (slow.cfg.qkv_bias, slow.cfg.o_bias, slow.cfg.tied_embedding) == ((1, 1, 0) if full else (0, 0, 1))
    assert (fast.cfg.n_layers, fast.cfg.vocab, fast.cfg.max_seq, fast.cfg.qk_norm, fast.cfg.o_bias) == (2, R, NCB, 0, 0)
    assert slow.hidden_dim == FD

    qz = lambda k: ora.quantize(ora.Q4K, _f32(src[k]))  # noqa: E731
    tally = _Tally()
    for eng, base, n_cb in ((slow, "text_model.model.layers", NCB), (fast, "audio_decoder.layers", 0)):
        W = {}
        for l in range(2):
            p = f"{base}.{l}"
            for role, nm in (("wqkv", "attention.wqkv"), ("wo", "attention.wo"), ("w1", "feed_forward.w1"),
                             ("w3", "feed_forward.w3"), ("w2", "feed_forward.w2")):
                W[(role, l)] = qz(f"{p}.{nm}.weight")
            W[("attn_norm", l)] = _f32(src[f"{p}.attention_norm.weight"])
            W[("ffn_norm", l)] = _f32(src[f"{p}.ffn_norm.weight"])
            if n_cb:
                W[("q_norm", l)] = _f32(src[f"{p}.attention.q_norm.weight"])
                W[("k_norm", l)] = _f32(src[f"{p}.attention.k_norm.weight"])
            if n_cb and full:
                W[("bqkv", l)] = _f32(src[f"{p}.attention.wqkv.bias"])
                W[("bo", l)] = _f32(src[f"{p}.attention.wo.bias"])
        if n_cb:  # the slow head (tied to the embeddings unless lm_head ships); MCF over the dense table
            W["head"] = qz("text_model.lm_head.weight" if full else "text_model.model.embeddings.weight")
            W["embed"] = _f32(src["text_model.model.embeddings.weight"])
            W["final_norm"] = _f32(src["text_model.model.norm.weight"])
            W["codebook"] = _f32(src["audio_decoder.codebook_embeddings.weight"])
            if full:
                W["project_in"] = qz("fast_project_in.weight")
                W["project_in_bias"] = _f32(src["fast_project_in.bias"])
        else:
            W["head"] = qz("audio_decoder.output.weight")
            W["final_norm"] = _f32(src["audio_decoder.norm.weight"])
            W["embed"] = _f32(src["audio_decoder.embeddings.weight"])
        orc = model_oracle.OracleDecoder(eng.cfg, W, 1)
        eng.reset(1)
        if n_cb:
            for frame in ([BEGIN + 3, 1, 2, 3, 4, 5, 6], [17, 0, 0, 0, 0, 0, 0], [BEGIN + 100, 9, 8, 7, 6, 5, 4]):
                lg, hid = eng.slow_step_batch(torch.tensor([frame], dtype=torch.int32), graph=False)
                want = orc.step_one(0, frame=np.array(frame))
                _check(lg[0].cpu().numpy(), orc, want, f"slow frame {frame[0]}", tally)
                _check(hid.reshape(-1).cpu().numpy(), orc, orc.hidden, "slow hidden (through fast_project_in)"
                       if full else "slow hidden")
        else:
            h0 = np.random.default_rng(5).standard_normal(FD).astype(np.float32)
            lg, _ = eng.step(embeds=torch.from_numpy(h0)[None])
            _check(lg[0].cpu().numpy(), orc, orc.step_one(0, embed=h0), "fast position 0", tally)
            for code in (3, 127, 0):
                lg, _ = eng.step(ids=torch.tensor([code], dtype=torch.int32))
                _check(lg[0].cpu().numpy(), orc, orc.step_one(0, frame=[code]), f"fast code {code}", tally)
    tally.mostly_tight()


def test_fish_engines_from_gguf_equal_engines_from_checkpoint(cuda, tmp_path, ora):
    """A checkpoint quantized once into GGUF (save_fish_gguf) and loaded back
    (load_fish_gguf: the stored blocks become QMatMuls without re-quantization) gives
    the engines of the safetensors load: the stored blocks are the oracle's from_float of
    the same weights, and the logits of both engines are bit-identical."""
    src = _fish_checkpoint(tmp_path)
    w = I.load_fish_lm(str(tmp_path), device=cuda)
    path = str(tmp_path / "fish.gguf")
    I.save_fish_gguf(w, path, GgmlDType.Q4K)
    from syrinx_amd import gguf as G
    c = G.Content.read(path)
    assert c.metadata["general.quantization"].to_string() == "Q4K"
    name = "layers.1.feed_forward.w2.weight"
    assert c.tensor_infos[name].ggml_dtype == int(GgmlDType.Q4K) and c.tensor_infos[name].shape == (FD, FI)
    assert bytes(c.tensor_bytes(name)) == ora.quantize(ora.Q4K, _f32(src[f"text_model.model.{name}"])).tobytes()
    assert c.tensor_infos["norm.weight"].ggml_dtype == 0
    assert c.tensor_infos["embeddings.weight"].ggml_dtype == 0  # the dense table the embedding gathers
    g = I.load_fish_gguf(path, device=cuda)
    kw = dict(n_codebooks=NCB, semantic_begin=BEGIN, semantic_end=BEGIN + R - 1, max_seq=16, max_batch=1,
              dtype=GgmlDType.Q4K, device=cuda)
    a_slow, a_fast = I.fish_engines(w, **kw)
    b_slow, b_fast = I.fish_engines(g, **kw)
    for frame in ([BEGIN + 3, 1, 2, 3, 4, 5, 6], [17, 0, 0, 0, 0, 0, 0]):
        la, _, ha = a_slow.step(ids=torch.tensor([frame], dtype=torch.int32), want_hidden=True)
        lb, _, hb = b_slow.step(ids=torch.tensor([frame], dtype=torch.int32), want_hidden=True)
        assert torch.equal(la, lb) and torch.equal(ha, hb)
    h0 = torch.from_numpy(np.random.default_rng(5).standard_normal(FD).astype(np.float32))[None]
    assert torch.equal(a_fast.step(embeds=h0)[0], b_fast.step(embeds=h0)[0])
    with pytest.raises(ValueError, match="Q4K"):
        I.fish_engines(g, **dict(kw, dtype=GgmlDType.Q8_0))
