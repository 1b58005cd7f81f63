"""Host logic of checkpoint ingest (syrinx_amd/ingest.py), no GPU: the s2 key remap
(crates/syrinx-fish/src/s2/load.rs:148-263), the q/k/v fusion (:271-312), shard
resolution (:96-136) and the CosyVoice2 load_quantized placement policy
(crates/syrinx-lm/src/cv2/load.rs:68-122, 194-203)."""
import json

import pytest
import torch

from syrinx_amd import ingest as I


@pytest.mark.parametrize("key,want", [
    # the real s2-pro layout
    ("text_model.model.layers.7.attention.wqkv.weight", "layers.7.attention.wqkv.weight"),
    ("text_model.model.layers.0.attention.q_norm.weight", "layers.0.attention.q_norm.weight"),
    ("text_model.model.embeddings.weight", "embeddings.weight"),
    ("text_model.model.norm.weight", "norm.weight"),
    ("text_model.lm_head.weight", "output.weight"),
    ("audio_decoder.layers.3.feed_forward.w2.weight", "fast_layers.3.feed_forward.w2.weight"),
    ("audio_decoder.embeddings.weight", "fast_embeddings.weight"),
    ("audio_decoder.codebook_embeddings.weight", "codebook_embeddings.weight"),
    ("audio_decoder.norm.weight", "fast_norm.weight"),
    ("audio_decoder.output.weight", "fast_output.weight"),
    # fish-native names pass through
    ("layers.2.attention.wo.weight", "layers.2.attention.wo.weight"),
    ("fast_project_in.bias", "fast_project_in.bias"),
    # HF-Qwen3 fallbacks
    ("model.embed_tokens.weight", "embeddings.weight"),
    ("lm_head.weight", "output.weight"),
    ("model.layers.5.self_attn.k_proj.weight", "layers.5.attention.wk.weight"),
    ("model.layers.5.mlp.gate_proj.weight", "layers.5.feed_forward.w1.weight"),
    ("model.layers.5.mlp.up_proj.weight", "layers.5.feed_forward.w3.weight"),
    ("model.layers.5.input_layernorm.weight", "layers.5.attention_norm.weight"),
    ("model.layers.5.rotary_emb.inv_freq", None),            # an unmapped layer tail is dropped
    ("fast_transformer.layers.1.self_attn.o_proj.weight", "fast_layers.1.attention.wo.weight"),
    ("model.audio_decoder.output.weight", "fast_output.weight"),
    ("model.fast_project_in.weight", "fast_project_in.weight"),
    ("text_model.model.layers.nodot", None),                 # no layer tail
    ("something.else", "something.else"),                    # unknown keys are kept
])
def test_remap_qwen3_key(key, want):
    assert I.remap_qwen3_key(key) == want


def test_fuse_qkv_weights_and_biases():
    m = {"layers.0.attention.wq.weight": torch.ones(4, 2), "layers.0.attention.wk.weight": 2 * torch.ones(1, 2),
         "layers.0.attention.wv.weight": 3 * torch.ones(1, 2), "layers.0.attention.wq.bias": torch.zeros(4),
         "layers.0.attention.wk.bias": torch.ones(1), "layers.0.attention.wv.bias": torch.ones(1),
         "layers.1.attention.wq.weight": torch.ones(4, 2)}  # incomplete triple: left alone
    I.fuse_qkv(m)
    assert m["layers.0.attention.wqkv.weight"][:, 0].tolist() == [1, 1, 1, 1, 2, 3]
    assert m["layers.0.attention.wqkv.bias"].tolist() == [0, 0, 0, 0, 1, 1]
    assert "layers.0.attention.wq.weight" not in m and "layers.1.attention.wq.weight" in m


def test_resolve_shards(tmp_path):
    with pytest.raises(FileNotFoundError):
        I.resolve_shards(str(tmp_path))
    (tmp_path / "model.safetensors").write_bytes(b"")
    assert I.resolve_shards(str(tmp_path)) == [str(tmp_path / "model.safetensors")]
    for n in (2, 1):
        (tmp_path / f"model-0000{n}-of-00002.safetensors").write_bytes(b"")
    assert [p.rsplit("/", 1)[1] for p in I.resolve_shards(str(tmp_path))] == [
        "model-00001-of-00002.safetensors", "model-00002-of-00002.safetensors"]
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps(
        {"weight_map": {"a": "b.safetensors", "c": "a.safetensors", "d": "b.safetensors"}}))
    assert [p.rsplit("/", 1)[1] for p in I.resolve_shards(str(tmp_path))] == ["a.safetensors", "b.safetensors"]


@pytest.mark.parametrize("name,shape,where", [
    ("llm.model.lm_head.weight", (151936, 896), "drop"),
    ("llm.model.model.embed_tokens.weight", (151936, 896), "embed"),
    ("speech_embedding.weight", (6564 + 3, 896), "embed"),
    ("llm_embedding.weight", (2, 896), "embed"),
    ("llm.model.model.layers.0.mlp.down_proj.weight", (896, 4864), "qmm"),
    ("llm_decoder.weight", (6564 + 3, 896), "qmm"),
    ("some.odd.weight", (16, 80), "f16"),
    ("llm.model.model.layers.0.self_attn.q_proj.bias", (896,), "f32"),
])
def test_cv2_placement_policy(name, shape, where):
    assert I.cv2_policy(name, shape) == where
