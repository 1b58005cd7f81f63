"""Checkpoint ingest: safetensors -> Candle-identical quantized weights -> the device engines.

Host mirror of the reference's two LM loaders, with every quantization on the GPU
(QTensor.quantize = Candle's from_float, QEmbed.quantize = quantize_embed):

* ``load_cv2_quantized`` -- Qwen2Lm::load_quantized (crates/syrinx-lm/src/cv2/load.rs:68-122):
  the unused ``lm_head`` dropped, the three embedding tables per-row int4 (int8 for odd
  widths), every other 2-D weight whose inner dim is a multiple of 32 a Q4_0 QMatMul, the
  other 2-D weights dense f16, 1-D weights f32; with its footprint report
  (cv2/load.rs:124-155, cv2/quant.rs:91-118).
* ``load_fish_lm`` -- s2's load_lm (crates/syrinx-fish/src/s2/load.rs:32-51): shard
  resolution (:96-136), the key remap onto the fish-native names (:148-263), the q/k/v fusion
  (:271-312); tensors are cast to f32 as they are read.
* ``cv2_engine`` / ``fish_engines`` -- wire a loaded checkpoint into ``Qwen2Lm`` and into
  ``SlowAr`` + ``FastAr`` (projections quantized to the engine's block type).

safetensors parsing uses the ``safetensors`` package (bf16 / f16 / f32 tensors); the
tensors are moved to the GPU before any conversion, so a checkpoint never exists as a
full f32 copy in host memory.
"""
from __future__ import annotations

import glob
import json
import os
import re
from dataclasses import dataclass, field

import torch

from .decoder import (ATTN_NORM, BK, BO, BQ, BV, CODEBOOK_EMBED, EMBED, FFN_NORM, FINAL_NORM, HEAD, HEAD_BIAS, K_NORM,
                      Q_NORM, W1, W2, W3, WK, WO, WQ, WQKV, WV, DecoderConfig, FastAr, Qwen2Lm, SlowAr,
                      cosyvoice2_lm_config, fish_s2_fast_ar_config, fish_s2_slow_ar_config)
from .embedding import DEFAULT_EMBED_SCHEME, QEmbed
from .quantized import GgmlDType, QMatMul, QTensor

Q4_0_BLOCK = 32


def read_safetensors(path: str, device) -> dict:
    """name -> tensor on `device`, in the file's dtype."""
    from safetensors import safe_open
    out = {}
    with safe_open(path, framework="pt", device="cpu") as f:
        for k in f.keys():
            out[k] = f.get_tensor(k).to(device)
    return out


# --------------------------------------------------------------------------- CosyVoice2
def is_unused_text_head(name: str) -> bool:
    """cv2/load.rs:158-170: the Qwen2 text head the speech path never calls."""
    return "lm_head" in name


CV2_EMBED_TABLES = ("llm.model.model.embed_tokens.weight", "llm_embedding.weight", "speech_embedding.weight")


def is_embedding_table(name: str) -> bool:
    """cv2/load.rs:172-177."""
    return name in CV2_EMBED_TABLES


@dataclass
class Footprint:
    """cv2/quant.rs:91-118."""
    quant_bytes: int
    embed_bytes: int
    dense_bytes: int
    n_quantized: int

    def total_bytes(self) -> int:
        return self.quant_bytes + self.embed_bytes + self.dense_bytes

    def total_mb(self) -> float:
        return self.total_bytes() / (1024.0 * 1024.0)


@dataclass
class Cv2Weights:
    """The loaded bags of Qwen2Lm (cv2/mod.rs:70-90): dense `w`, QMatMuls `qmm`, QEmbeds `qembed`."""
    w: dict = field(default_factory=dict)
    qmm: dict = field(default_factory=dict)
    qembed: dict = field(default_factory=dict)
    quant_bytes: int = 0

    def footprint(self) -> Footprint:
        dense = sum(t.numel() * t.element_size() for t in self.w.values())
        return Footprint(self.quant_bytes, sum(e.bytes for e in self.qembed.values()), dense, len(self.qmm))

    def dense_breakdown(self):
        """(name, bytes) of every dense weight, largest first (cv2/load.rs:140-155)."""
        v = [(k, t.numel() * t.element_size()) for k, t in self.w.items()]
        return sorted(v, key=lambda kv: -kv[1])


def cv2_policy(name: str, shape) -> str:
    """Where load_quantized puts a tensor: 'drop', 'embed', 'qmm', 'f16' or 'f32'."""
    if is_unused_text_head(name):
        return "drop"
    if is_embedding_table(name):
        return "embed"
    if len(shape) == 2 and shape[-1] % Q4_0_BLOCK == 0:
        return "qmm"
    if len(shape) == 2:
        return "f16"
    return "f32"


def load_cv2_quantized(path: str, device="cuda:0", embed_scheme: int = DEFAULT_EMBED_SCHEME,
                       dtype: GgmlDType = GgmlDType.Q4_0) -> Cv2Weights:
    """Qwen2Lm::load_quantized (cv2/load.rs:68-122) on the GPU."""
    device = torch.device(device)
    out = Cv2Weights()
    for k, v in read_safetensors(path, device).items():
        where = cv2_policy(k, tuple(v.shape))
        if where == "drop":
            continue
        vf = v.to(torch.float32)
        if where == "embed":
            out.qembed[k] = QEmbed.quantize(vf, embed_scheme)
        elif where == "qmm":
            qt = QTensor.quantize(vf.contiguous(), dtype)
            out.quant_bytes += qt.storage_size_in_bytes()
            out.qmm[k] = QMatMul.from_qtensor(qt)
        elif where == "f16":
            out.w[k] = vf.to(torch.float16)
        else:
            out.w[k] = vf
    return out


def _layer_count(names, pattern: str) -> int:
    rx = re.compile(pattern)
    idx = [int(m.group(1)) for n in names for m in [rx.match(n)] if m]
    return max(idx) + 1 if idx else 0


def cv2_engine(bag: Cv2Weights, max_seq: int = 1024, max_batch: int = 1, device="cuda:0") -> Qwen2Lm:
    """A Qwen2Lm decode engine over a load_cv2_quantized bag: per layer q/k/v (fused on
    upload) with their biases, o, gate/up/down, the two RMSNorms; the final norm, the
    llm_decoder head with its bias, and speech_embedding as the (quantized) input table.
    Geometry from the tensors; heads from head_dim 64 (cv2/mod.rs:36-56)."""
    pre = "llm.model.model.layers"
    names = list(bag.qmm) + list(bag.w)
    L = _layer_count(names, re.escape(pre) + r"\.(\d+)\.")
    q0 = bag.qmm[f"{pre}.0.self_attn.q_proj.weight"].shape
    k0 = bag.qmm[f"{pre}.0.self_attn.k_proj.weight"].shape
    gate = bag.qmm[f"{pre}.0.mlp.gate_proj.weight"].shape
    head = bag.qmm["llm_decoder.weight"].shape
    speech = bag.qembed.get("speech_embedding.weight")
    hd = 64
    dt = bag.qmm[f"{pre}.0.self_attn.q_proj.weight"].dtype()
    cfg = cosyvoice2_lm_config(n_layers=L, max_seq=max_seq, max_batch=max_batch, dtype=dt, dim=q0[1],
                               n_heads=q0[0] // hd, n_kv_heads=k0[0] // hd, head_dim=hd, intermediate=gate[0],
                               vocab=head[0], embed_rows=speech.rows_count if speech is not None else head[0] + 3,
                               head_bias=int("llm_decoder.bias" in bag.w))
    lm = Qwen2Lm(cfg, device=device)
    for l in range(L):
        p = f"{pre}.{l}"
        for slot, nm in ((WQ, "self_attn.q_proj"), (WK, "self_attn.k_proj"), (WV, "self_attn.v_proj"),
                         (WO, "self_attn.o_proj"), (W1, "mlp.gate_proj"), (W3, "mlp.up_proj"), (W2, "mlp.down_proj")):
            lm.set_linear(l, slot, bag.qmm[f"{p}.{nm}.weight"])
        for slot, nm in ((BQ, "self_attn.q_proj.bias"), (BK, "self_attn.k_proj.bias"), (BV, "self_attn.v_proj.bias"),
                         (ATTN_NORM, "input_layernorm.weight"), (FFN_NORM, "post_attention_layernorm.weight")):
            lm.set_vector(l, slot, bag.w[f"{p}.{nm}"])
    lm.set_linear(-1, HEAD, bag.qmm["llm_decoder.weight"])
    if cfg.head_bias:  # CosyVoice3's llm_decoder is bias-free (cv3/lm.rs:143-147)
        lm.set_vector(-1, HEAD_BIAS, bag.w["llm_decoder.bias"])
    lm.set_vector(-1, FINAL_NORM, bag.w["llm.model.model.norm.weight"])
    if speech is not None:
        lm.set_embed_quantized(speech)
    return lm


def cosyvoice_lm(bag: Cv2Weights, max_seq: int = 1024, device="cuda:0"):
    """Qwen2Lm (CosyVoice2) or Cv3Lm (CosyVoice3, told apart by the 6761-row bias-free head)
    ready to generate: cv2_engine over the bag plus its embedding tables (QEmbeds or dense)."""
    from .generate import COSYVOICE2, COSYVOICE3, CosyVoiceLm
    lm = cv2_engine(bag, max_seq=max_seq, max_batch=1, device=device)
    variant = COSYVOICE2 if lm.cfg.head_bias else COSYVOICE3

    def table(name):
        return bag.qembed.get(name, bag.w.get(name))
    return CosyVoiceLm(lm, table("llm.model.model.embed_tokens.weight"), table("speech_embedding.weight"),
                       table("llm_embedding.weight"), variant)


# --------------------------------------------------------------------------- Fish s2
def resolve_shards(d: str):
    """s2/load.rs:96-136: the index's weight map, else model-*.safetensors, else model.safetensors."""
    index = os.path.join(d, "model.safetensors.index.json")
    if os.path.exists(index):
        with open(index) as f:
            wm = json.load(f).get("weight_map") or {}
        files = sorted({v for v in wm.values() if isinstance(v, str)})
        if files:
            return [os.path.join(d, f) for f in files]
    globbed = sorted(p for p in glob.glob(os.path.join(d, "model-*.safetensors")))
    if globbed:
        return globbed
    single = os.path.join(d, "model.safetensors")
    if os.path.exists(single):
        return [single]
    raise FileNotFoundError(f"no LM safetensors shards found in {d}")


# Top-level renames of s2/load.rs:156-232, in the order the reference tries them.
_S2_TOP = {
    "text_model.model.embeddings.weight": "embeddings.weight",
    "text_model.model.norm.weight": "norm.weight",
    "text_model.lm_head.weight": "output.weight",
    "audio_decoder.embeddings.weight": "fast_embeddings.weight",
    "audio_decoder.codebook_embeddings.weight": "codebook_embeddings.weight",
    "audio_decoder.norm.weight": "fast_norm.weight",
    "audio_decoder.output.weight": "fast_output.weight",
}
_FISH_NATIVE = ("embeddings.weight", "codebook_embeddings.weight", "fast_embeddings.weight", "norm.weight",
                "fast_norm.weight", "fast_output.weight", "output.weight")
_HF_TOP = {
    "model.embed_tokens.weight": "embeddings.weight",
    "model.norm.weight": "norm.weight",
    "lm_head.weight": "output.weight",
    "codebook_embeddings.weight": "codebook_embeddings.weight",
}
_HF_FAST_TOP = {
    "model.audio_decoder.embeddings.weight": "fast_embeddings.weight",
    "audio_decoder.embeddings.weight": "fast_embeddings.weight",
    "model.audio_decoder.norm.weight": "fast_norm.weight",
    "audio_decoder.norm.weight": "fast_norm.weight",
    "model.audio_decoder.output.weight": "fast_output.weight",
    "audio_decoder.output.weight": "fast_output.weight",
    "model.codebook_embeddings.weight": "codebook_embeddings.weight",
    "model.fast_project_in.weight": "fast_project_in.weight",
    "model.fast_project_in.bias": "fast_project_in.bias",
    "fast_project_in.weight": "fast_project_in.weight",
    "fast_project_in.bias": "fast_project_in.bias",
}
_HF_TAIL = {
    "input_layernorm.weight": "attention_norm.weight",
    "post_attention_layernorm.weight": "ffn_norm.weight",
    "self_attn.q_proj.weight": "attention.wq.weight",
    "self_attn.q_proj.bias": "attention.wq.bias",
    "self_attn.k_proj.weight": "attention.wk.weight",
    "self_attn.k_proj.bias": "attention.wk.bias",
    "self_attn.v_proj.weight": "attention.wv.weight",
    "self_attn.v_proj.bias": "attention.wv.bias",
    "self_attn.o_proj.weight": "attention.wo.weight",
    "self_attn.o_proj.bias": "attention.wo.bias",
    "self_attn.q_norm.weight": "attention.q_norm.weight",
    "self_attn.k_norm.weight": "attention.k_norm.weight",
    "mlp.gate_proj.weight": "feed_forward.w1.weight",
    "mlp.up_proj.weight": "feed_forward.w3.weight",
    "mlp.down_proj.weight": "feed_forward.w2.weight",
}


def _split_layer(rest: str):
    """Rust's split_once('.'): (layer, tail), or (None, None) without a dot."""
    n, dot, tail = rest.partition(".")
    return (n, tail) if dot else (None, None)


def remap_qwen3_key(k: str):
    """s2/load.rs:148-237: the fish-native name of a checkpoint key, or None to drop it."""
    if k.startswith("text_model.model.layers."):
        n, tail = _split_layer(k[len("text_model.model.layers."):])
        return None if n is None else f"layers.{n}.{tail}"
    if k in _S2_TOP:
        return _S2_TOP[k]
    if k.startswith("audio_decoder.layers."):
        n, tail = _split_layer(k[len("audio_decoder.layers."):])
        return None if n is None else f"fast_layers.{n}.{tail}"
    if k.startswith("layers.") or k.startswith("fast_layers.") or k in _FISH_NATIVE or k.startswith("fast_project_in."):
        return k
    if k in _HF_TOP:
        return _HF_TOP[k]
    if k.startswith("model.layers."):
        n, tail = _split_layer(k[len("model.layers."):])
        if n is None or tail not in _HF_TAIL:
            return None
        return f"layers.{n}.{_HF_TAIL[tail]}"
    for pfx in ("model.audio_decoder.layers.", "audio_decoder.layers.", "fast_transformer.layers."):
        if k.startswith(pfx):
            n, tail = _split_layer(k[len(pfx):])
            if n is None or tail not in _HF_TAIL:
                return None
            return f"fast_layers.{n}.{_HF_TAIL[tail]}"
    if k in _HF_FAST_TOP:
        return _HF_FAST_TOP[k]
    return k


def fuse_qkv(m: dict) -> None:
    """s2/load.rs:271-312: <p>.wq/.wk/.wv (weights, and biases when all three ship) -> <p>.wqkv."""
    for wq in [k for k in m if k.endswith(".wq.weight")]:
        base = wq[: -len(".wq.weight")]
        for suf in ("weight", "bias"):
            q, k_, v, f = (f"{base}.{x}.{suf}" for x in ("wq", "wk", "wv", "wqkv"))
            if f not in m and q in m and k_ in m and v in m:
                m[f] = torch.cat([m.pop(q), m.pop(k_), m.pop(v)], 0)


def load_fish_lm(d: str, device="cuda:0") -> dict:
    """load_lm (s2/load.rs:32-51) with dt = f32: fish-native name -> f32 tensor on the GPU."""
    device = torch.device(device)
    out = {}
    for path in resolve_shards(d):
        for k, v in read_safetensors(path, device).items():
            if "audio_tower" in k or "visual" in k:
                continue
            key = remap_qwen3_key(k)
            if key is not None:
                out[key] = v.to(torch.float32)
    fuse_qkv(out)
    return out


def _fish_layers(w: dict, base: str) -> int:
    return _layer_count(w, re.escape(base) + r"\.(\d+)\.")


def _q(w: dict, name: str, dtype: GgmlDType) -> QMatMul:
    t = w[name]
    if isinstance(t, QTensor):  # already quantized (a GGUF checkpoint)
        if t.dtype() != dtype:
            raise ValueError(f"{name} is {t.dtype().name}, the engine runs {GgmlDType(dtype).name}")
        return QMatMul.from_qtensor(t)
    return QMatMul.from_qtensor(QTensor.quantize(t.contiguous(), dtype))


# The Fish weights fish_engines runs only as QMatMul projections; every other tensor is a
# vector or a dense table.  embeddings.weight is a dense table (the token embedding
# gathers it) even where the tied head quantizes it.
_FISH_LINEAR = re.compile(r"^(layers|fast_layers)\.\d+\.(attention\.(wqkv|wo)|feed_forward\.(w1|w2|w3))\.weight$")


def is_fish_projection(name: str) -> bool:
    return bool(_FISH_LINEAR.match(name)) or name in ("output.weight", "fast_output.weight", "fast_project_in.weight")


def save_fish_gguf(w: dict, path: str, dtype: GgmlDType = GgmlDType.Q4K) -> None:
    """Quantize a load_fish_lm bag once and store it as GGUF: the projections (and an untied
    slow head, the fast output and fast_project_in) as `dtype` blocks made by Candle's
    from_float; the norms, biases and embedding tables f32 -- embeddings.weight too, which
    the token embedding gathers and a tied head quantizes when the engines are built.
    load_fish_gguf reads it back for fish_engines."""
    from . import gguf
    tensors = []
    for name in sorted(w):
        t = w[name]
        if is_fish_projection(name) and not isinstance(t, QTensor):
            t = QTensor.quantize(t.contiguous(), dtype)
        tensors.append((name, t))
    gguf.save(path, [("general.architecture", "fish-s2"), ("general.quantization", GgmlDType(dtype).name)], tensors)


def load_fish_gguf(path: str, device="cuda:0") -> dict:
    """A GGUF checkpoint as a fish_engines bag: quantized tensors as QTensors on `device`
    (no re-quantization), f32/f16 tensors as f32 torch tensors."""
    from . import gguf
    c = gguf.Content.read(path)
    out = {}
    for name, ti in c.tensor_infos.items():
        out[name] = c.dense(name, device) if ti.ggml_dtype in (0, 1) else c.tensor(name, device)
    return out


def _attn_flags(w: dict, base: str) -> dict:
    """The attention variant of a block stack, from its tensors as the reference derives it
    (slow_ar.rs:86-98, fast_ar.rs:53-65): qkv / o bias and QK-RMSNorm present in layer 0."""
    return dict(qkv_bias=int(f"{base}.0.attention.wqkv.bias" in w), o_bias=int(f"{base}.0.attention.wo.bias" in w),
                qk_norm=int(f"{base}.0.attention.q_norm.weight" in w))


def _wire_fish(lm, w: dict, base: str, L: int, dtype: GgmlDType, qk_norm: bool) -> None:
    c = lm.cfg
    q, kv = c.n_heads * c.head_dim, c.n_kv_heads * c.head_dim
    for l in range(L):
        p = f"{base}.{l}"
        for slot, nm in ((WQKV, "attention.wqkv"), (WO, "attention.wo"), (W1, "feed_forward.w1"),
                         (W3, "feed_forward.w3"), (W2, "feed_forward.w2")):
            lm.set_linear(l, slot, _q(w, f"{p}.{nm}.weight", dtype))
        if c.qkv_bias:  # the fused [q; k; v] bias, split into the engine's three slots
            b = w[f"{p}.attention.wqkv.bias"].reshape(-1)
            lm.set_vector(l, BQ, b[:q])
            lm.set_vector(l, BK, b[q:q + kv])
            lm.set_vector(l, BV, b[q + kv:q + 2 * kv])
        if c.o_bias:
            lm.set_vector(l, BO, w[f"{p}.attention.wo.bias"])
        lm.set_vector(l, ATTN_NORM, w[f"{p}.attention_norm.weight"])
        lm.set_vector(l, FFN_NORM, w[f"{p}.ffn_norm.weight"])
        if qk_norm:
            lm.set_vector(l, Q_NORM, w[f"{p}.attention.q_norm.weight"])
            lm.set_vector(l, K_NORM, w[f"{p}.attention.k_norm.weight"])


def fish_engines(w: dict, n_codebooks: int = 10, semantic_begin: int = 151678, semantic_end: int = 155773,
                 max_seq: int = 1280, max_batch: int = 1, dtype: GgmlDType = GgmlDType.Q4K, device="cuda:0",
                 head_dim: int = 128):
    """SlowAr + FastAr over a load_fish_lm bag, projections quantized to `dtype`.  The slow
    head is tied to `embeddings` unless `output.weight` ships (slow_ar.rs:213-221), and the
    token embedding gathers the dense `embeddings.weight` either way (slow_ar.rs:117; a
    GGUF bag holds that table only quantized, and then the embedding dequantizes its
    rows).  qkv / o bias and QK-norm of each stack come from its tensors (slow_ar.rs:86-98,
    fast_ar.rs:53-65); a `fast_project_in` maps the slow hidden onto a narrower fast AR
    (slow_ar.rs:230-243)."""
    Ls, Lf = _fish_layers(w, "layers"), _fish_layers(w, "fast_layers")
    emb = w["embeddings.weight"]
    vocab, dim = emb.shape
    wqkv = w["layers.0.attention.wqkv.weight"]
    kv = w["layers.0.attention.k_norm.weight"].shape[0] if "layers.0.attention.k_norm.weight" in w else head_dim
    hd = kv
    n_heads = w["layers.0.attention.wo.weight"].shape[1] // hd
    n_kv = (wqkv.shape[0] - n_heads * hd) // (2 * hd)
    inter = w["layers.0.feed_forward.w1.weight"].shape[0]
    cb = w["codebook_embeddings.weight"]
    cfg = fish_s2_slow_ar_config(n_layers=Ls, max_seq=max_seq, max_batch=max_batch, dtype=dtype, n_codebooks=n_codebooks,
                                 dim=dim, n_heads=n_heads, n_kv_heads=n_kv, head_dim=hd, intermediate=inter,
                                 vocab=vocab, codebook_size=cb.shape[0] // n_codebooks, semantic_begin=semantic_begin,
                                 semantic_end=semantic_end, tied_embedding=int("output.weight" not in w),
                                 **_attn_flags(w, "layers"))
    slow = SlowAr(cfg, device=device)
    _wire_fish(slow, w, "layers", Ls, dtype, bool(cfg.qk_norm))
    slow.set_linear(-1, HEAD, _q(w, "output.weight" if "output.weight" in w else "embeddings.weight", dtype))
    if not isinstance(emb, QTensor):
        slow.set_vector(-1, EMBED, emb)
    elif not cfg.tied_embedding:
        raise ValueError("embeddings.weight is quantized but the head is output.weight: no table to embed from")
    slow.set_vector(-1, FINAL_NORM, w["norm.weight"])
    slow.set_vector(-1, CODEBOOK_EMBED, cb)
    if "fast_project_in.weight" in w:
        slow.set_project_in(_q(w, "fast_project_in.weight", dtype), w.get("fast_project_in.bias"))
    fe = w["fast_embeddings.weight"]
    fo = w["fast_output.weight"]
    fw = w["fast_layers.0.attention.wqkv.weight"]
    f_heads = w["fast_layers.0.attention.wo.weight"].shape[1] // hd
    fcfg = fish_s2_fast_ar_config(n_layers=Lf, num_codebooks=n_codebooks, residual_size=fo.shape[0],
                                  max_batch=max_batch, dtype=dtype, dim=fe.shape[1], n_heads=f_heads,
                                  n_kv_heads=(fw.shape[0] - f_heads * hd) // (2 * hd), head_dim=hd,
                                  intermediate=w["fast_layers.0.feed_forward.w1.weight"].shape[0],
                                  embed_rows=fe.shape[0], **_attn_flags(w, "fast_layers"))
    fast = FastAr(fcfg, device=device)
    _wire_fish(fast, w, "fast_layers", Lf, dtype, bool(fcfg.qk_norm))
    fast.set_linear(-1, HEAD, _q(w, "fast_output.weight", dtype))
    fast.set_vector(-1, FINAL_NORM, w["fast_norm.weight"])
    fast.set_vector(-1, EMBED, fe)
    return slow, fast


__all__ = ["DecoderConfig", "load_cv2_quantized", "cv2_engine", "cosyvoice_lm", "load_fish_lm", "fish_engines", "save_fish_gguf",
           "load_fish_gguf", "is_fish_projection", "remap_qwen3_key",
           "resolve_shards", "fuse_qkv", "cv2_policy", "Footprint", "Cv2Weights"]
