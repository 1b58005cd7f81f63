"""CPU oracle of one decoder step (test infrastructure only).

Restates, for one new token per stream, the reference's f32 decode step with every
projection through the oracle's QMatMul restatement (Candle's generic CPU path):
  Fish s2 slow AR   crates/syrinx-fish/src/s2/slow_ar.rs:101-161 (embed), :166-202
                    (run_layers), :207-246 (head); crates/syrinx-fish/src/s2/nn.rs:284-360
                    (attention: wqkv -> split -> QK-RMSNorm -> interleaved RoPE -> cache
                    append -> GQA SDPA -> wo), :452-457 (SwiGLU), :100-106 (RMSNorm);
  CosyVoice2 LM     crates/syrinx-lm/src/cv2/mod.rs:261-286 (forward_logits_cached),
                    crates/syrinx-lm/src/cv2/attention.rs:46-78 (q/k/v + bias ->
                    rotate-half RoPE -> append -> SDPA -> o_proj).
The only weights it takes are the canonical GGML blocks and f32 vectors the GPU engine
is given, so both sides multiply by identical quantized weights.  With
cfg.weight_dtype == F32 every projection is instead a dense f32 matrix [n, k] and
x.W^T is accumulated in f64 and rounded once per output (Weights::linear's dense
broadcast_matmul, crates/syrinx-fish/src/s2/nn.rs:61-74): the form in which the
reference's toy-LM fixtures (tests/golden/parity/lm_*.json, PARITY.md sections 2-5)
pin this step's composition.
"""
from __future__ import annotations

import numpy as np

import oracle as ora


class OracleDecoder:
    def __init__(self, cfg, weights: dict, n_streams: int):
        """cfg: an object with the DecoderConfig fields.  weights keys:
        ('wqkv', l), ('wo', l), ('w1', l), ('w3', l), ('w2', l), 'head'  -> uint8 blocks [n, row_bytes]
                                                                            (f32 [n, k] when weight_dtype is F32)
        ('attn_norm', l), ('ffn_norm', l), ('q_norm', l), ('k_norm', l), ('bqkv', l), ('bo', l),
        'final_norm', 'head_bias', 'embed', 'codebook', 'project_in_bias' -> f32 arrays;
        'project_in' (fast_project_in, optional)                         -> blocks like the projections.
        'embed' is the dense input table [rows, dim] (Fish: embeddings.weight, also the
        tied head's source); a tied model given no 'embed' embeds through the
        dequantized head rows instead."""
        self.c = cfg
        self.W = weights
        self.dt = int(cfg.weight_dtype)
        hd = cfg.head_dim
        if cfg.rope_interleaved:
            self.cos, self.sin = ora.rope_tables_interleaved(cfg.max_seq, hd, cfg.rope_theta)
        else:
            self.cos, self.sin = ora.rope_tables_half(cfg.max_seq, hd, cfg.rope_theta)
        # caches[s][l] = (K [n_kv, L, hd], V [n_kv, L, hd]) as python lists of rows
        self.margin = 1.0  # smallest quantization margin seen in the last step (oracle.quant_margin)
        self.k = [[[[] for _ in range(cfg.n_kv_heads)] for _ in range(cfg.n_layers)] for _ in range(n_streams)]
        self.v = [[[[] for _ in range(cfg.n_kv_heads)] for _ in range(cfg.n_layers)] for _ in range(n_streams)]

    def _mm(self, x, blocks, name=""):
        if self.dt == ora.F32:
            y = (np.asarray(blocks, np.float64) @ np.asarray(x, np.float64)).astype(np.float32)
            self.margins.append((name, 1.0))
            return y
        m = ora.quant_margin(ora.VEC_DOT[self.dt], x)
        self.margins.append((name, m))
        self.margin = min(self.margin, m)
        return ora.matmul(self.dt, x[None, :], blocks)[0]

    def load_prefix(self, s, layer, g, k_rows, v_rows):
        self.k[s][layer][g] = [np.asarray(r, np.float32) for r in k_rows]
        self.v[s][layer][g] = [np.asarray(r, np.float32) for r in v_rows]

    def reset(self, s):
        """An empty cache for stream s (the fast AR's fresh KvCache per frame)."""
        for l in range(self.c.n_layers):
            for g in range(self.c.n_kv_heads):
                self.k[s][l][g] = []
                self.v[s][l][g] = []

    def length(self, s):
        return len(self.k[s][0][0])

    def embed(self, frame):
        """The step's input row: SlowAr::embed (crates/syrinx-fish/src/s2/slow_ar.rs:101-161)
        -- the token's row of embeddings.weight (:117), plus on semantic positions the sum
        of the offset codebook rows (:120-128, zeroed elsewhere :131-144) scaled by
        1/sqrt(n_codebooks + 1) (:146-156); a plain gather without codebooks
        (Qwen2Lm::embed, crates/syrinx-lm/src/cv2/generate.rs:22-67)."""
        c = self.c
        tok = int(frame[0])
        if c.tied_embedding or c.n_codebooks:
            if "embed" in self.W:
                x = np.asarray(self.W["embed"][tok], np.float32).copy()
            elif self.dt == ora.F32:
                x = np.asarray(self.W["head"][tok], np.float32).copy()
            else:
                x = ora.dequantize(self.dt, self.W["head"][tok], c.dim)[0]
            if c.n_codebooks:
                vq = None
                for i in range(c.n_codebooks):
                    e = self.W["codebook"][int(frame[1 + i]) + i * c.codebook_size]
                    vq = e.copy() if vq is None else (vq + e).astype(np.float32)
                sem = c.semantic_begin <= tok <= c.semantic_end
                inv_scale = np.float32(1.0) / np.sqrt(np.float32(c.n_codebooks) + np.float32(1.0))
                x = ((x + vq * np.float32(1.0 if sem else 0.0)) * (inv_scale if sem else np.float32(1.0))).astype(np.float32)
            return x
        return self.W["embed"][tok].astype(np.float32)

    def step_one(self, s, frame=None, embed=None):
        c = self.c
        hd, nh, nkv = c.head_dim, c.n_heads, c.n_kv_heads
        G = nh // nkv
        h = (self.embed(frame) if embed is None else np.asarray(embed, np.float32)).astype(np.float32)
        pos = self.length(s)
        self.margin = 1.0
        self.margins = []
        self.trace = {}
        for l in range(c.n_layers):
            r = h
            hn = ora.rms_norm(h, self.W[("attn_norm", l)], c.norm_eps)
            qkv = self._mm(hn, self.W[("wqkv", l)], f"qkv{l}")
            if c.qkv_bias:
                qkv = (qkv + self.W[("bqkv", l)]).astype(np.float32)
            q = qkv[: nh * hd].reshape(nh, hd)
            k = qkv[nh * hd: (nh + nkv) * hd].reshape(nkv, hd)
            v = qkv[(nh + nkv) * hd:].reshape(nkv, hd)
            if c.qk_norm:
                q = np.stack([ora.rms_norm(q[i], self.W[("q_norm", l)], c.norm_eps) for i in range(nh)])
                k = np.stack([ora.rms_norm(k[i], self.W[("k_norm", l)], c.norm_eps) for i in range(nkv)])
            rope = ora.rope_interleaved if c.rope_interleaved else ora.rope_half
            q = rope(q, self.cos[pos], self.sin[pos])
            k = rope(k, self.cos[pos], self.sin[pos])
            for g in range(nkv):
                self.k[s][l][g].append(k[g].copy())
                self.v[s][l][g].append(v[g].copy())
            ctx = np.zeros(nh * hd, np.float32)
            for i in range(nh):
                g = i // G
                ctx[i * hd:(i + 1) * hd] = ora.attend_one(q[i], np.stack(self.k[s][l][g]), np.stack(self.v[s][l][g]))
            o = self._mm(ctx, self.W[("wo", l)], f"o{l}")
            if getattr(c, "o_bias", 0):
                o = (o + self.W[("bo", l)]).astype(np.float32)
            h = (r + o).astype(np.float32)
            attn_out = o
            r = h
            hn = ora.rms_norm(h, self.W[("ffn_norm", l)], c.norm_eps)
            g_ = self._mm(hn, self.W[("w1", l)], f"gate{l}")
            u_ = self._mm(hn, self.W[("w3", l)], f"up{l}")
            a = ora.silu_mul(g_, u_)
            d = self._mm(a, self.W[("w2", l)], f"down{l}")
            h = (r + d).astype(np.float32)
            self.trace.update({"qkv": qkv, "q": q.reshape(-1), "gu": np.concatenate([g_, u_]), "h": h})
            self.trace[("ctx", l)] = ctx
            self.trace[("attn", l)] = attn_out
            self.trace[("h", l)] = h
        hn = ora.rms_norm(h, self.W["final_norm"], c.norm_eps)
        # SlowAr::head's `hidden` (slow_ar.rs:230-243): the post-norm state (norm_fastlayer_input),
        # through fast_project_in when the checkpoint has one (a narrower fast AR)
        self.hidden = hn
        if "project_in" in self.W:
            self.hidden = self._mm(hn, self.W["project_in"], "project_in")
            if "project_in_bias" in self.W:
                self.hidden = (self.hidden + self.W["project_in_bias"]).astype(np.float32)
        logits = self._mm(hn, self.W["head"], "head")
        if c.head_bias:
            logits = (logits + self.W["head_bias"]).astype(np.float32)
        return logits
