"""Pins for the oracle's decode-step composition (oracle/model.py), on the CPU.

The reference holds golden vectors for exactly this composition: a toy LM whose
weights are a pure function of their names (FNV-1a 64 -> xorshift64 -> uniform
(-0.02, 0.02), PARITY.md section 2), run over the ids [1, 5, 9, 2, 0]
(tests/golden/parity/lm_embed.json, lm_attn0.json, lm_block0.json,
lm_forward.json, copied unchanged to tests/golden/reference_toy/).  The oracle runs
that model with dense f32 projections, one token at a time through its KV cache,
and must land on the fixtures: the embedding exactly, layer 0's attention output
and block output within 1e-4, the logits of all five positions within 1e-3 (the
fixtures' own tolerances).  That pins the pre-norm residual order, the contiguous
head split, interleaved RoPE on q and k only, the 1/sqrt(head_dim) scale, the
causal cache, the w1 (gate) / w3 (up) / w2 (down) roles and the final norm -> head.

The toy model has as many KV heads as query heads, so the GQA grouping
(g = i // (n_heads / n_kv_heads), repeat_kv at crates/syrinx-fish/src/s2/nn.rs:194-202)
and the Fish MCF embedding (crates/syrinx-fish/src/s2/slow_ar.rs:101-161) get
hand-derived checks of their own.  Each plausible slip is planted into a copy of
oracle/model.py's source (on the CPU) and must fail at least one check.
"""
import json
import os
import types

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden", "reference_toy")
MODEL_SRC = os.path.join(os.path.dirname(HERE), "oracle", "model.py")

IDS = [1, 5, 9, 2, 0]
TOY = dict(vocab=512, dim=128, n_layers=4, n_heads=4, head_dim=32, ffn=256, theta=10000.0, eps=1e-5)


def _gold(name):
    with open(os.path.join(GOLD, name + ".json")) as f:
        d = json.load(f)
    return np.asarray(d["data"], np.float64).reshape(d["shape"]), float(d["tol"])


# ------------------------------------------------------------- the fixtures' weight generator
def _fnv1a64(name: str) -> int:
    h = 0xCBF29CE484222325
    for b in name.encode("utf-8"):
        h ^= b
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def _weights(name: str, count: int) -> np.ndarray:
    """PARITY.md section 2: the first `count` values of the xorshift64 stream seeded by the
    name's FNV-1a hash, each (x >> 11) / 2^53 * 2 - 1 scaled by 0.02 and rounded to f32."""
    state = _fnv1a64(name) or 0x9E3779B97F4A7C15
    m = 0xFFFFFFFFFFFFFFFF
    out = np.empty(count, np.float32)
    for i in range(count):
        x = state
        x ^= (x << 13) & m
        x ^= x >> 7
        x ^= (x << 17) & m
        state = x
        out[i] = np.float32(((x >> 11) * (1.0 / 2.0 ** 53) * 2.0 - 1.0) * 0.02)
    return out


def _mat(name, rows, cols):
    return _weights(name, rows * cols).reshape(rows, cols)


def test_weight_generator_matches_reference_sample():
    want, _ = _gold("weights_sample")
    got = _weights("tok_embeddings", 8)
    np.testing.assert_array_equal(got, want.astype(np.float32))


def test_generator_constants_are_pinned():
    # FNV-1a of the empty string is the offset basis; of "a" the published 0xaf63dc4c8601ec8c.
    assert _fnv1a64("") == 0xCBF29CE484222325
    assert _fnv1a64("a") == 0xAF63DC4C8601EC8C
    # A different name gives a different stream (the weights really depend on the name).
    assert not np.array_equal(_weights("tok_embeddings", 8), _weights("output.weight", 8))


# ------------------------------------------------------------- the toy LM through the oracle
def _toy_cfg(**over):
    t = TOY
    c = dict(n_layers=t["n_layers"], dim=t["dim"], n_heads=t["n_heads"], n_kv_heads=t["n_heads"],
             head_dim=t["head_dim"], intermediate=t["ffn"], vocab=t["vocab"], embed_rows=0, max_seq=16,
             max_batch=1, weight_dtype=0, norm_eps=t["eps"], rope_theta=t["theta"], rope_interleaved=1,
             qk_norm=0, qkv_bias=0, head_bias=0, tied_embedding=0, n_codebooks=0, codebook_size=0,
             semantic_begin=0, semantic_end=-1, o_bias=0)
    c.update(over)
    return types.SimpleNamespace(**c)


@pytest.fixture(scope="module")
def toy_weights():
    t = TOY
    d, f, v = t["dim"], t["ffn"], t["vocab"]
    W = {"embed": _mat("tok_embeddings", v, d), "final_norm": _weights("norm.weight", d),
         "head": _mat("output.weight", v, d)}
    for l in range(t["n_layers"]):
        p = f"layers.{l}"
        W[("wqkv", l)] = np.concatenate([_mat(f"{p}.attention.{n}.weight", d, d) for n in ("wq", "wk", "wv")])
        W[("wo", l)] = _mat(f"{p}.attention.wo.weight", d, d)
        W[("w1", l)] = _mat(f"{p}.feed_forward.w1.weight", f, d)
        W[("w3", l)] = _mat(f"{p}.feed_forward.w3.weight", f, d)
        W[("w2", l)] = _mat(f"{p}.feed_forward.w2.weight", d, f)
        W[("attn_norm", l)] = _weights(f"{p}.attention_norm.weight", d)
        W[("ffn_norm", l)] = _weights(f"{p}.ffn_norm.weight", d)
    return W


def _load_model(plant=None):
    """oracle/model.py as a fresh module, optionally with one textual slip planted."""
    src = open(MODEL_SRC).read()
    if plant is not None:
        old, new = plant
        assert src.count(old) == 1, f"plant site not unique: {old!r}"
        src = src.replace(old, new)
    mod = types.ModuleType("model_planted" if plant else "model_copy")
    exec(compile(src, MODEL_SRC, "exec"), mod.__dict__)
    return mod


def _run_toy(W, mod=None, cfg=None):
    mod = mod or _load_model()
    orc = mod.OracleDecoder(cfg or _toy_cfg(), W, 1)
    out = {"embed": [], "attn0": [], "block0": [], "logits": []}
    for tok in IDS:
        frame = np.array([tok], np.int32)
        out["embed"].append(orc.embed(frame))
        out["logits"].append(orc.step_one(0, frame))
        out["attn0"].append(orc.trace[("attn", 0)])
        out["block0"].append(orc.trace[("h", 0)])
    return {k: np.stack(v).astype(np.float64) for k, v in out.items()}


@pytest.fixture(scope="module")
def toy_run(ora, toy_weights):
    return _run_toy(toy_weights)


def _err(got, name):
    want, tol = _gold(name)
    return float(np.abs(got - want).max()), tol


def test_toy_embedding_matches_fixture(toy_run):
    want, _ = _gold("lm_embed")
    np.testing.assert_array_equal(toy_run["embed"].astype(np.float32), want.astype(np.float32))


def test_toy_layer0_attention_matches_fixture(toy_run):
    err, tol = _err(toy_run["attn0"], "lm_attn0")
    assert err <= tol, err


def test_toy_layer0_block_matches_fixture(toy_run):
    err, tol = _err(toy_run["block0"], "lm_block0")
    assert err <= tol, err


def test_toy_forward_logits_match_fixture(toy_run):
    err, tol = _err(toy_run["logits"], "lm_forward")
    # The oracle's f32 glue against the fixture's f64-accumulated reference: far inside 1e-3.
    assert err <= min(tol, 1e-5), err


# Slips in the step composition that the fixtures catch: each must push at least one
# fixture past its tolerance.  (With the toy's 0.02-scale weights the attention is nearly
# uniform, so RoPE and head-split slips stay inside the fixtures' tolerances; the sharp
# attention check below catches those.)
SLIPS = {
    "residual on the normed input": ("h = (r + o).astype(np.float32)", "h = (hn + o).astype(np.float32)"),
    "no final norm": ('hn = ora.rms_norm(h, self.W["final_norm"], c.norm_eps)', "hn = h"),
    "FFN residual dropped": ("h = (r + d).astype(np.float32)", "h = d.astype(np.float32)"),
    "final norm with the last layer's FFN norm weight": (
        'hn = ora.rms_norm(h, self.W["final_norm"], c.norm_eps)',
        'hn = ora.rms_norm(h, self.W[("ffn_norm", c.n_layers - 1)], c.norm_eps)'),
}


@pytest.mark.parametrize("slip", sorted(SLIPS))
def test_planted_composition_slip_is_caught(ora, toy_weights, slip):
    run = _run_toy(toy_weights, _load_model(SLIPS[slip]))
    caught = []
    for key, name in (("attn0", "lm_attn0"), ("block0", "lm_block0"), ("logits", "lm_forward")):
        err, tol = _err(run[key], name)
        if err > tol:
            caught.append(name)
    assert caught, f"{slip}: every fixture still passes"


# ------------------------------------------------------------- sharp attention, matrix form
# PARITY.md 5.2 evaluated as the fixtures' generator does -- the whole sequence at once,
# scores masked by the causal matrix -- in f64 with RoPE as a complex rotation of the
# pairs (2i, 2i+1), against the oracle's one-token-at-a-time cached steps.  Weights of
# scale 0.5 make the softmax sharp, so RoPE, the head split and the grouping all matter.
def _sharp_setup(T=5, nh=4, nkv=2, hd=8, dim=16, theta=10000.0):
    rng = np.random.default_rng(11)
    cfg = _toy_cfg(n_layers=1, dim=dim, n_heads=nh, n_kv_heads=nkv, head_dim=hd, intermediate=8, vocab=T,
                   rope_theta=theta)
    W = {"embed": rng.standard_normal((T, dim)).astype(np.float32),
         ("wqkv", 0): (rng.standard_normal(((nh + 2 * nkv) * hd, dim)) * 0.5).astype(np.float32),
         ("wo", 0): (rng.standard_normal((dim, nh * hd)) * 0.5).astype(np.float32),
         ("w1", 0): np.zeros((8, dim), np.float32), ("w3", 0): np.zeros((8, dim), np.float32),
         ("w2", 0): np.zeros((dim, 8), np.float32),
         ("attn_norm", 0): (1.0 + 0.1 * rng.standard_normal(dim)).astype(np.float32),
         ("ffn_norm", 0): np.ones(dim, np.float32), "final_norm": np.ones(dim, np.float32),
         "head": np.zeros((T, dim), np.float32)}
    return cfg, W


def _sharp_expected(cfg, W):
    T, nh, nkv, hd = cfg.vocab, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
    x = W["embed"].astype(np.float64)
    xn = x / np.sqrt((x * x).mean(axis=1, keepdims=True) + cfg.norm_eps) * W[("attn_norm", 0)]
    qkv = xn @ W[("wqkv", 0)].astype(np.float64).T
    q = qkv[:, : nh * hd].reshape(T, nh, hd)
    k = qkv[:, nh * hd: (nh + nkv) * hd].reshape(T, nkv, hd)
    v = qkv[:, (nh + nkv) * hd:].reshape(T, nkv, hd)
    inv = cfg.rope_theta ** (-np.arange(0, hd, 2) / hd)
    rot = np.exp(1j * np.arange(T)[:, None] * inv[None, :])  # [T, hd/2]

    def rope(a):
        z = (a[..., 0::2] + 1j * a[..., 1::2]) * rot[:, None, :]
        out = np.empty_like(a)
        out[..., 0::2], out[..., 1::2] = z.real, z.imag
        return out

    q, k = rope(q), rope(k)
    mask = np.triu(np.full((T, T), -np.inf), 1)
    ctx = np.empty((T, nh, hd))
    for h in range(nh):
        g = h // (nh // nkv)
        sc = q[:, h, :] @ k[:, g, :].T / np.sqrt(hd) + mask
        p = np.exp(sc - sc.max(axis=1, keepdims=True))
        p /= p.sum(axis=1, keepdims=True)
        ctx[:, h, :] = p @ v[:, g, :]
    return ctx.reshape(T, nh * hd) @ W[("wo", 0)].astype(np.float64).T


def _sharp_oracle(mod):
    cfg, W = _sharp_setup()
    orc = mod.OracleDecoder(cfg, W, 1)
    out = []
    for t in range(cfg.vocab):
        orc.step_one(0, np.array([t], np.int32))
        out.append(orc.trace[("attn", 0)])
    return np.stack(out).astype(np.float64), _sharp_expected(cfg, W)


def test_sharp_attention_matches_matrix_form(ora):
    got, want = _sharp_oracle(_load_model())
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()


ATTN_SLIPS = {
    "rotate-half instead of interleaved RoPE": (
        "rope = ora.rope_interleaved if c.rope_interleaved else ora.rope_half", "rope = ora.rope_half"),
    "keys not rotated": ("k = rope(k, self.cos[pos], self.sin[pos])", "k = k"),
    "queries not rotated": ("q = rope(q, self.cos[pos], self.sin[pos])", "q = q"),
    "values rotated too": ("self.v[s][l][g].append(v[g].copy())",
                           "self.v[s][l][g].append(rope(v, self.cos[pos], self.sin[pos])[g].copy())"),
    "strided head split": ("q = qkv[: nh * hd].reshape(nh, hd)", "q = qkv[: nh * hd].reshape(hd, nh).T.copy()"),
    "interleaved GQA grouping": ("g = i // G", "g = i % nkv"),
    "queries rotated at the previous key's position": (
        "q = rope(q, self.cos[pos], self.sin[pos])", "q = rope(q, self.cos[max(pos - 1, 0)], self.sin[max(pos - 1, 0)])"),
}
# (A slip that moves every position by the same offset is invisible by construction:
# RoPE scores depend on position differences only.)


@pytest.mark.parametrize("slip", sorted(ATTN_SLIPS))
def test_planted_attention_slip_is_caught(ora, slip):
    got, want = _sharp_oracle(_load_model(ATTN_SLIPS[slip]))
    assert np.abs(got - want).max() > 1e-3 * np.abs(want).max(), slip


# ------------------------------------------------------------- SwiGLU roles, by hand
# With the toy's 0.02-scale weights silu(g) * u ~ g * u / 2 is nearly symmetric in g and u,
# so the fixtures cannot tell gate from up; a hand-built layer can.
def _swiglu_setup():
    dim, inter = 4, 2
    cfg = _toy_cfg(n_layers=1, dim=dim, n_heads=1, n_kv_heads=1, head_dim=4, intermediate=inter, vocab=2,
                   norm_eps=0.0)
    w1 = np.zeros((inter, dim), np.float32)
    w3 = np.zeros((inter, dim), np.float32)
    w1[:, 0] = [2.0, -1.0]   # gate rows: x . w1 = 2, -1 (x = ones)
    w3[:, 0] = [3.0, 0.5]    # up rows:   x . w3 = 3, 0.5
    w2 = np.zeros((dim, inter), np.float32)
    w2[0, 0] = 1.0
    w2[1, 1] = 1.0
    W = {"embed": np.ones((2, dim), np.float32), ("wqkv", 0): np.zeros((12, dim), np.float32),
         ("wo", 0): np.zeros((dim, 4), np.float32), ("w1", 0): w1, ("w3", 0): w3, ("w2", 0): w2,
         ("attn_norm", 0): np.ones(dim, np.float32), ("ffn_norm", 0): np.ones(dim, np.float32),
         "final_norm": np.ones(dim, np.float32), "head": np.zeros((2, dim), np.float32)}
    return cfg, W


def _swiglu_h(mod):
    cfg, W = _swiglu_setup()
    orc = mod.OracleDecoder(cfg, W, 1)
    orc.step_one(0, np.array([0], np.int32))
    return orc.trace[("h", 0)].astype(np.float64)


def _silu(v):
    return v / (1.0 + np.exp(-v))


def test_swiglu_gate_up_down_roles(ora):
    # h = x + w2 . (silu(x.w1) * (x.w3)); x = ones, attention output zero (wo = 0)
    want = np.array([1 + _silu(2.0) * 3.0, 1 + _silu(-1.0) * 0.5, 1.0, 1.0])
    np.testing.assert_allclose(_swiglu_h(_load_model()), want, rtol=1e-6)


def test_swiglu_role_slips_are_caught(ora):
    want = np.array([1 + _silu(2.0) * 3.0, 1 + _silu(-1.0) * 0.5, 1.0, 1.0])
    for slip in [('g_ = self._mm(hn, self.W[("w1", l)], f"gate{l}")', 'g_ = self._mm(hn, self.W[("w3", l)], f"gate{l}")'),
                 ('u_ = self._mm(hn, self.W[("w3", l)], f"up{l}")', 'u_ = self._mm(hn, self.W[("w1", l)], f"up{l}")'),
                 ("a = ora.silu_mul(g_, u_)", "a = ora.silu_mul(u_, g_)")]:
        got = _swiglu_h(_load_model(slip))
        assert not np.allclose(got, want, rtol=1e-6), slip


# ------------------------------------------------------------- GQA grouping, by hand
def _gqa_setup():
    """Dense model, 4 query heads over 2 KV heads of width 4, dim 8.  The attention norm
    weight is 1 and the input row is all ones, so the normed input is exactly ones and
    every projection row's output is that row's sum (eps 0: the norm of ones is exactly ones).
    v rows of group g sum to 10 + g."""
    nh, nkv, hd, dim = 4, 2, 4, 8
    cfg = _toy_cfg(n_layers=1, dim=dim, n_heads=nh, n_kv_heads=nkv, head_dim=hd, intermediate=8, vocab=4,
                   norm_eps=0.0)
    qkv = np.zeros(((nh + 2 * nkv) * hd, dim), np.float32)
    for g in range(nkv):
        for e in range(hd):
            qkv[(nh + nkv) * hd + g * hd + e, 0] = 10.0 + g + 0.25 * e  # v[g][e]
    W = {"embed": np.ones((4, dim), np.float32), ("wqkv", 0): qkv, ("wo", 0): np.zeros((dim, nh * hd), np.float32),
         ("w1", 0): np.zeros((8, dim), np.float32), ("w3", 0): np.zeros((8, dim), np.float32),
         ("w2", 0): np.zeros((dim, 8), np.float32), ("attn_norm", 0): np.ones(dim, np.float32),
         ("ffn_norm", 0): np.ones(dim, np.float32), "final_norm": np.ones(dim, np.float32),
         "head": np.zeros((4, dim), np.float32)}
    return cfg, W


def _gqa_ctx(mod):
    cfg, W = _gqa_setup()
    orc = mod.OracleDecoder(cfg, W, 1)
    orc.step_one(0, np.array([0], np.int32))
    return orc.trace[("ctx", 0)].reshape(cfg.n_heads, cfg.head_dim)


def test_gqa_query_heads_read_their_group(ora):
    # One cached position: softmax weight exactly 1, so head i's context is v of its group.
    # repeat_kv expands [kv, n, ...] -> kv * n, so heads 0, 1 read group 0 and 2, 3 group 1.
    ctx = _gqa_ctx(_load_model())
    v = np.array([[10.0 + g + 0.25 * e for e in range(4)] for g in range(2)], np.float32)
    np.testing.assert_array_equal(ctx, v[[0, 0, 1, 1]])


def test_gqa_interleaved_grouping_slip_is_caught(ora):
    ctx = _gqa_ctx(_load_model(("g = i // G", "g = i % nkv")))
    v = np.array([[10.0 + g + 0.25 * e for e in range(4)] for g in range(2)], np.float32)
    assert not np.array_equal(ctx, v[[0, 0, 1, 1]])


# ------------------------------------------------------------- Fish MCF embedding, by hand
def _mcf_cfg():
    # 3 codebooks of 4 codes: 1/sqrt(3 + 1) = 0.5 exactly; semantic ids 10..19.
    return _toy_cfg(dim=4, vocab=32, n_codebooks=3, codebook_size=4, semantic_begin=10, semantic_end=19,
                    tied_embedding=1)


def _mcf_weights():
    dim = 4
    embed = np.zeros((32, dim), np.float32)
    embed[12] = [8.0, 4.0, -2.0, 1.0]
    embed[3] = [1.0, 2.0, 3.0, 4.0]
    cb = np.zeros((12, dim), np.float32)
    # row code + i * 4 of codebook i: a distinct power of two per (codebook, code)
    for i in range(3):
        for code in range(4):
            cb[code + 4 * i] = np.float32(2.0 ** (4 * i + code)) * np.array([1, 0, 0, 1], np.float32)
    return {"embed": embed, "codebook": cb, "head": np.zeros((32, dim), np.float32)}


def test_mcf_embedding_semantic_and_text_positions(ora):
    orc = _load_model().OracleDecoder(_mcf_cfg(), _mcf_weights(), 1)
    # semantic id 12 with codes (1, 2, 3): rows 1, 4 + 2, 8 + 3 -> 2^1 + 2^6 + 2^11 = 2114 on dims 0 and 3
    got = orc.embed(np.array([12, 1, 2, 3], np.int32))
    np.testing.assert_array_equal(got, np.array([(8 + 2114) * 0.5, 4 * 0.5, -2 * 0.5, (1 + 2114) * 0.5], np.float32))
    # text id 3: codebook sum zeroed and no scale, whatever the codes
    got = orc.embed(np.array([3, 1, 2, 3], np.int32))
    np.testing.assert_array_equal(got, np.array([1, 2, 3, 4], np.float32))


def test_mcf_embedding_gathers_the_dense_table_not_the_head(ora):
    W = _mcf_weights()
    W["head"] = np.full((32, 4), 99.0, np.float32)  # the tied head's rows must not be read
    orc = _load_model().OracleDecoder(_mcf_cfg(), W, 1)
    np.testing.assert_array_equal(orc.embed(np.array([3, 0, 0, 0], np.int32)), np.array([1, 2, 3, 4], np.float32))


@pytest.mark.parametrize("slip", [
    ("e = self.W[\"codebook\"][int(frame[1 + i]) + i * c.codebook_size]", "e = self.W[\"codebook\"][int(frame[1 + i])]"),
    ("(inv_scale if sem else np.float32(1.0))", "inv_scale"),
    ("vq * np.float32(1.0 if sem else 0.0)", "vq"),
])
def test_mcf_slip_is_caught(ora, slip):
    orc = _load_model(slip).OracleDecoder(_mcf_cfg(), _mcf_weights(), 1)
    a = orc.embed(np.array([12, 1, 2, 3], np.int32))
    b = orc.embed(np.array([3, 1, 2, 3], np.int32))
    ok = (np.array_equal(a, np.array([(8 + 2114) * 0.5, 2, -1, (1 + 2114) * 0.5], np.float32))
          and np.array_equal(b, np.array([1, 2, 3, 4], np.float32)))
    assert not ok


# ------------------------------------------------------------- dense-convention fixtures
def test_linear_fixture_pins_the_nk_convention(ora):
    """linear.json: y = x W^T + b with W stored [out, in] (PARITY.md 4.3) -- the convention
    of every QMatMul here (weights [N, K], blocks along K)."""
    with open(os.path.join(GOLD, "linear.json")) as f:
        d = json.load(f)
    W = np.asarray(d["input"]["W"], np.float32)
    x = np.asarray(d["input"]["x"], np.float32)
    b = np.asarray(d["input"]["b"], np.float32)
    cfg = _toy_cfg(dim=W.shape[1], weight_dtype=0)
    orc = _load_model().OracleDecoder(cfg, {}, 1)
    orc.margins = []
    got = np.stack([orc._mm(r, W) + b for r in x])
    np.testing.assert_allclose(got, np.asarray(d["data"]).reshape(d["shape"]), atol=d["tol"], rtol=0)
    # the transposed reading (W as [in, out]) cannot even be applied to this x
    assert W.T.shape[1] != x.shape[1]


def test_matmul_fixture(ora):
    with open(os.path.join(GOLD, "matmul.json")) as f:
        d = json.load(f)
    A = np.asarray(d["input"]["A"], np.float32)
    B = np.asarray(d["input"]["B"], np.float32)
    cfg = _toy_cfg(weight_dtype=0)
    orc = _load_model().OracleDecoder(cfg, {}, 1)
    orc.margins = []
    # matmul(A, B) = rows of A against the columns of B, i.e. the [N, K] weight B^T
    got = np.stack([orc._mm(r, B.T.copy()) for r in A])
    np.testing.assert_array_equal(got, np.asarray(d["data"], np.float32).reshape(d["shape"]))


def test_causal_mask_fixture_is_the_cache_prefix(ora):
    """causal_mask.json: query i sees keys j <= i.  A decode step attends exactly the cache
    prefix it has appended, so softmax(s + mask) row i equals the softmax over keys 0..i."""
    with open(os.path.join(GOLD, "causal_mask.json")) as f:
        d = json.load(f)
    mask = np.array([[-np.inf if v == "-inf" else v for v in row] for row in d["data"]], np.float32)
    T = d["input"]["T"]
    rng = np.random.default_rng(3)
    hd = 8
    q = rng.standard_normal((T, hd)).astype(np.float32)
    k = rng.standard_normal((T, hd)).astype(np.float32)
    v = rng.standard_normal((T, hd)).astype(np.float32)
    scale = np.float32(1.0 / np.sqrt(hd))
    for i in range(T):
        s = (k.astype(np.float64) @ q[i].astype(np.float64) * scale).astype(np.float32) + mask[i]
        p = ora.softmax(s)
        want = (p[: i + 1].astype(np.float64) @ v[: i + 1].astype(np.float64))
        got = ora.attend_one(q[i], k[: i + 1], v[: i + 1])
        np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)
        assert (p[i + 1:] == 0).all()
