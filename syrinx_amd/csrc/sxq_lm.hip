// sxq_lm.hip -- the decoder-step engine behind sxq_lm_* (include/sxq.h).
//
// One object holds a model's projections in the GEMV device layout (q|k|v and
// gate|up fused row-wise, which leaves every output row's vec-dot unchanged), its
// norm weights, RoPE tables, a preallocated per-stream KV cache and the step's
// activation buffers.  A step is a fixed kernel sequence over fixed buffers, so it is
// captured once per batch size as a HIP graph and replayed per token; the only
// per-token host work is copying ids in and logits out.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdlib>
#include <cstring>
#include <algorithm>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "sxq_abi.h"
#include "sxq_decoder.h"

using namespace sxq;
using namespace sxq::abi;

namespace {


struct DevWeight {
    void* mem = nullptr;
    size_t hdr_pad = 0;
    QWeight w;
};

struct LmLayer {
    DevWeight wqkv, wo, w13, w2;
    float *attn_norm = nullptr, *ffn_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr, *bqkv = nullptr;
    float* bo = nullptr;  // wo bias (models with o_bias)
};

// A captured step is specific to its stream count, its input (ids or embeddings) and the
// trace buffer it records into (a graph keeps the pointer it was captured with).
struct GraphKey {
    int n;
    bool embeds;
    const float* trace;
    int splits;  // attention splits per (stream, KV head) in the grid
    bool operator<(const GraphKey& o) const {
        if (n != o.n) return n < o.n;
        if (embeds != o.embeds) return embeds < o.embeds;
        if (splits != o.splits) return splits < o.splits;
        return trace < o.trace;
    }
};

}  // namespace

struct sxq_lm {
    int device = 0;
    sxq_lm_config c{};
    int vdt = 0;            // activation (vec-dot) block type
    int qkv_n = 0, ctx = 0, ids_per = 1, max_splits = 0;
    int64_t kv_stream_stride = 0, kv_layer_stride = 0;
    std::vector<LmLayer> layers;
    DevWeight head;
    // embed: the dense input table; allocated at create for an untied model, on the first
    // SXQ_LM_EMBED upload for a tied one (until then a tied model embeds through the
    // dequantized head rows)
    float *head_bias = nullptr, *final_norm = nullptr, *embed = nullptr, *cb_embed = nullptr;
    int embed_scheme = 0;            // SXQ_EMBED_INT8 / _INT4 when the input table is held quantized
    uint8_t* embed_q = nullptr;      // its codes, and per-row scales
    float* embed_scale = nullptr;
    float *rope_cos = nullptr, *rope_sin = nullptr;
    float *kc = nullptr, *vc = nullptr;
    int* d_len = nullptr;
    std::vector<int> h_len;
    float *h = nullptr, *qkv = nullptr, *qbuf = nullptr, *part = nullptr, *gu = nullptr, *logits = nullptr;
    float* hn = nullptr;  // post-final-RMSNorm hidden of the step [max_batch][dim] (SlowAr::head's `hidden`)
    uint8_t *act_a = nullptr, *act_o = nullptr, *act_d = nullptr;
    // the same activations as matrix-core operand records (Q8_K models, 5..16 streams)
    MmaRec *rec_a = nullptr, *rec_o = nullptr, *rec_d = nullptr;
    int *d_ids = nullptr, *d_next = nullptr;
    float* am_val = nullptr;        // argmax partials [max_batch * kArgmaxSlices]
    int* am_idx = nullptr;
    unsigned* am_count = nullptr;   // per-stream arrival counters (zero between steps), kCounterStride apart
    unsigned* attn_count = nullptr; // per-(stream, KV head) arrival counters of the fused attention, likewise
    bool attn_fused = false;
    // one decode row: attention and the O projection as one launch, which waits on
    // per-layer counters (layer l's launch zeroes layer l + 1's); wo_dirty: a step was
    // enqueued only in part, so the counters are zeroed before the next one
    bool wo_fused = false, wo_dirty = false;
    unsigned* wo_ready = nullptr;  // [n_layers][kReadyCopies], likewise
    GemvRecWs rec_ws;              // 5..16 streams: the matrix-core GEMV's K-split workspace
    // one stream through the fused attention: stream 0's RoPE row, copied by the step's
    // embedding kernel (null: SXQ_ATTN_SPEC=0, the attention reads the tables after the length)
    float* rope_row = nullptr;
    bool swiglu = false;        // one decode row: gate|up GEMV with SwiGLU epilogue + quantizing down GEMV
    float* act_f32 = nullptr;   // SwiGLU output row of that pair [max_batch][intermediate]
    float* trace = nullptr;  // optional f32 record of every intermediate of a step (tests)
    int grid_splits = 0;     // attention splits the step being enqueued launches (0: all of max_seq)
    hipStream_t cap = nullptr;
    std::map<GraphKey, hipGraphExec_t> graphs;
    std::map<std::string, hipGraphExec_t> expand_graphs;  // keyed by the raw bytes of the arguments
    void* pf = nullptr;  // prefill workspace, grown to the largest prompt batch so far
    size_t pf_size = 0;
    std::vector<void*> allocs;
    std::mutex mu;
};

namespace {

// Rows of the dense input table (a tied model's is the head's source: vocab rows).
int64_t embed_rows(const sxq_lm_config& c) { return c.embed_rows > 0 && !c.tied_embedding ? c.embed_rows : c.vocab; }

hipError_t dalloc(sxq_lm* lm, void** p, size_t bytes) {
    hipError_t e = hipMalloc(p, bytes ? bytes : 1);
    if (e == hipSuccess) lm->allocs.push_back(*p);
    return e;
}

hipError_t alloc_weight(sxq_lm* lm, DevWeight& d, int dtype, int64_t n, int64_t k) {
    const int64_t nb = k / block_size(dtype), nblk = n * nb;
    const size_t hb = (size_t)nblk * weight_hdr_bytes(dtype);
    d.hdr_pad = (hb + 255) & ~(size_t)255;
    const size_t qb = (size_t)nblk * weight_qs_bytes(dtype);
    hipError_t e = dalloc(lm, &d.mem, d.hdr_pad + qb);
    if (e != hipSuccess) return e;
    d.w.dtype = dtype;
    d.w.n = n;
    d.w.k = k;
    d.w.nb = nb;
    d.w.hdr = (const uint8_t*)d.mem;
    d.w.qs = (const uint8_t*)d.mem + d.hdr_pad;
    return hipSuccess;
}

// Copy rows [0, src.n) of a device-layout weight into rows [r0, r0 + src.n) of dst.
hipError_t copy_rows(DevWeight& dst, const QWeight& src, int64_t r0, hipStream_t s) {
    const size_t hb = weight_hdr_bytes(dst.w.dtype), qb = weight_qs_bytes(dst.w.dtype);
    const size_t rows_blk = (size_t)src.n * (size_t)src.nb;
    hipError_t e = hipMemcpyAsync((uint8_t*)dst.w.hdr + (size_t)r0 * dst.w.nb * hb, src.hdr, rows_blk * hb,
                                  hipMemcpyDeviceToDevice, s);
    if (e != hipSuccess) return e;
    return hipMemcpyAsync((uint8_t*)dst.w.qs + (size_t)r0 * dst.w.nb * qb, src.qs, rows_blk * qb,
                          hipMemcpyDeviceToDevice, s);
}

// Fill rows [r0, r0 + n) of dst with from_float(N(0, std)) in row chunks; keep_f32 (or
// null) receives the f32 rows before quantization ([n][k], row r0 first).
hipError_t random_rows(DevWeight& dst, int64_t r0, int64_t n, uint64_t seed, float stdv, float* tmp_f32,
                       uint8_t* tmp_blk, int64_t tmp_elems, hipStream_t s, float* keep_f32 = nullptr) {
    const int64_t k = dst.w.k, nb = dst.w.nb;
    const int64_t chunk = tmp_elems / k;
    for (int64_t a = 0; a < n; a += chunk) {
        const int64_t rows = n - a < chunk ? n - a : chunk;
        hipError_t e = launch_fill_normal(tmp_f32, rows * k, seed * 1000003ull + (uint64_t)a, 0.0f, stdv, s);
        if (e == hipSuccess && keep_f32)
            e = hipMemcpyAsync(keep_f32 + a * k, tmp_f32, sizeof(float) * rows * k, hipMemcpyDeviceToDevice, s);
        if (e == hipSuccess) e = launch_from_float(dst.w.dtype, tmp_f32, rows * nb, tmp_blk, s);
        QWeight part = dst.w;
        const size_t hb = weight_hdr_bytes(dst.w.dtype), qb = weight_qs_bytes(dst.w.dtype);
        part.hdr = dst.w.hdr + (size_t)(r0 + a) * nb * hb;
        part.qs = dst.w.qs + (size_t)(r0 + a) * nb * qb;
        if (e == hipSuccess) e = launch_repack(dst.w.dtype, tmp_blk, rows * nb, (void*)part.hdr, (void*)part.qs, true, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

void drop_graphs(sxq_lm* lm) {
    for (auto& kv : lm->graphs) (void)hipGraphExecDestroy(kv.second);
    lm->graphs.clear();
    for (auto& kv : lm->expand_graphs) (void)hipGraphExecDestroy(kv.second);
    lm->expand_graphs.clear();
}

// Attention splits (of kAttnSplitFused positions) per (stream, KV head) the next step's
// grid holds: enough for the longest of its n streams, rounded up to a bucket of
// kSplitBucket so that a captured step serves several lengths.
constexpr int kSplitBucket = 4;
int step_grid_splits(const sxq_lm* lm, int n) {
    const int all = (lm->c.max_seq + kAttnSplitFused - 1) / kAttnSplitFused;
    static const bool full = getenv("SXQ_ATTN_FULL_GRID") != nullptr;  // A/B: the grid of every split
    if (full) return all;
    int need = 1;
    for (int s = 0; s < n; ++s) need = std::max(need, (lm->h_len[s] + kAttnSplitFused) / kAttnSplitFused);
    return std::min(all, (need + kSplitBucket - 1) / kSplitBucket * kSplitBucket);
}

// Per-layer trace segments (each [n, size] f32): hn_attn, qkv, q, ctx, h_mid, hn_ffn,
// gu, act, h_out; preceded by the embedding output and followed by hn_final.
size_t trace_layer_floats(const sxq_lm* lm, int n) {
    const sxq_lm_config& c = lm->c;
    return (size_t)n * (4 * (size_t)c.dim + lm->qkv_n + 2 * (size_t)lm->ctx + 3 * (size_t)c.intermediate);
}
size_t trace_floats(const sxq_lm* lm, int n) {
    return 2 * (size_t)n * lm->c.dim + (size_t)lm->c.n_layers * trace_layer_floats(lm, n);
}

hipError_t enqueue_step(sxq_lm* lm, int n, bool from_embeds, hipStream_t s) {
    const sxq_lm_config& c = lm->c;
    hipError_t e = hipSuccess;
#define STEP(x)                      \
    do {                             \
        e = (x);                     \
        if (e != hipSuccess) return e; \
    } while (0)
    float* tr = lm->trace;
    auto record = [&](const float* src, size_t floats) -> hipError_t {
        hipError_t r = hipMemcpyAsync(tr, src, floats * sizeof(float), hipMemcpyDeviceToDevice, s);
        tr += floats;
        return r;
    };
    auto slot = [&](size_t floats) {
        float* p = tr;
        tr += floats;
        return p;
    };
    // one stream through the fused attention: the embedding kernel also copies the step's
    // RoPE row, so that the attention splits issue their loads before the length returns
    const bool spec = lm->rope_row && n == 1 && lm->wo_fused && !from_embeds && !lm->embed_scheme;
    RopeRow rr;
    if (spec) {
        rr.len = lm->d_len;
        rr.cos_t = lm->rope_cos;
        rr.sin_t = lm->rope_sin;
        rr.half = c.head_dim / 2;
        rr.out = lm->rope_row;
    }
    if (!from_embeds) {
        if (c.n_codebooks > 0 || (c.tied_embedding && !lm->embed))
            STEP(launch_embed_mcf(lm->d_ids, lm->ids_per, n, lm->embed, embed_rows(c), lm->head.w, c.dim, lm->cb_embed,
                                  c.n_codebooks, c.codebook_size, c.semantic_begin, c.semantic_end, lm->h, s, rr));
        else if (lm->embed_scheme)
            STEP(launch_embed_gather(lm->embed_scheme, lm->embed_q, lm->embed_scale, embed_rows(c),
                                     c.dim, lm->d_ids, lm->ids_per, n, lm->h, s));
        else
            STEP(launch_embed_dense(lm->d_ids, lm->ids_per, n, lm->embed, embed_rows(c), c.dim,
                                    lm->h, s, rr));
    }
    if (tr) STEP(record(lm->h, (size_t)n * c.dim));
    const bool wo_fused = lm->wo_fused && n == 1;
    if (lm->wo_dirty) {
        STEP(launch_fill_int((int*)lm->wo_ready, c.n_layers * kReadyCopies * kCounterStride, 0, s));
        lm->wo_dirty = false;
    }
    lm->wo_dirty = wo_fused;  // until the whole step is enqueued
    const int I = c.intermediate;
    const size_t nd = (size_t)n * c.dim;
    auto norm_in = [&](const float* x, const float* w, float* normed) {
        NormIn ni;
        ni.x = x;
        ni.w = w;
        ni.eps = c.norm_eps;
        ni.normed = normed;
        return ni;
    };
    // 5..16 streams of a Q8_K model: the quantizers also write the matrix-core operand
    // records, which the Q4_K GEMVs then read (each producer and its consumer get the same
    // pointer; a GEMV that does not take records reads the Q8_K rows as before)
    const bool rec_ok = n >= 5 && n <= 16 && lm->rec_a != nullptr;
    MmaRec* rec_a = rec_ok ? lm->rec_a : nullptr;
    MmaRec* rec_o = rec_ok && lm->attn_fused && !wo_fused ? lm->rec_o : nullptr;
    MmaRec* rec_d = rec_ok ? lm->rec_d : nullptr;
    for (int l = 0; l < c.n_layers; ++l) {
        LmLayer& L = lm->layers[l];
        float* kc = lm->kc + (int64_t)l * lm->kv_layer_stride;
        float* vc = lm->vc + (int64_t)l * lm->kv_layer_stride;
        STEP(launch_gemv_rmsnorm(L.wqkv.w, norm_in(lm->h, L.attn_norm, tr ? slot(nd) : nullptr), n, lm->act_a, lm->qkv,
                                 lm->qkv_n, L.bqkv, nullptr, 0, s, rec_a));
        if (tr) STEP(record(lm->qkv, (size_t)n * lm->qkv_n));
        const float* qn = c.qk_norm ? L.q_norm : nullptr;
        const float* kn = c.qk_norm ? L.k_norm : nullptr;
        if (lm->attn_fused) {
            float* q_slot = tr ? slot((size_t)n * lm->ctx) : nullptr;
            float* ctx_slot = tr ? slot((size_t)n * lm->ctx) : nullptr;
            if (wo_fused)
                STEP(launch_attention_wo_decode(lm->vdt, lm->qkv, lm->qkv_n, c.n_heads, c.n_kv_heads, c.head_dim, qn, kn,
                                                c.norm_eps, c.rope_interleaved, lm->rope_cos, lm->rope_sin, lm->d_len,
                                                kc, vc, c.max_seq, lm->max_splits, lm->part, lm->attn_count, lm->act_o,
                                                L.wo.w, lm->h, lm->wo_ready + (size_t)l * kReadyCopies * counter_stride(),
                                                lm->wo_ready + (size_t)((l + 1) % c.n_layers) * kReadyCopies * counter_stride(),
                                                ctx_slot, q_slot, s, lm->grid_splits, spec ? lm->rope_row : nullptr));
            else
                STEP(launch_attention_decode(lm->vdt, lm->qkv, n, lm->qkv_n, c.n_heads, c.n_kv_heads, c.head_dim, qn,
                                             kn, c.norm_eps, c.rope_interleaved, lm->rope_cos, lm->rope_sin, lm->d_len,
                                             kc, vc, lm->kv_stream_stride, c.max_seq, lm->max_splits, lm->part,
                                             lm->attn_count, lm->act_o, ctx_slot, q_slot, s, rec_o, lm->grid_splits));
        } else {
            STEP(launch_qk_rope_append(lm->qkv, n, lm->qkv_n, c.n_heads, c.n_kv_heads, c.head_dim, qn, kn, c.norm_eps,
                                       c.rope_interleaved, lm->rope_cos, lm->rope_sin, lm->d_len, lm->qbuf, kc, vc,
                                       lm->kv_stream_stride, c.max_seq, s));
            if (tr) STEP(record(lm->qbuf, (size_t)n * lm->ctx));
            STEP(launch_attention(lm->vdt, lm->qbuf, kc, vc, lm->d_len, n, c.n_heads, c.n_kv_heads, c.head_dim,
                                  c.max_seq, lm->kv_stream_stride, kAttnSplit, lm->max_splits, lm->part, lm->act_o,
                                  tr ? slot((size_t)n * lm->ctx) : nullptr, s));
        }
        if (!wo_fused) STEP(launch_gemv_rec(L.wo.w, lm->act_o, rec_o, n, lm->h, c.dim, L.bo, lm->h, c.dim, s, &lm->rec_ws));
        if (tr) STEP(record(lm->h, nd));
        if (lm->swiglu && n == 1) {
            STEP(launch_swiglu_pair(L.w13.w, L.w2.w, norm_in(lm->h, L.ffn_norm, tr ? slot(nd) : nullptr), lm->gu,
                                    lm->act_f32, lm->h, lm->h, s));
            if (tr) STEP(record(lm->gu, (size_t)2 * I));
            if (tr) STEP(record(lm->act_f32, (size_t)I));
        } else {
            STEP(launch_gemv_rmsnorm(L.w13.w, norm_in(lm->h, L.ffn_norm, tr ? slot(nd) : nullptr), n, lm->act_a,
                                     lm->gu, 2 * I, nullptr, nullptr, 0, s, rec_a));
            if (tr) STEP(record(lm->gu, (size_t)n * 2 * I));
            STEP(launch_silu_mul_quant(lm->vdt, lm->gu, n, I, lm->act_d, tr ? slot((size_t)n * I) : nullptr, s, rec_d));
            STEP(launch_gemv_rec(L.w2.w, lm->act_d, rec_d, n, lm->h, c.dim, nullptr, lm->h, c.dim, s, &lm->rec_ws));
        }
        if (tr) STEP(record(lm->h, nd));
    }
    STEP(launch_gemv_rmsnorm(lm->head.w, norm_in(lm->h, lm->final_norm, lm->hn), n, lm->act_a, lm->logits, c.vocab,
                             c.head_bias ? lm->head_bias : nullptr, nullptr, 0, s, rec_a));
    if (tr) STEP(record(lm->hn, nd));
    STEP(launch_argmax(lm->logits, n, c.vocab, lm->d_ids, lm->ids_per, lm->d_next, lm->d_len, lm->am_val, lm->am_idx,
                       lm->am_count, s));
#undef STEP
    lm->wo_dirty = false;
    return hipSuccess;
}

// FastAr::expand_batch (crates/syrinx-fish/src/s2/fast_ar.rs:170-224) as one kernel
// sequence over the engine's buffers: the cache emptied (a fresh KvCache), position 0 run
// on the slow hidden (its logits unused), codebook 0 = first_code of the semantic id, then
// positions 1..n_codes-1 each embed the previous code (the dense shared table) and draw the
// next code from their logits on the device -- into the engine's ids (the next input) and
// into codes[s * codes_stride + cb].
constexpr size_t kMaxExpandGraphs = 16;  // captured expansions kept per engine

struct ExpandArgs {
    int n;
    const float* hidden;
    const int32_t* semantic;
    int sem_stride;
    const int32_t* active;
    sxq_fish_sampling p;
    uint64_t* rng;
    int n_codes;
    int32_t* codes;
    int codes_stride;
};

hipError_t enqueue_expand(sxq_lm* lm, const ExpandArgs& a, hipStream_t s) {
    const sxq_lm_config& c = lm->c;
    lm->grid_splits = 0;  // the expansion's positions run from 0 to n_codes - 1: every split
    hipError_t e = launch_fill_int(lm->d_len, a.n, 0, s);
    if (e == hipSuccess)
        e = hipMemcpyAsync(lm->h, a.hidden, sizeof(float) * (size_t)a.n * c.dim, hipMemcpyDeviceToDevice, s);
    if (e == hipSuccess) e = enqueue_step(lm, a.n, true, s);
    if (e == hipSuccess)
        e = launch_first_codes(a.semantic, a.sem_stride, a.n, a.p.semantic_begin, c.vocab, a.active, lm->d_ids, a.codes,
                               a.codes_stride, s);
    for (int cb = 1; cb < a.n_codes && e == hipSuccess; ++cb) {
        e = enqueue_step(lm, a.n, false, s);
        if (e == hipSuccess)
            e = launch_sample_codebook(lm->logits, c.vocab, a.n, c.vocab, a.p, a.rng, a.active, lm->d_ids, 1,
                                       a.codes + cb, a.codes_stride, s);
    }
    return e;
}

std::string expand_key(const ExpandArgs& a) {
    std::string k;
    auto put = [&](const void* p, size_t b) { k.append((const char*)p, b); };
    put(&a.n, sizeof a.n);
    put(&a.hidden, sizeof a.hidden);
    put(&a.semantic, sizeof a.semantic);
    put(&a.sem_stride, sizeof a.sem_stride);
    put(&a.active, sizeof a.active);
    put(&a.p.temperature, sizeof(float));
    put(&a.p.top_p, sizeof(float));
    put(&a.p.top_k, sizeof(int32_t));
    put(&a.p.repetition_penalty, sizeof(float));
    put(&a.p.semantic_begin, sizeof(int32_t));
    put(&a.rng, sizeof a.rng);
    put(&a.n_codes, sizeof a.n_codes);
    put(&a.codes, sizeof a.codes);
    put(&a.codes_stride, sizeof a.codes_stride);
    return k;
}

void destroy_lm(sxq_lm* lm) {
    for (auto& kv : lm->graphs) (void)hipGraphExecDestroy(kv.second);
    for (auto& kv : lm->expand_graphs) (void)hipGraphExecDestroy(kv.second);
    if (lm->pf) (void)hipFree(lm->pf);
    if (lm->cap) (void)hipStreamDestroy(lm->cap);
    for (void* p : lm->allocs) (void)hipFree(p);
    delete lm;
}

sxq_status check_config(const sxq_lm_config* c) {
    if (!c) return fail(SXQ_ERR_INVALID, "lm_create: null config");
    if (c->n_layers <= 0 || c->dim <= 0 || c->n_heads <= 0 || c->n_kv_heads <= 0 || c->head_dim <= 0 ||
        c->intermediate <= 0 || c->vocab <= 0 || c->max_seq <= 0)
        return fail(SXQ_ERR_INVALID, "lm_create: every size in the config must be positive");
    if (c->max_batch < 1 || c->max_batch > 16) return fail(SXQ_ERR_INVALID, "lm_create: max_batch must be 1..16");
    if (c->n_heads % c->n_kv_heads) return fail(SXQ_ERR_SHAPE, "lm_create: n_heads %% n_kv_heads != 0");
    if (c->head_dim > 256 || c->head_dim < 32 || c->head_dim % 8)
        return fail(SXQ_ERR_SHAPE, "lm_create: head_dim must be a multiple of 8 in [32, 256]");
    if (c->max_seq > kMaxSplits * kAttnSplit)
        return fail(SXQ_ERR_INVALID, "lm_create: max_seq %d exceeds %d positions", c->max_seq, kMaxSplits * kAttnSplit);
    const int dt = c->weight_dtype;
    if (dt != kQ4K && dt != kQ8_0 && dt != kQ4_0) return fail(SXQ_ERR_DTYPE, "lm_create: weight dtype %d not supported", dt);
    const int bs = block_size(dt);
    if (c->dim % bs || (c->n_heads * c->head_dim) % bs || c->intermediate % bs)
        return fail(SXQ_ERR_BLOCK_ALIGN,
                    "lm_create: dim %d, n_heads*head_dim %d and intermediate %d must be multiples of the block size %d",
                    c->dim, c->n_heads * c->head_dim, c->intermediate, bs);
    if (c->n_codebooks < 0 || (c->n_codebooks > 0 && c->codebook_size <= 0))
        return fail(SXQ_ERR_INVALID, "lm_create: codebooks need codebook_size > 0");
    return SXQ_OK;
}

// ---- prompt prefill -----------------------------------------------------------------

// One projection of T prompt rows: x_f32 [T][k] (f32 rows) and act (the same rows as
// device activation blocks) -> y [T][n] (+ bias, then res + that).  Q4_K: the f16 MFMA GEMM
// from kGemmMinRows rows unless `exact`; Q8_0 / Q4_0: the int8 matrix-core GEMM from
// kGemmQ80MinRows rows; otherwise the GEMV, 16 rows at a time (Candle's bits).
hipError_t pf_proj(const sxq_lm* lm, const QWeight& w, const float* x, const uint8_t* act, int T, float* y,
                   const float* bias, const float* res, bool exact, void* gemm_ws, hipStream_t s) {
    const int64_t n = w.n;
    if (w.dtype == kQ4K && !exact && T >= kGemmMinRows) {
        hipError_t e = launch_gemm_q4k_prep(x, w.k, T, n, (int)w.k, gemm_ws, s);
        return e == hipSuccess ? launch_gemm_q4k(w, gemm_ws, T, y, n, bias, res, n, s) : e;
    }
    if (w.dtype != kQ4K && T >= kGemmQ80MinRows) return launch_gemm_q80(w, act, T, y, n, bias, res, n, s);
    const size_t rowb = (size_t)(w.k / block_size(lm->vdt)) * act_block_bytes(lm->vdt);
    for (int r0 = 0; r0 < T; r0 += 16) {
        const int mm = T - r0 < 16 ? T - r0 : 16;
        hipError_t e = launch_gemv(w, act + (size_t)r0 * rowb, mm, y + (int64_t)r0 * n, n, bias,
                                   res ? res + (int64_t)r0 * n : nullptr, n, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// Device buffers of one prefill of T tokens over n streams (offsets into lm->pf).
struct PfLayout {
    size_t h, hn, qkv, q, cx, gu, af, act, gemm, tok, tiles, last, total;
};

PfLayout pf_layout(const sxq_lm* lm, int T, int n) {
    const sxq_lm_config& c = lm->c;
    auto up = [](size_t v) { return (v + 255) & ~(size_t)255; };
    const size_t bs = block_size(lm->vdt), ab = act_block_bytes(lm->vdt);
    int64_t kmax = c.dim > lm->ctx ? c.dim : lm->ctx;
    if (c.intermediate > kmax) kmax = c.intermediate;
    size_t gemm = 0;
    if (c.weight_dtype == kQ4K) {
        const LmLayer& L = lm->layers[0];
        for (const QWeight* w : {&L.wqkv.w, &L.wo.w, &L.w13.w, &L.w2.w}) {
            const size_t g = gemm_q4k_workspace(w->n, T, w->k);
            if (g > gemm) gemm = g;
        }
        const size_t g = gemm_q4k_workspace(lm->head.w.n, T, lm->head.w.k);
        if (g > gemm) gemm = g;
    }
    PfLayout p{};
    size_t o = 0;
    auto take = [&](size_t bytes) {
        const size_t at = o;
        o += up(bytes);
        return at;
    };
    p.h = take(sizeof(float) * (size_t)T * c.dim);
    p.hn = take(sizeof(float) * (size_t)T * c.dim);
    p.qkv = take(sizeof(float) * (size_t)T * lm->qkv_n);
    p.q = take(sizeof(float) * (size_t)T * lm->ctx);
    p.cx = take(sizeof(float) * (size_t)T * lm->ctx);
    p.gu = take(sizeof(float) * (size_t)T * 2 * c.intermediate);
    p.af = take(sizeof(float) * (size_t)T * c.intermediate);
    p.act = take((size_t)T * (size_t)(kmax / (int64_t)bs) * ab);
    p.gemm = take(gemm);
    p.tok = take(sizeof(int) * 2 * (size_t)T);
    p.tiles = take(sizeof(int) * 4 * (size_t)(T + n));
    p.last = take(sizeof(int) * (size_t)n);
    p.total = o;
    return p;
}

size_t pf_trace_floats(const sxq_lm* lm, int T) { return trace_floats(lm, T); }

hipError_t enqueue_prefill(sxq_lm* lm, const PrefillMeta& pm, int T, const int* ids, const float* embeds,
                           float* logits_all, float* hidden_all, bool exact, float* tr, hipStream_t s) {
    const sxq_lm_config& c = lm->c;
    const PfLayout P = pf_layout(lm, T, pm.n);
    uint8_t* base = (uint8_t*)lm->pf;
    float* h = (float*)(base + P.h);
    float* hn = (float*)(base + P.hn);
    float* qkv = (float*)(base + P.qkv);
    float* q = (float*)(base + P.q);
    float* cx = (float*)(base + P.cx);
    float* gu = (float*)(base + P.gu);
    float* af = (float*)(base + P.af);
    uint8_t* act = base + P.act;
    void* gws = base + P.gemm;
    int* tok = (int*)(base + P.tok);
    int* tiles = (int*)(base + P.tiles);
    int* last = (int*)(base + P.last);
    const int I = c.intermediate, n = pm.n;
    const size_t Td = (size_t)T * c.dim;
    hipError_t e = hipSuccess;
#define PF(x)                          \
    do {                               \
        e = (x);                       \
        if (e != hipSuccess) return e; \
    } while (0)
    auto record = [&](const float* src, size_t floats) -> hipError_t {
        if (!tr) return hipSuccess;
        hipError_t r = hipMemcpyAsync(tr, src, floats * sizeof(float), hipMemcpyDeviceToDevice, s);
        tr += floats;
        return r;
    };
    int n_tiles = 0;
    for (int i = 0; i < n; ++i) n_tiles += (pm.counts[i] + pm.tile_tokens - 1) / pm.tile_tokens;
    PF(launch_prefill_tables(pm, T, tok, tiles, last, s));
    if (embeds) {
        PF(hipMemcpyAsync(h, embeds, sizeof(float) * Td, hipMemcpyDeviceToDevice, s));
    } else if (c.n_codebooks > 0 || (c.tied_embedding && !lm->embed)) {
        PF(launch_embed_mcf(ids, lm->ids_per, T, lm->embed, embed_rows(c), lm->head.w, c.dim, lm->cb_embed,
                            c.n_codebooks, c.codebook_size, c.semantic_begin, c.semantic_end, h, s));
    } else {
        if (lm->embed_scheme)
            PF(launch_embed_gather(lm->embed_scheme, lm->embed_q, lm->embed_scale, embed_rows(c),
                                   c.dim, ids, lm->ids_per, T, h, s));
        else
            PF(launch_embed_dense(ids, lm->ids_per, T, lm->embed, embed_rows(c), c.dim, h, s));
    }
    PF(record(h, Td));
    for (int l = 0; l < c.n_layers; ++l) {
        LmLayer& L = lm->layers[l];
        float* kc = lm->kc + (int64_t)l * lm->kv_layer_stride;
        float* vc = lm->vc + (int64_t)l * lm->kv_layer_stride;
        PF(launch_rmsnorm_quant(lm->vdt, h, T, c.dim, L.attn_norm, c.norm_eps, act, hn, s));
        PF(record(hn, Td));
        PF(pf_proj(lm, L.wqkv.w, hn, act, T, qkv, L.bqkv, nullptr, exact, gws, s));
        PF(record(qkv, (size_t)T * lm->qkv_n));
        PF(launch_prefill_rope_kv(qkv, T, lm->qkv_n, c.n_heads, c.n_kv_heads, c.head_dim,
                                  c.qk_norm ? L.q_norm : nullptr, c.qk_norm ? L.k_norm : nullptr, c.norm_eps,
                                  c.rope_interleaved, lm->rope_cos, lm->rope_sin, tok, q, kc, vc,
                                  lm->kv_stream_stride, c.max_seq, s));
        PF(record(q, (size_t)T * lm->ctx));
        PF(launch_prefill_attn(q, kc, vc, tiles, n_tiles, c.n_heads, c.n_kv_heads, c.head_dim, c.max_seq,
                               lm->kv_stream_stride, cx, s));
        PF(record(cx, (size_t)T * lm->ctx));
        PF(launch_quantize_act(lm->vdt, false, cx, lm->ctx, T, lm->ctx, act, s));
        PF(pf_proj(lm, L.wo.w, cx, act, T, h, L.bo, h, exact, gws, s));
        PF(record(h, Td));
        PF(launch_rmsnorm_quant(lm->vdt, h, T, c.dim, L.ffn_norm, c.norm_eps, act, hn, s));
        PF(record(hn, Td));
        PF(pf_proj(lm, L.w13.w, hn, act, T, gu, nullptr, nullptr, exact, gws, s));
        PF(record(gu, (size_t)T * 2 * I));
        PF(launch_silu_mul_quant(lm->vdt, gu, T, I, act, af, s));
        PF(record(af, (size_t)T * I));
        PF(pf_proj(lm, L.w2.w, af, act, T, h, nullptr, h, exact, gws, s));
        PF(record(h, Td));
    }
    const float* hb = c.head_bias ? lm->head_bias : nullptr;
    if (logits_all) {  // the head over every prompt row (Qwen2Lm::forward_logits_cached)
        PF(launch_rmsnorm_quant(lm->vdt, h, T, c.dim, lm->final_norm, c.norm_eps, act, hn, s));
        PF(pf_proj(lm, lm->head.w, hn, act, T, logits_all, hb, nullptr, exact, gws, s));
        if (hidden_all) PF(hipMemcpyAsync(hidden_all, hn, sizeof(float) * Td, hipMemcpyDeviceToDevice, s));
        PF(record(hn, Td));
        PF(launch_gather_rows(hn, last, n, c.dim, lm->hn, s));
        PF(launch_gather_rows(logits_all, last, n, c.vocab, lm->logits, s));
    } else {  // the head on each stream's last row (SlowAr::head), as the decode step runs it
        PF(launch_gather_rows(h, last, n, c.dim, lm->h, s));
        NormIn ni;
        ni.x = lm->h;
        ni.w = lm->final_norm;
        ni.eps = c.norm_eps;
        ni.normed = lm->hn;
        PF(launch_gemv_rmsnorm(lm->head.w, ni, n, lm->act_a, lm->logits, c.vocab, hb, nullptr, 0, s));
        PF(record(lm->hn, (size_t)n * c.dim));
    }
    PF(launch_argmax(lm->logits, n, c.vocab, lm->d_ids, lm->ids_per, lm->d_next, nullptr, lm->am_val, lm->am_idx,
                     lm->am_count, s));
    PF(launch_prefill_advance(pm, lm->d_len, s));
#undef PF
    return hipSuccess;
}

}  // namespace

extern "C" {

sxq_status sxq_lm_create(int device, const sxq_lm_config* cfg, sxq_lm** out) {
    if (!out) return fail(SXQ_ERR_INVALID, "lm_create: null output handle");
    *out = nullptr;
    sxq_status st = check_config(cfg);
    if (st != SXQ_OK) return st;
    DeviceGuard g(device);
    HIP_TRY(g.err, "hipSetDevice");
    sxq_lm* lm = new sxq_lm();
    lm->device = device;
    lm->c = *cfg;
    const sxq_lm_config& c = lm->c;
    const int dt = c.weight_dtype;
    lm->vdt = vec_dot_type(dt);
    lm->ctx = c.n_heads * c.head_dim;
    lm->qkv_n = lm->ctx + 2 * c.n_kv_heads * c.head_dim;
    lm->ids_per = 1 + c.n_codebooks;
    lm->max_splits = (c.max_seq + kAttnSplit - 1) / kAttnSplit;
    lm->kv_stream_stride = (int64_t)c.n_kv_heads * c.max_seq * c.head_dim;
    lm->kv_layer_stride = lm->kv_stream_stride * c.max_batch;
    const int MB = c.max_batch, I = c.intermediate, hd = c.head_dim;
    hipError_t e = hipSuccess;
    auto A = [&](void** p, size_t bytes) {
        if (e == hipSuccess) e = dalloc(lm, p, bytes);
    };
    lm->layers.resize(c.n_layers);
    for (auto& L : lm->layers) {
        if (e == hipSuccess) e = alloc_weight(lm, L.wqkv, dt, lm->qkv_n, c.dim);
        if (e == hipSuccess) e = alloc_weight(lm, L.wo, dt, c.dim, lm->ctx);
        if (e == hipSuccess) e = alloc_weight(lm, L.w13, dt, 2 * (int64_t)I, c.dim);
        if (e == hipSuccess) e = alloc_weight(lm, L.w2, dt, c.dim, I);
        A((void**)&L.attn_norm, sizeof(float) * c.dim);
        A((void**)&L.ffn_norm, sizeof(float) * c.dim);
        A((void**)&L.q_norm, sizeof(float) * hd);
        A((void**)&L.k_norm, sizeof(float) * hd);
        A((void**)&L.bqkv, sizeof(float) * lm->qkv_n);
        if (c.o_bias) A((void**)&L.bo, sizeof(float) * c.dim);
    }
    if (e == hipSuccess) e = alloc_weight(lm, lm->head, dt, c.vocab, c.dim);
    A((void**)&lm->head_bias, sizeof(float) * c.vocab);
    A((void**)&lm->final_norm, sizeof(float) * c.dim);
    if (!c.tied_embedding) A((void**)&lm->embed, sizeof(float) * (size_t)embed_rows(c) * c.dim);
    if (c.n_codebooks > 0) A((void**)&lm->cb_embed, sizeof(float) * (size_t)c.n_codebooks * c.codebook_size * c.dim);
    A((void**)&lm->rope_cos, sizeof(float) * (size_t)c.max_seq * (hd / 2));
    A((void**)&lm->rope_sin, sizeof(float) * (size_t)c.max_seq * (hd / 2));
    A((void**)&lm->kc, sizeof(float) * (size_t)lm->kv_layer_stride * c.n_layers);
    A((void**)&lm->vc, sizeof(float) * (size_t)lm->kv_layer_stride * c.n_layers);
    A((void**)&lm->d_len, sizeof(int) * MB);
    A((void**)&lm->h, sizeof(float) * (size_t)MB * c.dim);
    A((void**)&lm->hn, sizeof(float) * (size_t)MB * c.dim);
    A((void**)&lm->qkv, sizeof(float) * (size_t)MB * lm->qkv_n);
    A((void**)&lm->qbuf, sizeof(float) * (size_t)MB * lm->ctx);
    A((void**)&lm->part, sizeof(float) * (size_t)MB * c.n_heads * lm->max_splits * (hd + 4));
    A((void**)&lm->gu, sizeof(float) * (size_t)MB * 2 * I);
    A((void**)&lm->act_f32, sizeof(float) * (size_t)MB * I);
    A((void**)&lm->logits, sizeof(float) * (size_t)MB * c.vocab);
    const size_t ab = act_block_bytes(lm->vdt), bs = block_size(lm->vdt);
    A((void**)&lm->act_a, ab * MB * (c.dim / bs));
    A((void**)&lm->act_o, ab * MB * (lm->ctx / bs));
    A((void**)&lm->act_d, ab * MB * (I / bs));
    if (lm->vdt == kQ8K) {
        A((void**)&lm->rec_a, sizeof(MmaRec) * (size_t)(c.dim / 256));
        A((void**)&lm->rec_o, sizeof(MmaRec) * (size_t)(lm->ctx / 256));
        A((void**)&lm->rec_d, sizeof(MmaRec) * (size_t)(I / 256));
        if (MB >= 5) {
            A((void**)&lm->rec_ws.part, GemvRecWs::part_bytes());
            A((void**)&lm->rec_ws.count, GemvRecWs::count_bytes());
        }
    }
    A((void**)&lm->d_ids, sizeof(int) * MB * lm->ids_per);
    A((void**)&lm->d_next, sizeof(int) * MB);
    A((void**)&lm->am_val, sizeof(float) * MB * kArgmaxSlices);
    A((void**)&lm->am_idx, sizeof(int) * MB * kArgmaxSlices);
    A((void**)&lm->am_count, sizeof(unsigned) * MB * kCounterStride);
    A((void**)&lm->attn_count, sizeof(unsigned) * MB * c.n_kv_heads * kCounterStride);
    A((void**)&lm->wo_ready, sizeof(unsigned) * c.n_layers * kReadyCopies * kCounterStride);
    if (const char* e_spec = getenv("SXQ_ATTN_SPEC"); !(e_spec && e_spec[0] == '0'))
        A((void**)&lm->rope_row, sizeof(float) * 256);
    if (e != hipSuccess) {
        destroy_lm(lm);
        return hip_fail(e, "lm_create: allocation");
    }
    // RoPE tables, computed on the host with the reference's f32 formula:
    // inv_freq[i] = 1 / base^(2i/hd), angle = t * inv_freq[i] (s2/nn.rs:125-135, cv2/attention.rs:110-118).
    {
        const int half = hd / 2;
        std::vector<float> cs((size_t)c.max_seq * half), sn((size_t)c.max_seq * half);
        for (int i = 0; i < half; ++i) {
            const float inv = 1.0f / powf(c.rope_theta, 2.0f * (float)i / (float)hd);
            for (int t = 0; t < c.max_seq; ++t) {
                const float a = (float)t * inv;
                cs[(size_t)t * half + i] = cosf(a);
                sn[(size_t)t * half + i] = sinf(a);
            }
        }
        e = hipMemcpy(lm->rope_cos, cs.data(), cs.size() * sizeof(float), hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(lm->rope_sin, sn.data(), sn.size() * sizeof(float), hipMemcpyHostToDevice);
    }
    // defaults: norm weights 1, biases 0, lengths 0, ids 0
    for (auto& L : lm->layers) {
        if (e == hipSuccess) e = launch_fill_value(L.attn_norm, c.dim, 1.0f, nullptr);
        if (e == hipSuccess) e = launch_fill_value(L.ffn_norm, c.dim, 1.0f, nullptr);
        if (e == hipSuccess) e = launch_fill_value(L.q_norm, hd, 1.0f, nullptr);
        if (e == hipSuccess) e = launch_fill_value(L.k_norm, hd, 1.0f, nullptr);
        if (e == hipSuccess) e = launch_fill_value(L.bqkv, lm->qkv_n, 0.0f, nullptr);
        if (e == hipSuccess && L.bo) e = launch_fill_value(L.bo, c.dim, 0.0f, nullptr);
    }
    if (e == hipSuccess) e = launch_fill_value(lm->final_norm, c.dim, 1.0f, nullptr);
    if (e == hipSuccess) e = launch_fill_value(lm->head_bias, c.vocab, 0.0f, nullptr);
    if (e == hipSuccess) e = hipMemset(lm->d_len, 0, sizeof(int) * MB);
    if (e == hipSuccess) e = hipMemset(lm->d_ids, 0, sizeof(int) * MB * lm->ids_per);
    if (e == hipSuccess) e = hipMemset(lm->am_count, 0, sizeof(unsigned) * MB * kCounterStride);
    if (e == hipSuccess) e = hipMemset(lm->attn_count, 0, sizeof(unsigned) * MB * c.n_kv_heads * kCounterStride);
    if (e == hipSuccess) e = hipMemset(lm->wo_ready, 0, sizeof(unsigned) * c.n_layers * kReadyCopies * kCounterStride);
    if (e == hipSuccess) e = hipMemset(lm->act_f32, 0, sizeof(float) * (size_t)MB * I);
    if (e == hipSuccess && lm->rec_a) e = hipMemset(lm->rec_a, 0, sizeof(MmaRec) * (size_t)(c.dim / 256));
    if (e == hipSuccess && lm->rec_o) e = hipMemset(lm->rec_o, 0, sizeof(MmaRec) * (size_t)(lm->ctx / 256));
    if (e == hipSuccess && lm->rec_d) e = hipMemset(lm->rec_d, 0, sizeof(MmaRec) * (size_t)(I / 256));
    if (e == hipSuccess && lm->rec_ws.count) e = hipMemset(lm->rec_ws.count, 0, GemvRecWs::count_bytes());
    lm->attn_fused = getenv("SXQ_ATTN_UNFUSED") == nullptr && attn_decode_fits(lm->vdt, c.n_heads, c.n_kv_heads, hd, lm->max_splits);
    lm->swiglu = getenv("SXQ_SWIGLU_UNFUSED") == nullptr && swiglu_pair_fits(lm->layers[0].w13.w, lm->layers[0].w2.w);
    if (e == hipSuccess && lm->attn_fused &&
        attn_decode_prepare(lm->vdt, c.n_heads, c.n_kv_heads, hd, lm->max_splits) != hipSuccess) {
        (void)hipGetLastError();  // clear it: the three-kernel path needs no opt-in
        lm->attn_fused = false;
    }
    // (the fused launch's O projection has no bias epilogue: o_bias models run it as its own GEMV)
    lm->wo_fused = lm->attn_fused && c.n_layers >= 2 && !c.o_bias && getenv("SXQ_ATTN_WO_UNFUSED") == nullptr &&
                   attn_wo_decode_fits(lm->vdt, c.n_heads, c.n_kv_heads, hd, lm->max_splits, lm->layers[0].wo.w, c.dim);
    if (e == hipSuccess && lm->wo_fused &&
        attn_wo_decode_prepare(lm->vdt, c.n_heads, c.n_kv_heads, hd, lm->max_splits, lm->layers[0].wo.w) != hipSuccess) {
        (void)hipGetLastError();
        lm->wo_fused = false;
    }
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&lm->cap, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        destroy_lm(lm);
        return hip_fail(e, "lm_create: initialisation");
    }
    lm->h_len.assign(MB, 0);
    *out = lm;
    return SXQ_OK;
}

sxq_status sxq_lm_destroy(sxq_lm* lm) {
    if (!lm) return SXQ_OK;
    DeviceGuard g(lm->device);
    (void)hipDeviceSynchronize();
    destroy_lm(lm);
    return SXQ_OK;
}

sxq_status sxq_lm_set_linear(sxq_lm* lm, int layer, int which, const sxq_qmm* q) {
    if (!lm || !q) return fail(SXQ_ERR_INVALID, "lm_set_linear: null handle");
    const sxq_lm_config& c = lm->c;
    if (q->w.dtype != c.weight_dtype)
        return fail(SXQ_ERR_DTYPE, "lm_set_linear: weight dtype %d, the model uses %d", q->w.dtype, c.weight_dtype);
    if (which != SXQ_LM_HEAD && (layer < 0 || layer >= c.n_layers))
        return fail(SXQ_ERR_INVALID, "lm_set_linear: layer %d out of range", layer);
    const int hd = c.head_dim;
    DevWeight* dst = nullptr;
    int64_t r0 = 0, rows = 0, k = 0;
    switch (which) {
    case SXQ_LM_WQKV: dst = &lm->layers[layer].wqkv; rows = lm->qkv_n; k = c.dim; break;
    case SXQ_LM_WQ: dst = &lm->layers[layer].wqkv; rows = lm->ctx; k = c.dim; break;
    case SXQ_LM_WK: dst = &lm->layers[layer].wqkv; r0 = lm->ctx; rows = (int64_t)c.n_kv_heads * hd; k = c.dim; break;
    case SXQ_LM_WV:
        dst = &lm->layers[layer].wqkv;
        r0 = lm->ctx + (int64_t)c.n_kv_heads * hd;
        rows = (int64_t)c.n_kv_heads * hd;
        k = c.dim;
        break;
    case SXQ_LM_WO: dst = &lm->layers[layer].wo; rows = c.dim; k = lm->ctx; break;
    case SXQ_LM_W1: dst = &lm->layers[layer].w13; rows = c.intermediate; k = c.dim; break;
    case SXQ_LM_W3: dst = &lm->layers[layer].w13; r0 = c.intermediate; rows = c.intermediate; k = c.dim; break;
    case SXQ_LM_W2: dst = &lm->layers[layer].w2; rows = c.dim; k = c.intermediate; break;
    case SXQ_LM_HEAD: dst = &lm->head; rows = c.vocab; k = c.dim; break;
    default: return fail(SXQ_ERR_INVALID, "lm_set_linear: unknown slot %d", which);
    }
    if (q->w.n != rows || q->w.k != k)
        return fail(SXQ_ERR_SHAPE, "lm_set_linear: slot %d expects [%lld, %lld], got [%lld, %lld]", which,
                    (long long)rows, (long long)k, (long long)q->w.n, (long long)q->w.k);
    std::lock_guard<std::mutex> lock(lm->mu);
    DeviceGuard g(lm->device);
    HIP_TRY(g.err, "hipSetDevice");
    HIP_TRY(copy_rows(*dst, q->w, r0, nullptr), "lm_set_linear: copy");
    HIP_TRY(hipDeviceSynchronize(), "lm_set_linear");
    return SXQ_OK;
}

sxq_status sxq_lm_set_vector(sxq_lm* lm, int layer, int which, const float* data, int64_t n, int src_is_device) {
    if (!lm || !data) return fail(SXQ_ERR_INVALID, "lm_set_vector: null pointer");
    const sxq_lm_config& c = lm->c;
    const bool per_layer = which <= SXQ_LM_BV || which == SXQ_LM_BO;
    if (per_layer && (layer < 0 || layer >= c.n_layers)) return fail(SXQ_ERR_INVALID, "lm_set_vector: layer out of range");
    const int hd = c.head_dim;
    float* dst = nullptr;
    int64_t want = 0;
    switch (which) {
    case SXQ_LM_ATTN_NORM: dst = lm->layers[layer].attn_norm; want = c.dim; break;
    case SXQ_LM_FFN_NORM: dst = lm->layers[layer].ffn_norm; want = c.dim; break;
    case SXQ_LM_Q_NORM: dst = lm->layers[layer].q_norm; want = hd; break;
    case SXQ_LM_K_NORM: dst = lm->layers[layer].k_norm; want = hd; break;
    case SXQ_LM_BQ: dst = lm->layers[layer].bqkv; want = lm->ctx; break;
    case SXQ_LM_BK: dst = lm->layers[layer].bqkv + lm->ctx; want = (int64_t)c.n_kv_heads * hd; break;
    case SXQ_LM_BV: dst = lm->layers[layer].bqkv + lm->ctx + (int64_t)c.n_kv_heads * hd; want = (int64_t)c.n_kv_heads * hd; break;
    case SXQ_LM_BO:
        if (!lm->layers[layer].bo) return fail(SXQ_ERR_INVALID, "lm_set_vector: this model has no wo bias (o_bias 0)");
        dst = lm->layers[layer].bo;
        want = c.dim;
        break;
    case SXQ_LM_FINAL_NORM: dst = lm->final_norm; want = c.dim; break;
    case SXQ_LM_HEAD_BIAS: dst = lm->head_bias; want = c.vocab; break;
    case SXQ_LM_EMBED:
        // a tied model gets its dense table on the first upload (embeddings.weight, which the
        // head quantizes: the embedding then gathers it, as SlowAr::embed does)
        dst = lm->embed;
        want = (int64_t)embed_rows(c) * c.dim;
        break;
    case SXQ_LM_CODEBOOK_EMBED:
        if (!lm->cb_embed) return fail(SXQ_ERR_INVALID, "lm_set_vector: this model has no codebooks");
        dst = lm->cb_embed;
        want = (int64_t)c.n_codebooks * c.codebook_size * c.dim;
        break;
    default: return fail(SXQ_ERR_INVALID, "lm_set_vector: unknown slot %d", which);
    }
    if (n != want) return fail(SXQ_ERR_SHAPE, "lm_set_vector: slot %d expects %lld values, got %lld", which, (long long)want, (long long)n);
    std::lock_guard<std::mutex> lock(lm->mu);
    DeviceGuard g(lm->device);
    HIP_TRY(g.err, "hipSetDevice");
    if (which == SXQ_LM_EMBED && !lm->embed) {
        HIP_TRY(hipDeviceSynchronize(), "lm_set_vector: drain");
        HIP_TRY(dalloc(lm, (void**)&lm->embed, sizeof(float) * (size_t)want), "lm_set_vector: dense input table");
        drop_graphs(lm);  // captured with the head-row embedding
        dst = lm->embed;
    }
    HIP_TRY(hipMemcpy(dst, data, sizeof(float) * n, src_is_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice),
            "lm_set_vector: copy");
    return SXQ_OK;
}

sxq_status sxq_lm_set_embed_quantized(sxq_lm* lm, int scheme, const uint8_t* q, const float* scale) {
    if (!lm) return fail(SXQ_ERR_INVALID, "lm_set_embed_quantized: null handle");
    const sxq_lm_config& c = lm->c;
    if (c.tied_embedding || !lm->embed)
        return fail(SXQ_ERR_INVALID, "lm_set_embed_quantized: this model has a tied embedding");
    if (c.n_codebooks > 0)
        return fail(SXQ_ERR_INVALID, "lm_set_embed_quantized: the codebook (MCF) embedding gathers a dense table");
    if (scheme != SXQ_EMBED_INT8 && scheme != SXQ_EMBED_INT4)
        return fail(SXQ_ERR_INVALID, "lm_set_embed_quantized: unknown scheme %d", scheme);
    if (embed_effective_scheme(scheme, c.dim) != scheme)
        return fail(SXQ_ERR_INVALID, "lm_set_embed_quantized: int4 needs an even row width (dim %d)", c.dim);
    if (!q || !scale) return fail(SXQ_ERR_INVALID, "lm_set_embed_quantized: null pointer");
    std::lock_guard<std::mutex> lock(lm->mu);
    DeviceGuard g(lm->device);
    HIP_TRY(g.err, "hipSetDevice");
    const int64_t rows = embed_rows(c);
    const size_t qb = embed_code_bytes(scheme, rows, c.dim);
    if (!lm->embed_q) {  // sized for int8, the larger of the two
        HIP_TRY(dalloc(lm, (void**)&lm->embed_q, embed_code_bytes(SXQ_EMBED_INT8, rows, c.dim)), "lm_set_embed_quantized");
        HIP_TRY(dalloc(lm, (void**)&lm->embed_scale, sizeof(float) * rows), "lm_set_embed_quantized");
    }
    HIP_TRY(hipDeviceSynchronize(), "lm_set_embed_quantized: drain");
    HIP_TRY(hipMemcpy(lm->embed_q, q, qb, hipMemcpyDefault), "lm_set_embed_quantized: codes");
    HIP_TRY(hipMemcpy(lm->embed_scale, scale, sizeof(float) * rows, hipMemcpyDefault), "lm_set_embed_quantized: scales");
    lm->embed_scheme = scheme;
    drop_graphs(lm);  // captured with the dense gather
    return SXQ_OK;
}

sxq_status sxq_lm_init_random(sxq_lm* lm, uint64_t seed, float stdv) {
    if (!lm) return fail(SXQ_ERR_INVALID, "lm_init_random: null handle");
    std::lock_guard<std::mutex> lock(lm->mu);
    const sxq_lm_config& c = lm->c;
    DeviceGuard g(lm->device);
    HIP_TRY(g.err, "hipSetDevice");
    const int64_t tmp_elems = (int64_t)64 << 20;  // 256 MB of f32 staging
    float* tmp = nullptr;
    uint8_t* blk = nullptr;
    HIP_TRY(hipMalloc(&tmp, sizeof(float) * tmp_elems), "lm_init_random: staging");
    hipError_t e = hipMalloc(&blk, (size_t)tmp_elems * 2);  // >= bytes of any block encoding of tmp_elems
    uint64_t sd = seed * 0x9E3779B97F4A7C15ull + 1;
    auto W = [&](DevWeight& d, int64_t r0, int64_t n) {
        if (e == hipSuccess) e = random_rows(d, r0, n, sd++, stdv, tmp, blk, tmp_elems, nullptr);
    };
    auto V = [&](float* p, int64_t n, float mean, float sdv) {
        if (e == hipSuccess) e = sdv > 0 ? launch_fill_normal(p, n, sd++, mean, sdv, nullptr) : launch_fill_value(p, n, mean, nullptr);
    };
    for (auto& L : lm->layers) {
        W(L.wqkv, 0, lm->qkv_n);
        W(L.wo, 0, c.dim);
        W(L.w13, 0, c.intermediate);
        W(L.w13, c.intermediate, c.intermediate);
        W(L.w2, 0, c.dim);
        V(L.attn_norm, c.dim, 1.0f, 0.0f);
        V(L.ffn_norm, c.dim, 1.0f, 0.0f);
        V(L.q_norm, c.head_dim, 1.0f, 0.0f);
        V(L.k_norm, c.head_dim, 1.0f, 0.0f);
        V(L.bqkv, lm->qkv_n, 0.0f, c.qkv_bias ? stdv : 0.0f);
        if (L.bo) V(L.bo, c.dim, 0.0f, stdv);
    }
    if (c.tied_embedding) {
        // the tied head quantizes the dense table, which the embedding gathers: keep the
        // f32 rows the head is made from as that table
        if (!lm->embed && e == hipSuccess) {
            e = hipDeviceSynchronize();
            if (e == hipSuccess) e = dalloc(lm, (void**)&lm->embed, sizeof(float) * (size_t)c.vocab * c.dim);
            drop_graphs(lm);
        }
        if (e == hipSuccess) e = random_rows(lm->head, 0, c.vocab, sd++, stdv, tmp, blk, tmp_elems, nullptr, lm->embed);
    } else {
        W(lm->head, 0, c.vocab);
    }
    V(lm->final_norm, c.dim, 1.0f, 0.0f);
    V(lm->head_bias, c.vocab, 0.0f, c.head_bias ? stdv : 0.0f);
    if (lm->embed && !c.tied_embedding) V(lm->embed, (int64_t)embed_rows(c) * c.dim, 0.0f, stdv);
    if (lm->cb_embed) V(lm->cb_embed, (int64_t)c.n_codebooks * c.codebook_size * c.dim, 0.0f, stdv);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    (void)hipFree(tmp);
    if (blk) (void)hipFree(blk);
    if (e != hipSuccess) return hip_fail(e, "lm_init_random");
    return SXQ_OK;
}

sxq_status sxq_lm_set_lengths(sxq_lm* lm, const int32_t* lengths, int n) {
    if (!lm || !lengths) return fail(SXQ_ERR_INVALID, "lm_set_lengths: null pointer");
    if (n < 1 || n > lm->c.max_batch) return fail(SXQ_ERR_INVALID, "lm_set_lengths: %d streams (max %d)", n, lm->c.max_batch);
    for (int s = 0; s < n; ++s)
        if (lengths[s] < 0 || lengths[s] > lm->c.max_seq)
            return fail(SXQ_ERR_INVALID, "lm_set_lengths: length %d outside [0, %d]", lengths[s], lm->c.max_seq);
    std::lock_guard<std::mutex> lock(lm->mu);
    DeviceGuard g(lm->device);
    HIP_TRY(g.err, "hipSetDevice");
    HIP_TRY(hipDeviceSynchronize(), "lm_set_lengths");
    for (int s = 0; s < n; ++s) lm->h_len[s] = lengths[s];
    HIP_TRY(hipMemcpy(lm->d_len, lm->h_len.data(), sizeof(int) * lm->c.max_batch, hipMemcpyHostToDevice), "lm_set_lengths");
    return SXQ_OK;
}

sxq_status sxq_lm_reset(sxq_lm* lm, int n, void* stream) {
    if (!lm) return fail(SXQ_ERR_INVALID, "lm_reset: null handle");
    if (n < 1 || n > lm->c.max_batch) return fail(SXQ_ERR_INVALID, "lm_reset: %d streams (max %d)", n, lm->c.max_batch);
    std::lock_guard<std::mutex> lock(lm->mu);
    DeviceGuard g(lm->device);
    HIP_TRY(g.err, "hipSetDevice");
    HIP_TRY(hipMemsetAsync(lm->d_len, 0, sizeof(int) * n, (hipStream_t)stream), "lm_reset");
    for (int s = 0; s < n; ++s) lm->h_len[s] = 0;
    return SXQ_OK;
}

sxq_status sxq_lm_get_lengths(const sxq_lm* lm, int32_t* lengths, int n) {
    if (!lm || !lengths) return fail(SXQ_ERR_INVALID, "lm_get_lengths: null pointer");
    if (n < 1 || n > lm->c.max_batch) return fail(SXQ_ERR_INVALID, "lm_get_lengths: bad stream count");
    for (int s = 0; s < n; ++s) lengths[s] = lm->h_len[s];
    return SXQ_OK;
}

sxq_status sxq_lm_kv_fill_random(sxq_lm* lm, const int32_t* lengths, int n, uint64_t seed) {
    if (!lm) return fail(SXQ_ERR_INVALID, "lm_kv_fill_random: null handle");
    {
        std::lock_guard<std::mutex> lock(lm->mu);
        DeviceGuard g(lm->device);
        HIP_TRY(g.err, "hipSetDevice");
        const int64_t total = lm->kv_layer_stride * lm->c.n_layers;
        HIP_TRY(launch_fill_normal(lm->kc, total, seed * 2 + 11, 0.0f, 1.0f, nullptr), "lm_kv_fill_random");
        HIP_TRY(launch_fill_normal(lm->vc, total, seed * 2 + 12, 0.0f, 1.0f, nullptr), "lm_kv_fill_random");
        HIP_TRY(hipDeviceSynchronize(), "lm_kv_fill_random");
    }
    return lengths ? sxq_lm_set_lengths(lm, lengths, n) : SXQ_OK;
}

sxq_status sxq_lm_step(sxq_lm* lm, int n, const int32_t* ids, const float* embeds, float* logits, float* hidden,
                       int32_t* next_ids, unsigned flags, void* stream) {
    if (!lm) return fail(SXQ_ERR_INVALID, "lm_step: null handle");
    if (n < 1 || n > lm->c.max_batch) return fail(SXQ_ERR_INVALID, "lm_step: %d streams (max %d)", n, lm->c.max_batch);
    if (flags & ~SXQ_LM_GRAPH) return fail(SXQ_ERR_INVALID, "lm_step: unknown flags 0x%x", flags);
    std::lock_guard<std::mutex> lock(lm->mu);
    for (int s = 0; s < n; ++s)
        if (lm->h_len[s] >= lm->c.max_seq)
            return fail(SXQ_ERR_INVALID, "lm_step: stream %d KV cache is full (%d positions)", s, lm->c.max_seq);
    DeviceGuard g(lm->device);
    HIP_TRY(g.err, "hipSetDevice");
    hipStream_t st = (hipStream_t)stream;
    const bool emb = embeds != nullptr;
    if (ids) HIP_TRY(hipMemcpyAsync(lm->d_ids, ids, sizeof(int) * n * lm->ids_per, hipMemcpyDeviceToDevice, st), "lm_step: ids");
    if (emb) HIP_TRY(hipMemcpyAsync(lm->h, embeds, sizeof(float) * n * lm->c.dim, hipMemcpyDeviceToDevice, st), "lm_step: embeds");
    lm->grid_splits = step_grid_splits(lm, n);
    if (flags & SXQ_LM_GRAPH) {
        const GraphKey key{n, emb, lm->trace, lm->grid_splits};
        auto it = lm->graphs.find(key);
        if (it == lm->graphs.end()) {
            // Capture on the library's own stream (the legacy default stream cannot capture).
            hipGraph_t graph = nullptr;
            hipGraphExec_t exec = nullptr;
            HIP_TRY(hipStreamSynchronize(st), "lm_step: sync before capture");
            HIP_TRY(hipStreamBeginCapture(lm->cap, hipStreamCaptureModeThreadLocal), "lm_step: begin capture");
            hipError_t e = enqueue_step(lm, n, emb, lm->cap);
            hipError_t e2 = hipStreamEndCapture(lm->cap, &graph);
            if (e == hipSuccess) e = e2;
            if (e == hipSuccess) e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
            if (graph) (void)hipGraphDestroy(graph);
            if (e != hipSuccess) return hip_fail(e, "lm_step: graph capture");
            it = lm->graphs.emplace(key, exec).first;
        }
        HIP_TRY(hipGraphLaunch(it->second, st), "lm_step: graph launch");
    } else {
        HIP_TRY(enqueue_step(lm, n, emb, st), "lm_step");
    }
    for (int s = 0; s < n; ++s) lm->h_len[s] += 1;
    if (logits)
        HIP_TRY(hipMemcpyAsync(logits, lm->logits, sizeof(float) * n * lm->c.vocab, hipMemcpyDeviceToDevice, st), "lm_step: logits");
    if (hidden)
        HIP_TRY(hipMemcpyAsync(hidden, lm->hn, sizeof(float) * n * lm->c.dim, hipMemcpyDeviceToDevice, st), "lm_step: hidden");
    if (next_ids) HIP_TRY(hipMemcpyAsync(next_ids, lm->d_next, sizeof(int) * n, hipMemcpyDeviceToDevice, st), "lm_step: next ids");
    return SXQ_OK;
}

sxq_status sxq_fish_fast_expand(sxq_lm* lm, int n, const float* hidden, const int32_t* semantic, int semantic_stride,
                                const int32_t* active, const sxq_fish_sampling* params, uint64_t* rng, int n_codes,
                                int32_t* codes, int codes_stride, unsigned flags, void* stream) {
    if (!lm) return fail(SXQ_ERR_INVALID, "fast_expand: null handle");
    const sxq_lm_config& c = lm->c;
    if (n < 1 || n > c.max_batch) return fail(SXQ_ERR_INVALID, "fast_expand: %d streams (max %d)", n, c.max_batch);
    if (!hidden || !semantic || !params || !rng || !codes) return fail(SXQ_ERR_INVALID, "fast_expand: null pointer");
    if (flags & ~SXQ_LM_GRAPH) return fail(SXQ_ERR_INVALID, "fast_expand: unknown flags 0x%x", flags);
    if (c.n_codebooks != 0 || c.tied_embedding || (c.embed_rows > 0 && c.embed_rows < c.vocab))
        return fail(SXQ_ERR_INVALID,
                    "fast_expand: the engine must embed single code ids from a dense table of >= vocab rows "
                    "(n_codebooks 0, tied_embedding 0)");
    if (n_codes < 1 || n_codes > c.max_seq)
        return fail(SXQ_ERR_INVALID, "fast_expand: %d codes per frame (the local cache holds %d)", n_codes, c.max_seq);
    if (semantic_stride < 1 || codes_stride < 1) return fail(SXQ_ERR_INVALID, "fast_expand: strides must be >= 1");
    if (!fish_sampling_fits(*params)) return fail(SXQ_ERR_INVALID, "fast_expand: top_k %d is negative", params->top_k);
    std::lock_guard<std::mutex> lock(lm->mu);
    if (lm->trace) return fail(SXQ_ERR_INVALID, "fast_expand: clear the step trace first");
    DeviceGuard g(lm->device);
    HIP_TRY(g.err, "hipSetDevice");
    hipStream_t st = (hipStream_t)stream;
    const ExpandArgs a{n, hidden, semantic, semantic_stride, active, *params, rng, n_codes, codes, codes_stride};
    if (flags & SXQ_LM_GRAPH) {
        const std::string key = expand_key(a);
        auto it = lm->expand_graphs.find(key);
        if (it == lm->expand_graphs.end()) {
            if (lm->expand_graphs.size() >= kMaxExpandGraphs) {  // callers cycling buffers: start over
                HIP_TRY(hipStreamSynchronize(st), "fast_expand: sync before dropping graphs");
                for (auto& kv : lm->expand_graphs) (void)hipGraphExecDestroy(kv.second);
                lm->expand_graphs.clear();
            }
            hipGraph_t graph = nullptr;
            hipGraphExec_t exec = nullptr;
            HIP_TRY(hipStreamSynchronize(st), "fast_expand: sync before capture");
            HIP_TRY(hipStreamBeginCapture(lm->cap, hipStreamCaptureModeThreadLocal), "fast_expand: begin capture");
            hipError_t e = enqueue_expand(lm, a, lm->cap);
            hipError_t e2 = hipStreamEndCapture(lm->cap, &graph);
            if (e == hipSuccess) e = e2;
            if (e == hipSuccess) e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
            if (graph) (void)hipGraphDestroy(graph);
            if (e != hipSuccess) return hip_fail(e, "fast_expand: graph capture");
            it = lm->expand_graphs.emplace(key, exec).first;
        }
        HIP_TRY(hipGraphLaunch(it->second, st), "fast_expand: graph launch");
    } else {
        HIP_TRY(enqueue_expand(lm, a, st), "fast_expand");
    }
    for (int s = 0; s < n; ++s) lm->h_len[s] = n_codes;
    return SXQ_OK;
}

sxq_status sxq_lm_prefill_trace_floats(const sxq_lm* lm, int64_t tokens, size_t* floats) {
    if (!lm || !floats) return fail(SXQ_ERR_INVALID, "lm_prefill_trace_floats: null pointer");
    if (tokens < 1 || tokens > 65535) return fail(SXQ_ERR_INVALID, "lm_prefill_trace_floats: bad token count");
    *floats = pf_trace_floats(lm, (int)tokens);
    return SXQ_OK;
}

sxq_status sxq_lm_prefill(sxq_lm* lm, int n, const int32_t* counts, const int32_t* ids, const float* embeds,
                          float* logits, float* hidden, int32_t* next_ids, unsigned flags, float* trace,
                          size_t trace_capacity, void* stream) {
    if (!lm) return fail(SXQ_ERR_INVALID, "lm_prefill: null handle");
    if (n < 1 || n > lm->c.max_batch) return fail(SXQ_ERR_INVALID, "lm_prefill: %d streams (max %d)", n, lm->c.max_batch);
    if (!counts) return fail(SXQ_ERR_INVALID, "lm_prefill: null token counts");
    if (flags & ~(SXQ_LM_EXACT | SXQ_LM_ALL_LOGITS)) return fail(SXQ_ERR_INVALID, "lm_prefill: unknown flags 0x%x", flags);
    if (!ids == !embeds) return fail(SXQ_ERR_INVALID, "lm_prefill: give exactly one of ids and embeds");
    const sxq_lm_config& c = lm->c;
    if (!prefill_attn_supported(c.n_heads, c.n_kv_heads, c.head_dim))
        return fail(SXQ_ERR_SHAPE, "lm_prefill: head_dim %d (64 or 128) or %d query heads per KV head unsupported",
                    c.head_dim, c.n_heads / c.n_kv_heads);
    std::lock_guard<std::mutex> lock(lm->mu);
    PrefillMeta pm{};
    pm.n = n;
    pm.tile_tokens = prefill_tile_tokens(c.n_heads, c.n_kv_heads);
    int64_t T = 0;
    for (int s = 0; s < n; ++s) {
        if (counts[s] < 0) return fail(SXQ_ERR_INVALID, "lm_prefill: negative token count for stream %d", s);
        if ((int64_t)lm->h_len[s] + counts[s] > c.max_seq)
            return fail(SXQ_ERR_INVALID, "lm_prefill: stream %d: %d cached + %d new positions exceed %d", s,
                        lm->h_len[s], counts[s], c.max_seq);
        pm.counts[s] = counts[s];
        pm.lens[s] = lm->h_len[s];
        T += counts[s];
    }
    if (T == 0) return SXQ_OK;
    if (T > 65535) return fail(SXQ_ERR_INVALID, "lm_prefill: %lld tokens exceed 65535", (long long)T);
    for (int s = 0; s < n; ++s)
        if (counts[s] == 0) return fail(SXQ_ERR_INVALID, "lm_prefill: stream %d has no tokens", s);
    if (trace && trace_capacity < pf_trace_floats(lm, (int)T))
        return fail(SXQ_ERR_SHAPE, "lm_prefill: trace of %zu floats, %zu needed", trace_capacity,
                    pf_trace_floats(lm, (int)T));
    DeviceGuard g(lm->device);
    HIP_TRY(g.err, "hipSetDevice");
    hipStream_t st = (hipStream_t)stream;
    const PfLayout P = pf_layout(lm, (int)T, n);
    if (lm->pf_size < P.total) {
        HIP_TRY(hipDeviceSynchronize(), "lm_prefill: sync before regrowing the workspace");
        if (lm->pf) (void)hipFree(lm->pf);
        lm->pf = nullptr;
        lm->pf_size = 0;
        HIP_TRY(hipMalloc(&lm->pf, P.total), "lm_prefill: workspace");
        lm->pf_size = P.total;
    }
    const bool all = (flags & SXQ_LM_ALL_LOGITS) != 0;
    if (all && !logits) return fail(SXQ_ERR_INVALID, "lm_prefill: SXQ_LM_ALL_LOGITS needs a logits buffer");
    HIP_TRY(enqueue_prefill(lm, pm, (int)T, ids, embeds, all ? logits : nullptr, all ? hidden : nullptr,
                            (flags & SXQ_LM_EXACT) != 0, trace, st),
            "lm_prefill");
    for (int s = 0; s < n; ++s) lm->h_len[s] += counts[s];
    if (logits && !all)
        HIP_TRY(hipMemcpyAsync(logits, lm->logits, sizeof(float) * n * c.vocab, hipMemcpyDeviceToDevice, st),
                "lm_prefill: logits");
    if (hidden && !all)
        HIP_TRY(hipMemcpyAsync(hidden, lm->hn, sizeof(float) * n * c.dim, hipMemcpyDeviceToDevice, st),
                "lm_prefill: hidden");
    if (next_ids) HIP_TRY(hipMemcpyAsync(next_ids, lm->d_next, sizeof(int) * n, hipMemcpyDeviceToDevice, st), "lm_prefill: ids");
    return SXQ_OK;
}

sxq_status sxq_lm_gemv_pass(sxq_lm* lm, int n, int with_head, void* stream) {
    if (!lm) return fail(SXQ_ERR_INVALID, "lm_gemv_pass: null handle");
    if (n < 1 || n > lm->c.max_batch) return fail(SXQ_ERR_INVALID, "lm_gemv_pass: %d streams", n);
    std::lock_guard<std::mutex> lock(lm->mu);
    DeviceGuard g(lm->device);
    HIP_TRY(g.err, "hipSetDevice");
    hipStream_t s = (hipStream_t)stream;
    const sxq_lm_config& c = lm->c;
    const int I = c.intermediate;
    // the step's GEMVs on whatever the buffers hold (records where the step reads them)
    const bool rec_ok = n >= 5 && n <= 16 && lm->rec_a != nullptr;
    const MmaRec* rec_a = rec_ok ? lm->rec_a : nullptr;
    const MmaRec* rec_o = rec_ok && lm->attn_fused ? lm->rec_o : nullptr;
    const MmaRec* rec_d = rec_ok ? lm->rec_d : nullptr;
    for (int l = 0; l < c.n_layers; ++l) {
        LmLayer& L = lm->layers[l];
        const GemvRecWs* ws = &lm->rec_ws;
        HIP_TRY(launch_gemv_rec(L.wqkv.w, lm->act_a, rec_a, n, lm->qkv, lm->qkv_n, L.bqkv, nullptr, 0, s, ws), "lm_gemv_pass");
        HIP_TRY(launch_gemv_rec(L.wo.w, lm->act_o, rec_o, n, lm->gu, c.dim, L.bo, nullptr, 0, s, ws), "lm_gemv_pass");
        HIP_TRY(launch_gemv_rec(L.w13.w, lm->act_a, rec_a, n, lm->gu, 2 * I, nullptr, nullptr, 0, s, ws), "lm_gemv_pass");
        HIP_TRY(launch_gemv_rec(L.w2.w, lm->act_d, rec_d, n, lm->gu, c.dim, nullptr, nullptr, 0, s, ws), "lm_gemv_pass");
    }
    if (with_head)
        HIP_TRY(launch_gemv_rec(lm->head.w, lm->act_a, rec_a, n, lm->logits, c.vocab, nullptr, nullptr, 0, s),
                "lm_gemv_pass");
    return SXQ_OK;
}

sxq_status sxq_lm_read_kv(const sxq_lm* lm, int layer, int s, int g, int pos0, int count, float* k_out, float* v_out,
                          void* stream) {
    if (!lm) return fail(SXQ_ERR_INVALID, "lm_read_kv: null handle");
    const sxq_lm_config& c = lm->c;
    if (layer < 0 || layer >= c.n_layers || s < 0 || s >= c.max_batch || g < 0 || g >= c.n_kv_heads || pos0 < 0 ||
        count < 0 || pos0 + count > c.max_seq)
        return fail(SXQ_ERR_INVALID, "lm_read_kv: out of range");
    DeviceGuard gd(lm->device);
    HIP_TRY(gd.err, "hipSetDevice");
    const int64_t off = (int64_t)layer * lm->kv_layer_stride + (int64_t)s * lm->kv_stream_stride +
                        ((int64_t)g * c.max_seq + pos0) * c.head_dim;
    const size_t bytes = sizeof(float) * (size_t)count * c.head_dim;
    hipStream_t st = (hipStream_t)stream;
    if (k_out) HIP_TRY(hipMemcpyAsync(k_out, lm->kc + off, bytes, hipMemcpyDeviceToDevice, st), "lm_read_kv");
    if (v_out) HIP_TRY(hipMemcpyAsync(v_out, lm->vc + off, bytes, hipMemcpyDeviceToDevice, st), "lm_read_kv");
    return SXQ_OK;
}

sxq_status sxq_lm_trace_floats(const sxq_lm* lm, int n, size_t* floats) {
    if (!lm || !floats) return fail(SXQ_ERR_INVALID, "lm_trace_floats: null pointer");
    if (n < 1 || n > lm->c.max_batch) return fail(SXQ_ERR_INVALID, "lm_trace_floats: bad stream count");
    *floats = trace_floats(lm, n);
    return SXQ_OK;
}

sxq_status sxq_lm_set_trace(sxq_lm* lm, float* trace, size_t capacity_floats) {
    if (!lm) return fail(SXQ_ERR_INVALID, "lm_set_trace: null handle");
    if (trace && capacity_floats < trace_floats(lm, lm->c.max_batch))
        return fail(SXQ_ERR_SHAPE, "lm_set_trace: %zu floats given, %zu needed", capacity_floats,
                    trace_floats(lm, lm->c.max_batch));
    std::lock_guard<std::mutex> lock(lm->mu);
    lm->trace = trace;
    return SXQ_OK;
}

sxq_status sxq_lm_read_state(const sxq_lm* lm, int which, int n, float* out, void* stream) {
    if (!lm || !out) return fail(SXQ_ERR_INVALID, "lm_read_state: null pointer");
    if (n < 1 || n > lm->c.max_batch) return fail(SXQ_ERR_INVALID, "lm_read_state: bad stream count");
    const float* src = nullptr;
    size_t per = 0;
    switch (which) {
    case 0: src = lm->h; per = lm->c.dim; break;
    case 1: src = lm->logits; per = lm->c.vocab; break;
    case 2: src = lm->qkv; per = lm->qkv_n; break;
    case 3: src = lm->gu; per = 2 * (size_t)lm->c.intermediate; break;
    case 4: src = lm->qbuf; per = lm->ctx; break;
    case 5: src = lm->act_f32; per = lm->c.intermediate; break;
    default: return fail(SXQ_ERR_INVALID, "lm_read_state: unknown buffer %d", which);
    }
    DeviceGuard g(lm->device);
    HIP_TRY(g.err, "hipSetDevice");
    HIP_TRY(hipMemcpyAsync(out, src, sizeof(float) * per * n, hipMemcpyDeviceToDevice, (hipStream_t)stream),
            "lm_read_state");
    return SXQ_OK;
}

sxq_status sxq_lm_paths(const sxq_lm* lm, unsigned* paths) {
    if (!lm || !paths) return fail(SXQ_ERR_INVALID, "lm_paths: null pointer");
    *paths = (lm->attn_fused ? SXQ_LM_PATH_ATTN : 0u) | (lm->wo_fused ? SXQ_LM_PATH_ATTN_WO : 0u) |
             (lm->swiglu ? SXQ_LM_PATH_SWIGLU : 0u);
    return SXQ_OK;
}

sxq_status sxq_lm_weight_bytes(const sxq_lm* lm, size_t* layer_bytes, size_t* head_bytes) {
    if (!lm) return fail(SXQ_ERR_INVALID, "lm_weight_bytes: null handle");
    const int dt = lm->c.weight_dtype;
    auto canon = [&](const QWeight& w) { return (size_t)w.n * (size_t)w.nb * (size_t)type_size(dt); };
    size_t lb = 0;
    for (const auto& L : lm->layers) lb += canon(L.wqkv.w) + canon(L.wo.w) + canon(L.w13.w) + canon(L.w2.w);
    if (layer_bytes) *layer_bytes = lb;
    if (head_bytes) *head_bytes = canon(lm->head.w);
    return SXQ_OK;
}

}  // extern "C"
