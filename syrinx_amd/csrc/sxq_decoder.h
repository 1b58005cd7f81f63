// sxq_decoder.h -- launchers of the decoder-step glue kernels (sxq_decoder.hip).
#pragma once
#include "sxq_kernels.h"

namespace sxq {

// rec (optional, Q8_K, rows <= 16): also fill the rows' MmaRec records [dim / 256].
hipError_t launch_rmsnorm_quant(int vdt, const float* h, int rows, int dim, const float* w, float eps, uint8_t* act,
                                float* normed, hipStream_t s, MmaRec* rec = nullptr);
hipError_t launch_qk_rope_append(const float* qkv, int B, int qkv_n, int nh, int nkv, int hd, const float* qn,
                                 const float* kn, float eps, int interleaved, const float* cos_t, const float* sin_t,
                                 const int* len, float* qout, float* kc, float* vc, int64_t kv_stream_stride,
                                 int max_seq, hipStream_t s);
// Attention splits: at most kMaxSplits partials per head are merged, so a stream holds
// at most kMaxSplits * kAttnSplit positions.
constexpr int kAttnSplit = 32;
// Positions per split of the fused decode attention (fewer, larger splits: a cheaper merge).
constexpr int kAttnSplitFused = 64;
constexpr int kMaxSplits = 512;
// The fused kernel: workgroup size and the most splits one of its merges takes.
constexpr int kAttnThreads = 512;
constexpr int kMaxSplitsFused = kMaxSplits * kAttnSplit / kAttnSplitFused;
// The stride the launches use: kCounterStride, or 1 with SXQ_COUNTERS_PACKED set (for
// comparison; the buffers are sized for kCounterStride either way).
int counter_stride();
// The O projection's ready counter is kept in copies (counter_stride() words apart): every
// context slice bumps each copy, and each projection workgroup polls one, so that the
// hundreds of pollers and the slices' atomics do not all meet on one line.  ready_copies():
// kReadyCopies, or SXQ_READY_COPIES (1..kReadyCopies).
constexpr int kReadyCopies = 8;
int ready_copies();
size_t attn_partial_lds(int nh, int nkv, int hd, int P);
hipError_t launch_attention(int vdt, const float* q, const float* kc, const float* vc, const int* len, int B, int nh,
                            int nkv, int hd, int max_seq, int64_t kv_stream_stride, int P, int max_splits,
                            float* part, uint8_t* act, float* ctx_out, hipStream_t s);
// Fused decode attention (QK-norm + RoPE + KV append + split partials + last-arriver
// merge + quantization of the context); counter: [B * nkv * kCounterStride] zero before
// the first call (each call leaves it zero).  q_out / ctx_out optional (tests).  Returns
// hipErrorInvalidValue when the head group is not a whole number of activation blocks
// (attn_decode_fits); the caller then uses the three-kernel path.
bool attn_decode_fits(int vdt, int nh, int nkv, int hd, int max_splits);
// grid_splits (both fused launches): the splits per (stream, KV head) the grid holds, at
// least every stream's (len + 64) / 64 at this launch; 0 = every split of max_seq.  A
// smaller grid leaves out workgroups that would only find their split empty.
// Allow the fused kernel its dynamic LDS (above 64 KB); call once before launching.
hipError_t attn_decode_prepare(int vdt, int nh, int nkv, int hd, int max_splits);
hipError_t launch_attention_decode(int vdt, const float* qkv, int B, int qkv_n, int nh, int nkv, int hd, const float* qn,
                                   const float* kn, float eps, int interleaved, const float* cos_t, const float* sin_t,
                                   const int* len, float* kc, float* vc, int64_t kv_stream_stride, int max_seq,
                                   int max_splits, float* part, unsigned* counter, uint8_t* act, float* ctx_out,
                                   float* q_out, hipStream_t s, MmaRec* rec = nullptr, int grid_splits = 0);
hipError_t launch_silu_mul_quant(int vdt, const float* gu, int B, int I, uint8_t* act, float* act_f32, hipStream_t s,
                                 MmaRec* rec = nullptr);
// The RoPE row at stream 0's length, copied by the step's embedding kernel (beside its own
// work) for the fused attention of every layer: out[i] = cos_t[len[0] * half + i],
// out[half + i] = sin_t[...], i < half (<= 128).
struct RopeRow {
    const int* len = nullptr;
    const float* cos_t = nullptr;
    const float* sin_t = nullptr;
    int half = 0;
    float* out = nullptr;
};
// table: the dense input table [table_rows][dim], or null to dequantize the rows of the tied head w
hipError_t launch_embed_mcf(const int* ids, int ids_per, int B, const float* table, int64_t table_rows,
                            const QWeight& w, int dim, const float* cb, int n_cb, int cb_size, int sem_begin,
                            int sem_end, float* h, hipStream_t s, const RopeRow& rr = RopeRow());
hipError_t launch_embed_dense(const int* ids, int ids_per, int B, const float* table, int rows, int dim, float* h,
                              hipStream_t s, const RopeRow& rr = RopeRow());
// Greedy argmax per stream; with `len` also advances each stream's cached length.
// pval/pidx: [B * kArgmaxSlices] partials; counter: [B * kCounterStride], zero before the
// first call (each call leaves it zero again).
constexpr int kArgmaxSlices = 64;
hipError_t launch_argmax(const float* logits, int B, int vocab, int* ids, int ids_per, int* out_ids, int* len,
                         float* pval, int* pidx, unsigned* counter, hipStream_t s);
hipError_t launch_fill_value(float* y, int64_t n, float v, hipStream_t s);
// A fill kernel (not a memset node, so it may sit inside a captured graph).
hipError_t launch_fill_int(int* y, int n, int v, hipStream_t s);

// ---- prompt prefill (sxq_prefill.hip) -------------------------------------------------
// Per-token QK-RMSNorm + RoPE + KV write: tok[2 t] = stream, tok[2 t + 1] = position of
// prompt token t; queries -> qout [T][nh * hd].  hd in {64, 128}.
hipError_t launch_prefill_rope_kv(const float* qkv, int T, int qkv_n, int nh, int nkv, int hd, const float* qn,
                                  const float* kn, float eps, int interleaved, const float* cos_t, const float* sin_t,
                                  const int* tok, float* qout, float* kc, float* vc, int64_t kv_stream_stride,
                                  int max_seq, hipStream_t s);
// Causal GQA attention of the prompt's queries over each stream's cache; tiles[4 i ..]
// = {stream, first token row, token count (<= prefill_tile_tokens), first position}.
bool prefill_attn_supported(int nh, int nkv, int hd);
int prefill_tile_tokens(int nh, int nkv);
hipError_t launch_prefill_attn(const float* q, const float* kc, const float* vc, const int* tiles, int n_tiles, int nh,
                               int nkv, int hd, int max_seq, int64_t kv_stream_stride, float* ctx, hipStream_t s);
// The token and tile tables of one prefill, built on the device from the per-stream
// token counts and cache lengths (streams 0 .. n-1, tokens stream-major): tok (2 ints per
// token), tiles (4 ints per tile, at most T + n tiles), last[s] = row of stream s's last
// token (-1 without tokens); lengths[s] += counts[s] when `advance` (after the layers).
struct PrefillMeta {
    int n, tile_tokens;
    int counts[16], lens[16];
};
hipError_t launch_prefill_tables(const PrefillMeta& pm, int T, int* tok, int* tiles, int* last, hipStream_t s);
hipError_t launch_prefill_advance(const PrefillMeta& pm, int* len, hipStream_t s);
// dst[i] = src[idx[i]] for n rows of `cols` floats.
hipError_t launch_gather_rows(const float* src, const int* idx, int n, int cols, float* dst, hipStream_t s);

// Arguments of the fused decode attention over one step of B streams.
struct AttnArgs {
    const float* qkv;  // [B][qkv_n]: q (nh*hd) | k (nkv*hd) | v (nkv*hd)
    int qkv_n, nh, nkv;
    const float *qn, *kn;  // QK-norm weights [hd], or null
    float eps, inv_hd, scale;
    int interleaved;
    const float *cos_t, *sin_t;  // RoPE tables [max_seq][hd/2]
    const int* len;              // [B] cached positions before this step
    float *kc, *vc;              // caches [B][nkv][max_seq][hd], stream stride kv_stream_stride
    int64_t kv_stream_stride;
    int max_seq;
    float* part;  // partial records [B][nh][max_splits][hd + 4]
    int max_splits;
    unsigned* counter;       // [B][nkv] arrival counters, cstride words apart, zero between launches
    int cstride;
    uint8_t* act;            // [B] quantized context rows (the O projection's input)
    float *ctx_out, *q_out;  // optional f32 copies of the context and the roped queries
    unsigned* ready;         // k_attn_wo_decode: context slices published so far (ready_copies copies)
    int ready_copies;
    uint32_t pub_off;        // k_attn_wo_decode: LDS byte offset of the slice staging
    MmaRec* rec;             // optional (Q8_K, B <= 16): the context rows' MmaRec records too
    const float* rope_row;   // k_attn_wo_decode: stream 0's RoPE row (cos [hd/2], sin [hd/2]), or null
};

// Batch-1 decode attention and the O projection (Q4_K, y += ctx . Wo^T in place) as one
// launch: the projection's workgroups follow the attention's and wait for the n_kv
// context slices.  ready: this launch's counter, zero at the launch; ready_next: a counter
// that no launch in flight uses, zeroed by this one (the counters of consecutive layers
// chain this way: layer l's launch zeroes layer l + 1's); each is kReadyCopies counters
// counter_stride() words apart.
bool attn_wo_decode_fits(int vdt, int nh, int nkv, int hd, int max_splits, const QWeight& wo, int dim);
hipError_t attn_wo_decode_prepare(int vdt, int nh, int nkv, int hd, int max_splits, const QWeight& wo);
// rope_row (optional): the step's RoPE row at stream 0's length (cos [hd/2] then sin,
// copied there earlier in the step, e.g. by launch_embed_* with RopeRow): the splits then
// issue their loads before the length returns (the queries' and new key's inputs with
// that row, both tiles); without it they wait for the length first.
hipError_t launch_attention_wo_decode(int vdt, const float* qkv, int qkv_n, int nh, int nkv, int hd, const float* qn,
                                      const float* kn, float eps, int interleaved, const float* cos_t,
                                      const float* sin_t, const int* len, float* kc, float* vc, int max_seq,
                                      int max_splits, float* part, unsigned* counter, uint8_t* act, const QWeight& wo,
                                      float* y, unsigned* ready, unsigned* ready_next, float* ctx_out, float* q_out,
                                      hipStream_t s, int grid_splits = 0, const float* rope_row = nullptr);

}  // namespace sxq
