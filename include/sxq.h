/*
 * sxq.h -- C-ABI of the MI355X (gfx950) quantized-linear library, libsxq.so.
 *
 * This is the boundary a Rust (or any FFI) caller binds to replace candle-core 0.8's
 * quantized matmul behind syrinx's projection layers.  Every entry point names the
 * reference interface it replaces.  Plain pointers and sizes only; every call returns
 * an sxq_status and leaves a message in sxq_last_error() (thread-local) on failure.
 *
 * Pointer spaces: functions documented "device" take device pointers and enqueue on
 * `stream` (a hipStream_t; NULL = the default stream).  sxq_qmm_forward also accepts
 * host pointers with SXQ_HOST_PTRS (then it copies and synchronises).
 *
 * Threading: every function is safe to call concurrently from several host threads,
 * including sxq_qmm_forward on one handle (the handle is read-only after creation),
 * mirroring the reference's shared `Arc<Qwen2Lm>` use (tests/real_lm_hammer.rs:48-83).
 * sxq_qmm_forward's workspace is one buffer per device kept between calls (grown to at
 * least the largest call so far, held until the process ends); calls take turns on it
 * through an event, so concurrent calls on one device run one after another on the GPU.
 * A forward on a stream that is being captured into a graph must not use that shared
 * buffer (a replay could overlap any later eager call): sxq_qmm_forward refuses it, and
 * the caller passes a workspace of its own to sxq_qmm_forward_ws, which the graph then
 * keeps alive.
 * A decode engine (sxq_lm) owns its KV caches and work buffers, like the reference's
 * `&mut self` steps: its calls are serialised on the host (a per-engine lock), and the
 * GPU work of calls enqueued on one stream runs in call order.  Calls of one engine on
 * different streams share those buffers, so the caller orders them (an event).
 */
#ifndef SXQ_H
#define SXQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  The Rust shim maps each to candle_core::Error::Msg(sxq_last_error()). */
typedef enum {
    SXQ_OK = 0,
    SXQ_ERR_INVALID = 1,        /* null handle / pointer, negative size, bad flag   */
    SXQ_ERR_DTYPE = 2,          /* dtype not supported on this path                 */
    SXQ_ERR_BLOCK_ALIGN = 3,    /* last dim not a multiple of the block size        */
    SXQ_ERR_SHAPE = 4,          /* input incompatible with the weight shape         */
    SXQ_ERR_NOT_CONTIGUOUS = 5, /* strided input (QMatMul needs contiguous)         */
    SXQ_ERR_DEVICE = 6,         /* HIP runtime error / no device                    */
    SXQ_ERR_OOM = 7,            /* device allocation failed                         */
} sxq_status;

/* GgmlDType discriminants (candle-core quantized::GgmlDType; the reference selects
 * Q4_0 at crates/syrinx-lm/src/cv2/load.rs:101-102). */
typedef enum {
    SXQ_F32 = 0,
    SXQ_F16 = 1,
    SXQ_Q4_0 = 2,
    SXQ_Q8_0 = 8,
    SXQ_Q4K = 12,
    SXQ_Q8K = 15,
} sxq_dtype;

/* sxq_qmm_forward flags */
#define SXQ_DEVICE_PTRS 0u /* x, y, bias are device pointers; async on `stream` */
#define SXQ_HOST_PTRS 1u   /* x, y, bias are host pointers; the call synchronises */
#define SXQ_BIT_EXACT 2u   /* every row count through Candle's integer vec-dot (bit-identical); without it
                              a Q4_K weight with >= 64 rows of x runs the f16 MFMA prefill GEMM, whose
                              outputs differ from Candle's by less than 2^-10 * sum_k |w_k x_k| */
#define SXQ_BF16_INPUT 4u  /* x holds bf16 values (the Fish GPU path's activations,
                              crates/syrinx-fish/src/s2/mod.rs:113), passed through the same `x`
                              pointer; they widen to f32 exactly on the device, so y is that of an f32
                              x holding the same values, bit for bit.  y and bias stay f32. */

/* Thread-local text of the last failure on this thread ("" if none). */
const char *sxq_last_error(void);
/* Library version string. */
const char *sxq_version(void);

/* GgmlDType::block_size() (used as the alignment predicate at
 * crates/syrinx-lm/src/cv2/load.rs:101).  0 for an unknown dtype. */
size_t sxq_block_size(int dtype);
/* GgmlDType::type_size(): bytes per block (storage accounting at load.rs:103). */
size_t sxq_type_size(int dtype);
/* Number of visible GPUs. */
sxq_status sxq_device_count(int *count);

/* QTensor::quantize(&Tensor, GgmlDType) (crates/syrinx-lm/src/cv2/load.rs:102), device:
 * x f32 [rows, k] -> canonical GGML block bytes [rows, k/bs*type_size] (Candle's
 * from_float, byte-identical).  dtype in {Q4_0, Q8_0, Q4K, Q8K}. */
sxq_status sxq_quantize_rows(int device, int dtype, const float *x, int64_t rows, int64_t k, void *out_blocks,
                             void *stream);

/* QTensor::dequantize(&Device) (crates/syrinx-vocoder/src/cv2/mod.rs:172,
 * crates/syrinx-speaker/src/campplus/mod.rs:172), device: canonical blocks -> f32
 * (Candle's to_float, bit-identical). */
sxq_status sxq_dequantize_rows(int device, int dtype, const void *blocks, int64_t rows, int64_t k, float *out,
                               void *stream);

/* Activation quantization exactly as Candle's QMatMul forward performs it before the
 * vec-dot (k_quants::matmul step 1): x f32 [m, k] -> canonical Q8_0 (vec_dtype =
 * SXQ_Q8_0) or Q8_K (SXQ_Q8K) blocks, device.  This is the same wave quantizer the
 * GEMV path uses, exported in canonical bytes so the bit-exact test can read it. */
sxq_status sxq_act_quantize(int device, int vec_dtype, const float *x, int64_t m, int64_t k, void *out_blocks,
                            void *stream);

/* ---- QMatMul --------------------------------------------------------------------- */
typedef struct sxq_qmm sxq_qmm;

/* QMatMul::from_qtensor(QTensor::quantize(w, dtype)) (crates/syrinx-lm/src/cv2/load.rs:102-104):
 * a weight of shape [n, k] given as canonical GGML blocks (`blocks`, `nbytes` =
 * n*k/bs*type_size), from host memory (src_is_device = 0) or device memory (1).  The
 * library copies and repacks them; the caller keeps its buffer.
 * dtype in {Q4_0, Q8_0, Q4K}. */
sxq_status sxq_qmm_create(int device, int dtype, int64_t n, int64_t k, const void *blocks, size_t nbytes,
                          int src_is_device, sxq_qmm **out);

/* impl Module for QMatMul::forward(&self, xs) (called at crates/syrinx-lm/src/cv2/mod.rs:197,
 * plus the f32 bias add of :207-210 when `bias` is non-null):
 * x f32 with shape x_shape[0..x_ndim) whose last dim must equal k (Candle: "input
 * tensor ... incompatible with ..."), x_ndim >= 2 ("input tensor has only one
 * dimension"), contiguous (x_strides NULL or row-major; else NOT_CONTIGUOUS);
 * y f32 [prod(x_shape[:-1]), n].  Outputs equal Candle's CPU vec-dot bit for bit for
 * every row count of Q8_0 / Q4_0 weights (the decode GEMV up to 127 rows, 16 at a time;
 * from 128 rows a GEMM on the int8 matrix cores that keeps Candle's per-block float
 * order), and of Q4_K weights below 64 rows or with SXQ_BIT_EXACT; Q4_K with 64 or more
 * rows runs the f16 MFMA prefill GEMM (error bound at SXQ_BIT_EXACT above). */
sxq_status sxq_qmm_forward(const sxq_qmm *qmm, const float *x, const int64_t *x_shape, int x_ndim,
                           const int64_t *x_strides, float *y, const float *bias, unsigned flags, void *stream);

/* Device workspace bytes sxq_qmm_forward_ws needs for m rows of x (with `flags` as the
 * forward will get them).  No reference counterpart: Candle allocates inside forward. */
sxq_status sxq_qmm_workspace_size(const sxq_qmm *qmm, int64_t m, unsigned flags, size_t *bytes);

/* QMatMul::forward exactly as sxq_qmm_forward (same checks, kernels and bits), on device
 * pointers, with a caller-provided device workspace (`workspace_bytes` >=
 * sxq_qmm_workspace_size, 256-byte aligned) instead of the library's shared one: for
 * code under graph capture (the graph owns the workspace, so replays never alias other
 * calls) and callers that manage their own memory.  Calls that share one workspace
 * must not overlap.  flags: SXQ_BIT_EXACT, SXQ_BF16_INPUT. */
sxq_status sxq_qmm_forward_ws(const sxq_qmm *qmm, const float *x, const int64_t *x_shape, int x_ndim,
                              const int64_t *x_strides, float *y, const float *bias, unsigned flags,
                              void *workspace, size_t workspace_bytes, void *stream);

/* QMatMul::forward as sxq_qmm_forward (same checks, kernels and bits) on device pointers
 * for callers that cannot allocate device memory: code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc.  No counterpart in the reference
 * (Candle allocates inside forward).  Its workspace is a fixed 64 MiB scratch array in
 * the library's device image, one per GPU, held until the process ends; a call whose
 * workspace would exceed it fails with SXQ_ERR_INVALID before any GPU work (the decode
 * GEMV fits at any usual row count, the prefill GEMM up to ~1024 rows at the Qwen3-4B
 * shapes).  Every call on one GPU shares that scratch: calls that overlap on a GPU (on
 * different streams, or replays of graphs holding such calls) race and must be ordered
 * by the caller.  flags: SXQ_BIT_EXACT, SXQ_BF16_INPUT. */
sxq_status sxq_qmm_forward_noalloc(const sxq_qmm *qmm, const float *x, const int64_t *x_shape, int x_ndim,
                                   const int64_t *x_strides, float *y, const float *bias, unsigned flags,
                                   void *stream);

/* QTensor::{dtype, shape, storage_size_in_bytes} (storage accounting: load.rs:103). */
sxq_status sxq_qmm_info(const sxq_qmm *qmm, int *dtype, int64_t *n, int64_t *k, size_t *storage_bytes);

/* QTensor::dequantize for the weight held by a QMatMul: f32 [n, k], device. */
sxq_status sxq_qmm_dequantize(const sxq_qmm *qmm, float *out, void *stream);

/* Export the weight back as canonical GGML block bytes (device), e.g. to persist it. */
sxq_status sxq_qmm_export(const sxq_qmm *qmm, void *out_blocks, void *stream);

/* Drop the QMatMul (Rust Drop of the last Arc).  NULL is accepted. */
sxq_status sxq_qmm_destroy(sxq_qmm *qmm);

/* Fill device memory with N(mean, std) f32 samples (counter-based SplitMix64 +
 * Box-Muller): synthetic weights for benchmarks.  No reference counterpart. */
sxq_status sxq_fill_normal(int device, float *out, int64_t n, uint64_t seed, float mean, float std_dev,
                           void *stream);

/* ---- Embedding tables: per-row int8 / int4 with dequant-on-gather -------------------
 * quantize_embed (crates/syrinx-lm/src/cv2/quant.rs:38-89) and embed_rows
 * (crates/syrinx-lm/src/cv2/generate.rs:22-67), the embedding policy of
 * Qwen2Lm::load_quantized (cv2/load.rs:86-91).  Row r of an f32 table [rows, h] gets
 * scale[r] = max|row| / qmax + 1e-12 and codes round(x / scale) in [-qmax, qmax]:
 *   SXQ_EMBED_INT8: qmax 127, q [rows, h] bytes code + 128;
 *   SXQ_EMBED_INT4: qmax 7, q [rows, h / 2] bytes, element 2j in the low nibble of byte j,
 *                   2j + 1 in the high one, each code + 8 (h must be even).
 * A gathered element is (float)code * scale[row], bit for bit the reference's. */
enum { SXQ_EMBED_INT4 = 4, SXQ_EMBED_INT8 = 8 };
/* The scheme a table of row width h is stored at: int4 falls back to int8 for odd h
 * (quant.rs:41-46). */
sxq_status sxq_embed_scheme(int requested, int64_t h, int *effective);
/* Quantize a device f32 table into device q (rows * h or rows * h / 2 bytes) and scale
 * (rows floats), enqueued on `stream`. */
sxq_status sxq_embed_quantize(int device, int scheme, const float *table, int64_t rows, int64_t h, uint8_t *q,
                              float *scale, void *stream);
/* out f32 [n, h] = the dequantized rows ids[0..n) (device int32; an id outside the table
 * gives a zero row), enqueued on `stream`. */
sxq_status sxq_embed_gather(int device, int scheme, const uint8_t *q, const float *scale, int64_t rows, int64_t h,
                            const int32_t *ids, int n, float *out, void *stream);

/* ---- Decoder step: the callers of QMatMul in one autoregressive LM token ------------
 *
 * One decode step of a Qwen2/Qwen3-style LM for up to 16 independent streams, all on
 * the device: embedding -> n_layers x [RMSNorm -> fused QKV projection (+bias) ->
 * QK-RMSNorm -> RoPE -> KV append -> GQA attention -> O projection + residual ->
 * RMSNorm -> gate|up projection -> SiLU*mul -> down projection + residual] -> final
 * RMSNorm -> head projection (+bias) -> logits and greedy argmax.  Every projection is
 * the library's QMatMul GEMV over the same weight dtype.  It replaces, per token:
 *   Fish s2 slow AR:  SlowAr::slow_step / slow_step_batch (crates/syrinx-fish/src/s2/slow_ar.rs:259-271,456-499),
 *                     run_layers (:166-202), head (:207-246), embed (:101-161);
 *   CosyVoice2 LM:    Qwen2Lm::forward_logits_cached (crates/syrinx-lm/src/cv2/mod.rs:261-286),
 *                     attn_cached (crates/syrinx-lm/src/cv2/attention.rs:46-78);
 * with the per-token loops of crates/syrinx-fish/src/common/dualar.rs:188-219 and
 * crates/syrinx-lm/src/cv2/generate.rs:150-161 keeping their host-side sampling.
 * Streams may hold different cache lengths (ragged batches) and need no left padding.
 */
typedef struct sxq_lm sxq_lm;

typedef struct {
    int32_t n_layers;
    int32_t dim;              /* hidden size */
    int32_t n_heads;          /* query heads */
    int32_t n_kv_heads;       /* key/value heads (GQA) */
    int32_t head_dim;         /* <= 256, multiple of 4 */
    int32_t intermediate;     /* SwiGLU width */
    int32_t vocab;            /* head output rows */
    int32_t embed_rows;       /* rows of a dense embedding table (0 = vocab); unused when tied */
    int32_t max_seq;          /* KV capacity per stream (positions) */
    int32_t max_batch;        /* streams per step, 1..16 */
    int32_t weight_dtype;     /* SXQ_Q4K, SXQ_Q8_0 or SXQ_Q4_0 for every projection */
    float norm_eps;           /* RMSNorm eps (also QK-RMSNorm) */
    float rope_theta;         /* RoPE base */
    int32_t rope_interleaved; /* 1: rotate pairs (2i, 2i+1) (Fish); 0: (i, i + hd/2) (Qwen2) */
    int32_t qk_norm;          /* per-head RMSNorm of q and k before RoPE (Qwen3) */
    int32_t qkv_bias;         /* biases on q, k, v (Qwen2) */
    int32_t head_bias;        /* bias on the head (CosyVoice2 llm_decoder) */
    int32_t tied_embedding;   /* the head is the quantized input table (Fish embeddings.weight): the token
                                 embedding gathers the dense table once one is uploaded (SXQ_LM_EMBED, as
                                 SlowAr::embed does, crates/syrinx-fish/src/s2/slow_ar.rs:117), else the
                                 dequantized head row */
    int32_t n_codebooks;      /* Fish MCF: codebook rows summed on semantic positions; 0 = none */
    int32_t codebook_size;
    int32_t semantic_begin;   /* semantic token id range (inclusive) for the MCF scale */
    int32_t semantic_end;
    int32_t o_bias;           /* bias on wo (Fish `attention.wo.bias`, detected from the checkpoint at
                                 crates/syrinx-fish/src/s2/slow_ar.rs:91-93) */
} sxq_lm_config;

/* Projection slots for sxq_lm_set_linear (layer-local unless noted). */
enum {
    SXQ_LM_WQKV = 0, /* fused [q; k; v] rows (Fish wqkv, crates/syrinx-fish/src/s2/load.rs:271-312) */
    SXQ_LM_WQ = 1,   /* separate q/k/v (Qwen2 q_proj/k_proj/v_proj) fused on upload */
    SXQ_LM_WK = 2,
    SXQ_LM_WV = 3,
    SXQ_LM_WO = 4,
    SXQ_LM_W1 = 5,   /* gate */
    SXQ_LM_W3 = 6,   /* up */
    SXQ_LM_W2 = 7,   /* down */
    SXQ_LM_HEAD = 8  /* model-level: output head (tied embedding table for Fish) */
};
/* Vector slots for sxq_lm_set_vector. */
enum {
    SXQ_LM_ATTN_NORM = 0,
    SXQ_LM_FFN_NORM = 1,
    SXQ_LM_Q_NORM = 2,
    SXQ_LM_K_NORM = 3,
    SXQ_LM_BQ = 4,
    SXQ_LM_BK = 5,
    SXQ_LM_BV = 6,
    SXQ_LM_FINAL_NORM = 7,     /* model-level */
    SXQ_LM_HEAD_BIAS = 8,      /* model-level */
    SXQ_LM_EMBED = 9,          /* model-level dense table [embed_rows, dim] */
    SXQ_LM_CODEBOOK_EMBED = 10, /* model-level [n_codebooks * codebook_size, dim] */
    SXQ_LM_BO = 11              /* wo bias [dim] (o_bias models) */
};

/* sxq_lm_step flags */
#define SXQ_LM_GRAPH 1u /* replay the step as a captured HIP graph (captured on first use per batch size) */

sxq_status sxq_lm_create(int device, const sxq_lm_config *cfg, sxq_lm **out);
/* Copy a QMatMul's weight into a projection slot (shape and dtype must match). */
sxq_status sxq_lm_set_linear(sxq_lm *lm, int layer, int which, const sxq_qmm *w);
/* Copy an f32 vector (norm weight, bias, embedding table) into a slot. */
sxq_status sxq_lm_set_vector(sxq_lm *lm, int layer, int which, const float *data, int64_t n, int src_is_device);
/* Hold the model's dense input table (SXQ_LM_EMBED, [embed_rows, dim]) as a per-row int8 /
 * int4 table instead (sxq_embed_quantize's layout, device pointers copied in): every step
 * and prefill then dequantizes the rows it gathers (Qwen2Lm::embed_rows of the quantized
 * build, cv2/generate.rs:22-67).  Only for models with an untied input table. */
sxq_status sxq_lm_set_embed_quantized(sxq_lm *lm, int scheme, const uint8_t *q, const float *scale);
/* Synthetic weights: every projection N(0, std) quantized with from_float, norm weights
 * 1, biases / tables N(0, std).  For benchmarks; no reference counterpart. */
sxq_status sxq_lm_init_random(sxq_lm *lm, uint64_t seed, float std_dev);
/* Fill the whole KV cache with N(0, 1) and set the first n_streams lengths (a
 * prefilled cache for decode benchmarks). */
sxq_status sxq_lm_kv_fill_random(sxq_lm *lm, const int32_t *lengths, int n_streams, uint64_t seed);
/* Set / read the cached lengths (= next positions) of the first n_streams streams
 * (KvCache::len, crates/syrinx-fish/src/s2/nn.rs:237-240).  Setting 0 resets a stream
 * (SlowAr::reset, slow_ar.rs:79-81). */
sxq_status sxq_lm_set_lengths(sxq_lm *lm, const int32_t *lengths, int n_streams);
sxq_status sxq_lm_get_lengths(const sxq_lm *lm, int32_t *lengths, int n_streams);
/* Empty the caches of streams 0..n_streams-1, ordered on `stream` (no host wait): the
 * per-frame reset of the Fish fast AR's local cache (crates/syrinx-fish/src/s2/fast_ar.rs:
 * a new KvCache per expand), and SlowAr::reset.  Must not be recorded into a graph. */
sxq_status sxq_lm_reset(sxq_lm *lm, int n_streams, void *stream);
/* One decode step for streams 0..n_streams-1 (device pointers, enqueued on `stream`):
 *   ids      int32 [n_streams, 1 + n_codebooks] token ids (Fish frame: semantic id then
 *            codes), or NULL to reuse the previous step's argmax (codes kept);
 *   embeds   f32 [n_streams, dim] input embeddings instead of ids (CosyVoice2 passes
 *            embeddings to forward_logits_cached), or NULL;
 *   logits   f32 [n_streams, vocab] output, or NULL;
 *   hidden   f32 [n_streams, dim] output, or NULL: the post-final-RMSNorm hidden state the
 *            head multiplies (the `hidden` SlowAr::head returns for the fast AR,
 *            crates/syrinx-fish/src/s2/slow_ar.rs:207-246, consumed at
 *            crates/syrinx-fish/src/common/dualar.rs:196);
 *   next_ids int32 [n_streams] greedy argmax of the logits, or NULL.
 * Each stream's token is placed at its current length, which then advances by one.
 * Projections keep Candle's bits, except with 5..16 streams where a projection's 16-row
 * tiles would leave compute units idle (the 2560-row wo and w2): their K is split over
 * workgroups whose partials are added in a fixed order (deterministic; within 1e-6 of
 * sum |w x| per output).  The environment variable SXQ_BIT_EXACT=1 (read at each
 * launch, so at capture for a graph) keeps every projection bit-identical. */
sxq_status sxq_lm_step(sxq_lm *lm, int n_streams, const int32_t *ids, const float *embeds, float *logits,
                       float *hidden, int32_t *next_ids, unsigned flags, void *stream);
/* sxq_lm_prefill flags */
#define SXQ_LM_EXACT 2u      /* Q4_K projections through Candle's integer vec-dot (bit-identical) rather than the
                                f16 MFMA GEMM; Q8_0 / Q4_0 are bit-identical either way */
#define SXQ_LM_ALL_LOGITS 4u /* logits (and hidden) for every prompt token, as Qwen2Lm::forward_logits_cached
                                returns them; otherwise only each stream's last prompt token (SlowAr::prefill) */

/* Prompt prefill of streams 0..n_streams-1 (device pointers, enqueued on `stream`):
 *   SlowAr::prefill / prefill_batch (crates/syrinx-fish/src/s2/slow_ar.rs:250-256, 404-454),
 *   Qwen2Lm::forward_logits_cached with t_new > 1 (crates/syrinx-lm/src/cv2/mod.rs:261-286).
 * counts  host int32 [n_streams], tokens per stream (>= 1 each; ragged, no padding);
 * ids     int32 [sum counts, 1 + n_codebooks] stream-major token frames, or NULL;
 * embeds  f32 [sum counts, dim] input embeddings instead of ids, or NULL;
 * Stream s's tokens take positions len[s] .. len[s] + counts[s] - 1 (each query attends its
 * own stream's cache up to its own position), their keys and values are written to the
 * cache, and len[s] advances by counts[s].  Outputs (each may be NULL): logits f32
 * [n_streams, vocab] and hidden f32 [n_streams, dim] (post-final-RMSNorm) of each stream's
 * last token, or with SXQ_LM_ALL_LOGITS [sum counts, vocab] / [sum counts, dim];
 * next_ids int32 [n_streams] the greedy argmax of each stream's last logits.  Every
 * projection runs on all sum(counts) rows at once (the prefill GEMMs).
 * trace (test instrumentation, NULL for none): the f32 intermediates as for
 * sxq_lm_set_trace with n = sum(counts) rows per segment (the final hidden: one row per
 * stream, or per token with SXQ_LM_ALL_LOGITS); sxq_lm_prefill_trace_floats gives its size.
 * head_dim must be 64 or 128. */
sxq_status sxq_lm_prefill(sxq_lm *lm, int n_streams, const int32_t *counts, const int32_t *ids,
                          const float *embeds, float *logits, float *hidden, int32_t *next_ids, unsigned flags,
                          float *trace, size_t trace_capacity_floats, void *stream);
sxq_status sxq_lm_prefill_trace_floats(const sxq_lm *lm, int64_t tokens, size_t *floats);

/* ---- Samplers: the reference's seeded token draws on the device ---------------------
 * A decode loop samples each step's logits on the GPU and writes the token straight into
 * the next step's ids, so only token ids (not logit rows) ever cross to the host.  Each
 * stream has its own SplitMix64 state (rng[s], device uint64, seeded by the caller with the
 * reference's seed and advanced per draw exactly as the reference advances it).  The Fish
 * draws take any top_k >= 0 (0 = unbounded, common/sampling.rs:50-52); beyond 64 kept
 * candidates the top-p cut is decided on fixed-point (2^-60) masses rather than the
 * reference's f64 running sum, which can differ only when that sum lands within ~n * 2^-60
 * of top_p.  The CosyVoice draw takes top_k 1..64 (its reference pins 25); RAS windows hold
 * at most 64 ids.  out[s * out_stride] receives stream s's token (an ids frame's semantic
 * slot, say). */
typedef struct {
    float temperature;        /* softmax temperature of the normal draw */
    float top_p;              /* nucleus cutoff */
    int32_t top_k;            /* candidate cap; 0 = unbounded */
    float repetition_penalty; /* codebook draws: divides positive / multiplies negative logits of `recent` ids; 1 = off */
    int32_t ras_win_size;     /* semantic draws: RAS window (recent semantic ids), <= 64 */
    float ras_high_temp;      /* RAS fallback draw */
    float ras_high_top_p;
    int32_t semantic_begin;   /* semantic draws may pick only [begin, end] and stop_id (begin > end: any id) */
    int32_t semantic_end;
    int32_t stop_id;
} sxq_fish_sampling;

/* Sampler::sample_semantic (crates/syrinx-fish/src/common/sampling.rs:150-163) for n
 * streams: logits f32 [n][vocab] (row stride logits_stride floats, left unchanged), the
 * semantic constraint, a normal and a high-temperature draw, the high one used when the
 * normal token is a semantic id already in the stream's window.  window int32
 * [n][ras_win_size] (oldest first) and window_len int32 [n] (device, may both be NULL): the
 * driver's rolling window (common/dualar.rs:188-205), updated with the drawn token unless
 * it is stop_id.  active int32 [n] (device, or NULL): drive_batch's per-stream "not
 * finished" flag (common/dualar.rs:286-305): a stream whose flag is 0 draws nothing (its rng
 * and window are kept, its token is written as 0, the inert pad), and a stream that draws
 * stop_id has its flag cleared. */
sxq_status sxq_sample_semantic(int device, const float *logits, int64_t logits_stride, int n, int vocab,
                               const sxq_fish_sampling *params, uint64_t *rng, int32_t *window, int32_t *window_len,
                               int32_t *active, int32_t *out, int out_stride, void *stream);
/* Sampler::sample_codebook (common/sampling.rs:139-145): the repetition penalty over recent
 * [n][n_recent] ids (or NULL), then the temperature / top-p / top-k draw.  active as for
 * sxq_sample_semantic, read only (FastAr::expand_batch's `active`, s2/fast_ar.rs:206-213). */
sxq_status sxq_sample_codebook(int device, const float *logits, int64_t logits_stride, int n, int vocab,
                               const sxq_fish_sampling *params, uint64_t *rng, const int32_t *recent, int n_recent,
                               const int32_t *active, int32_t *out, int out_stride, void *stream);
/* CosyVoice ras_sampling after log_softmax_vec (crates/syrinx-lm/src/cv2/sampling.rs:13-22,
 * 104-124; the generate loop at crates/syrinx-lm/src/cv2/generate.rs:150-161): logits f32
 * [n][vocab] are overwritten with their log-probabilities (ids [eos_begin, eos_end) at -inf
 * when ignore_eos), a nucleus draw (top_p, top_k), replaced by a draw from the full
 * distribution when it repeats >= win * tau_r times among the stream's last `win` tokens.
 * decoded int32 [n][win] (oldest first) and decoded_len [n] (device, may both be NULL): that
 * history, extended by the drawn token unless it is a stop id. */
sxq_status sxq_sample_ras(int device, float *logits, int64_t logits_stride, int n, int vocab, int ignore_eos,
                          int eos_begin, int eos_end, float top_p, int top_k, int win, float tau_r, uint64_t *rng,
                          int32_t *decoded, int32_t *decoded_len, int32_t *out, int out_stride, void *stream);

/* FastAr::expand / expand_batch (crates/syrinx-fish/src/s2/fast_ar.rs:116-224) on the
 * device, over a fast-AR engine `fast` (sxq_lm with n_codebooks 0, a dense embedding table
 * -- the shared fast_embeddings -- of >= vocab rows, vocab = the residual codebook size,
 * max_seq >= n_codes), for streams 0..n_streams-1, enqueued on `stream`:
 *   hidden   f32 [n_streams, dim] (device) the slow head's hidden (sxq_lm_step's `hidden`),
 *            run at position 0 (the conditioning prefix; its logits are unused);
 *   semantic int32, stream s at semantic[s * semantic_stride]: the sampled semantic ids;
 *            codebook 0 is first_code = clamp(semantic - params->semantic_begin, 0, vocab - 1);
 *   active   int32 [n_streams] or NULL: 0 marks a finished stream, which draws nothing (its
 *            rng is kept and its codes are 0), as expand_batch's `active`;
 *   codes    int32 output, codebook cb of stream s at codes[s * codes_stride + cb],
 *            cb = 0..n_codes-1; codebook cb >= 1 is Sampler::sample_codebook (params, rng[s],
 *            no repetition list: the reference passes an empty `recent`) of position cb's
 *            logits, and position cb + 1 embeds it.
 * The engine's caches are emptied first (a fresh KvCache per frame) and hold n_codes
 * positions afterwards.  With SXQ_LM_GRAPH the whole expansion is one HIP graph, captured
 * per distinct argument set (pointers, strides, sampling values) and replayed after.
 * Fish's slow ids frame [semantic, code 0 .. code n_codes-1] is filled in place by passing
 * semantic = frame, codes = frame + 1 and both strides = 1 + n_codes. */
sxq_status sxq_fish_fast_expand(sxq_lm *fast, int n_streams, const float *hidden, const int32_t *semantic,
                                int semantic_stride, const int32_t *active, const sxq_fish_sampling *params,
                                uint64_t *rng, int n_codes, int32_t *codes, int codes_stride, unsigned flags,
                                void *stream);

/* Enqueue only the projection GEMVs of one step (every layer's fused QKV, O, gate|up
 * and down, plus the head if with_head) on the step's current activations: the
 * GEMV share of a token, for bandwidth measurement.  No reference counterpart. */
sxq_status sxq_lm_gemv_pass(sxq_lm *lm, int n_streams, int with_head, void *stream);
/* Read cached post-RoPE keys and values [count, head_dim] (device) for tests. */
sxq_status sxq_lm_read_kv(const sxq_lm *lm, int layer, int stream_idx, int kv_head, int pos0, int count, float *k_out,
                          float *v_out, void *stream);
/* Copy a step buffer of the first n streams (device) for tests: 0 = residual stream
 * after the last layer [n, dim], 1 = logits [n, vocab], 2 = last layer's q|k|v
 * projection [n, qkv], 3 = last layer's gate|up [n, 2*intermediate], 4 = last layer's
 * post-RoPE queries [n, n_heads*head_dim], 5 = the silu(g)*u row the fused one-row
 * gate|up GEMV last wrote [n, intermediate] (zero until it runs).  No reference
 * counterpart. */
sxq_status sxq_lm_read_state(const sxq_lm *lm, int which, int n_streams, float *out, void *stream);
/* Test instrumentation (no reference counterpart): with a trace buffer set, every
 * step also records its f32 intermediates, for n_streams streams, in this order:
 * embedding output [n, dim]; per layer hn_attn [n, dim], qkv [n, qkv], post-RoPE q
 * [n, n_heads*head_dim], attention context [n, n_heads*head_dim], h after the O
 * residual [n, dim], hn_ffn [n, dim], gate|up [n, 2*intermediate], silu*mul [n,
 * intermediate], h after the down residual [n, dim]; then the final hn [n, dim].
 * sxq_lm_trace_floats gives the size for n streams; the buffer must hold the size
 * for max_batch.  NULL turns tracing off. */
sxq_status sxq_lm_trace_floats(const sxq_lm *lm, int n_streams, size_t *floats);
sxq_status sxq_lm_set_trace(sxq_lm *lm, float *trace, size_t capacity_floats);
/* Bytes of quantized projection weights read by one step (layers + head). */
sxq_status sxq_lm_weight_bytes(const sxq_lm *lm, size_t *layer_bytes, size_t *head_bytes);
/* Which fused launches a one-stream step of this engine runs (test instrumentation, no
 * reference counterpart): bit 0 the decode attention in one kernel, bit 1 attention and
 * the O projection in one launch, bit 2 the SwiGLU pair (gate|up with the SiLU*mul
 * epilogue, down with the quantizing prologue). */
#define SXQ_LM_PATH_ATTN 1u
#define SXQ_LM_PATH_ATTN_WO 2u
#define SXQ_LM_PATH_SWIGLU 4u
sxq_status sxq_lm_paths(const sxq_lm *lm, unsigned *paths);
sxq_status sxq_lm_destroy(sxq_lm *lm);

#ifdef __cplusplus
}
#endif
#endif
