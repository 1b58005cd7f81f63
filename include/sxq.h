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
 * including sxq_qmm_forward on one handle (the handle is read-only after creation and
 * each call allocates its own stream-ordered workspace), mirroring the reference's
 * shared `Arc<Qwen2Lm>` use (tests/real_lm_hammer.rs:48-83).
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
 * every row count (rows are processed 16 at a time on the decode GEMV). */
sxq_status sxq_qmm_forward(const sxq_qmm *qmm, const float *x, const int64_t *x_shape, int x_ndim,
                           const int64_t *x_strides, float *y, const float *bias, unsigned flags, void *stream);

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

#ifdef __cplusplus
}
#endif
#endif
