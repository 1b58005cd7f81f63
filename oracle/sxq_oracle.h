/*
 * sxq_oracle.h -- CPU restatement of Candle 0.8's quantized CPU path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (syrinx_amd/, include/) links,
 * loads or calls this code.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, and only to check results / as the timed CPU baseline.
 *
 * What it restates.  The reference (syrinx) calls the third-party crate
 * `candle-core` 0.8 (crates.io; version requirement "0.8", no Cargo.lock, so the
 * patch level is unpinned; not vendored in the reference tree) at:
 *   crates/syrinx-lm/src/cv2/load.rs:101-104   QTensor::quantize + QMatMul::from_qtensor
 *   crates/syrinx-lm/src/cv2/mod.rs:195-211    QMatMul::forward (Module) + f32 bias add
 *   crates/syrinx-acoustic/src/cv3/mod.rs:158-164,200-203 (same API, other caller)
 * The arithmetic lives in candle-core's `src/quantized/{k_quants.rs,utils.rs,mod.rs}`
 * (GGML block formats, `from_float`, `to_float`, the generic `vec_dot_unopt` and
 * `matmul`).  Those files are absent here, so this is a restatement of their
 * published algorithm, which is the GGML `k_quants` block algebra:
 *   Q8_0  {d: f16, qs: i8[32]}                          34 B / 32 weights
 *   Q4_0  {d: f16, qs: u8[16]}                          18 B / 32 weights
 *   Q4_K  {d: f16, dmin: f16, scales: u8[12], qs: u8[128]} 144 B / 256 weights
 *   Q8_K  {d: f32, qs: i8[256], bsums: i16[16]}        292 B / 256 weights
 * The vec-dot accumulation order is the generic (non-SIMD) one, which is what a
 * default x86_64 Rust build (no `target-cpu`, no AVX target feature; the reference
 * sets no rustflags, Cargo.toml:1-60) selects.
 *
 * Each function below names the Candle function it follows.  How each one is pinned
 * (golden vectors, closed forms, brute force, exact-arithmetic known answers) is listed
 * in tests/test_oracle_*.py: f16 conversion (numpy's RNE), Q8_0/Q4_0/Q8_K from_float
 * (closed-form known answers), Q4_K from_float and make_qkx1_quants (known answers
 * derived in exact arithmetic, each catching a named slip that the tests plant into a
 * copy of this file), all to_float (hand-packed blocks), all vec_dot and matmul (f64
 * bilinear form, one-hot activations), the glue ops (the reference's fixtures, closed
 * forms).  What stays open is Candle's exact float accumulation order of vec_dot in a
 * SIMD build (the generic order is restated; the f64 bound covers either).
 */
#ifndef SXQ_ORACLE_H
#define SXQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GgmlDType discriminants (candle-core quantized/mod.rs GgmlDType). */
enum {
    ORA_F32 = 0,
    ORA_F16 = 1,
    ORA_Q4_0 = 2,
    ORA_Q8_0 = 8,
    ORA_Q4K = 12,
    ORA_Q8K = 15,
};

typedef struct { uint16_t d; int8_t qs[32]; } ora_block_q8_0;
typedef struct { uint16_t d; uint8_t qs[16]; } ora_block_q4_0;
typedef struct { float d; int8_t qs[256]; int16_t bsums[16]; } ora_block_q8k;
typedef struct { uint16_t d; uint16_t dmin; uint8_t scales[12]; uint8_t qs[128]; } ora_block_q4k;

/* Sizes / block sizes (GgmlDType::type_size, GgmlDType::block_size). 0 = unknown. */
size_t ora_type_size(int dtype);
size_t ora_block_size(int dtype);
int ora_vec_dot_type(int dtype);

/* half::f16::from_f32 (round to nearest even) and f16::to_f32. */
uint16_t ora_f32_to_f16(float f);
float ora_f16_to_f32(uint16_t h);

/* T::from_float over one row of k floats (k a multiple of the block size).
 * Returns 0, or -1 if k is not a multiple of the block size / dtype unknown. */
int ora_quantize_row(int dtype, const float *x, int64_t k, void *blocks);
/* T::to_float over one row of k elements. */
int ora_dequantize_row(int dtype, const void *blocks, int64_t k, float *y);
/* make_qkx1_quants(nmax, ntry, x[n]) -> (scale, -min). */
void ora_make_qkx1_quants(int nmax, int ntry, const float *x, int n, float *scale, float *min_out);

/* T::vec_dot_unopt(k, w_blocks, act_blocks) where act is T::VecDotType. */
float ora_vec_dot(int dtype, int64_t k, const void *w_blocks, const void *act_blocks);

/* k_quants::matmul((m,k,n), lhs f32 [m,k], rhs_t blocks [n, k/bs], dst [m,n]),
 * parallel over output columns on `threads` host threads (<=0: all cores).
 * Returns 0 or -1 (bad dtype / alignment). */
int ora_matmul(int dtype, int64_t m, int64_t k, int64_t n, const float *lhs,
               const void *rhs_blocks, float *dst, int threads);

/* f64 brute force of the same bilinear form: sum_i dequant(W_row)[i] *
 * dequant(quantize_vecdot(x))[i], accumulated in double. */
double ora_dot_f64(int dtype, int64_t k, const void *w_row_blocks, const float *x);

/* Glue ops on f32, restating the reference's op order (see sxq_oracle.c). */
void ora_rms_norm(const float *x, const float *w, int64_t n, double eps, float *y);
void ora_rope_tables_interleaved(int64_t seq_len, int64_t head_dim, double base,
                                 float *cos_out, float *sin_out);
void ora_rope_tables_half(int64_t seq_len, int64_t head_dim, float theta,
                          float *cos_out, float *sin_out);
void ora_rope_interleaved(float *x, int64_t n_heads, int64_t head_dim, const float *cos_row,
                          const float *sin_row);
void ora_rope_half(float *x, int64_t n_heads, int64_t head_dim, const float *cos_row,
                   const float *sin_row);
void ora_softmax(float *x, int64_t n);
float ora_silu(float x);
/* out[i] = silu(g[i]) * u[i] (candle_nn::ops::silu then Tensor::mul). */
void ora_silu_mul(const float *g, const float *u, int64_t n, float *out);
/* One query row of GQA decode attention for one q head over L cached positions.
 * k_cache/v_cache: [L, head_dim] for this head's kv head. */
void ora_attend_one(const float *q, const float *k_cache, const float *v_cache, int64_t L,
                    int64_t head_dim, float *out);

#ifdef __cplusplus
}
#endif
#endif
