// sxq_decoder.hip -- the per-token glue between the quantized projections of one
// decoder step, on the device: RMSNorm (+ activation quantization), QK-RMSNorm + RoPE
// + KV-cache append, split-K GQA decode attention (+ activation quantization of the
// context), SiLU*mul (+ quantization), embeddings, argmax and length bookkeeping.
//
// Reference (what each kernel restates, f32 throughout as on the reference CPU path):
//   RMSNorm            crates/syrinx-fish/src/s2/nn.rs:100-106, crates/syrinx-lm/src/cv2/mod.rs:181-186
//   QK-RMSNorm         crates/syrinx-fish/src/s2/nn.rs:325-331
//   RoPE interleaved   crates/syrinx-fish/src/s2/nn.rs:154-166 (tables :117-141)
//   RoPE rotate-half   crates/syrinx-lm/src/cv2/attention.rs:82-88 (tables :108-119)
//   KV append          crates/syrinx-fish/src/s2/nn.rs:244-254, crates/syrinx-lm/src/cv2/mod.rs:147-157
//   decode attention   crates/syrinx-fish/src/s2/nn.rs:340-352, crates/syrinx-lm/src/cv2/attention.rs:67-76
//   SwiGLU             crates/syrinx-fish/src/s2/nn.rs:452-457, crates/syrinx-lm/src/cv2/mod.rs:222-228
//   MCF embedding      crates/syrinx-fish/src/s2/slow_ar.rs:101-161
// The quantization kernels feed the next projection exactly what QMatMul::forward would
// compute from the same f32 input (the wave quantizers of sxq_quant_dev.h).
#include "sxq_attn_dev.h"
#include "sxq_decoder.h"
#include "sxq_gemv_dev.h"
#include "sxq_sync_dev.h"
#include "sxq_quant_dev.h"

namespace sxq {

SXQ_DEV float wave_sum_f32(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Quantize chunk c of a row of `dim` elements (elements c*256 .. c*256+255, whose
// values start at `vals`) into the device activation layout `act_row` (row of blocks).
template <int VDT>
SXQ_DEV void quantize_chunk(const float* vals, int c, int dim, int lane, uint8_t* act_row) {
    const int e0 = c * 256 + 4 * lane;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (e0 < dim) v = make_float4(vals[4 * lane], vals[4 * lane + 1], vals[4 * lane + 2], vals[4 * lane + 3]);
    if (VDT == kQ8K) {
        wave_quantize_q8k<false>(v, lane, act_row + (size_t)c * sizeof(ActQ8K));
    } else {
        const int nb = dim / 32;
        wave_quantize_q8_0<false>(v, lane, c * 8 + (lane >> 3) < nb, act_row + (size_t)c * 8 * sizeof(ActQ8_0));
    }
}

// ---------------------------------------------------------------------------- RMSNorm
// y = (x / sqrt(sum(x*x) * inv_n + eps)) * w  over each row; then quantized.  The sum
// is a fixed-order tree here (rmsnorm_sumsq_1024) and sequential in Candle's CPU loop:
// results agree to rounding.  grid (rows, ceil(dim/256)), 1024 threads: every
// workgroup reduces the whole row (an L2-resident read) and then its first wave
// normalises and quantizes the workgroup's own 256-element chunk.
template <int VDT>
__global__ __launch_bounds__(1024) void k_rmsnorm_quant(const float* __restrict__ h, int dim, const float* __restrict__ w,
                                                        float inv_n, float eps, uint8_t* __restrict__ act,
                                                        float* __restrict__ normed, MmaRec* __restrict__ rec) {
    __shared__ float red[16];
    const int row = blockIdx.x, c = blockIdx.y, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const float* x = h + (int64_t)row * dim;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < dim / 4; i += 1024) {  // dim is a multiple of 32
        const float4 v = ((const float4*)x)[i];
        ss += v.x * v.x;
        ss += v.y * v.y;
        ss += v.z * v.z;
        ss += v.w * v.w;
    }
    ss = rmsnorm_sumsq_1024(ss, red);
    const float var = ss * inv_n + 0.0f;
    const float den = sqrtf(var * 1.0f + eps);
    if (wave != 0) return;
    const int e0 = c * 256 + 4 * lane;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (e0 < dim) {
        const float4 xv = *(const float4*)(x + e0), wv = *(const float4*)(w + e0);
        v.x = (xv.x / den) * wv.x;
        v.y = (xv.y / den) * wv.y;
        v.z = (xv.z / den) * wv.z;
        v.w = (xv.w / den) * wv.w;
        if (normed) *(float4*)(normed + (int64_t)row * dim + e0) = v;
    }
    const int nb = VDT == kQ8K ? dim / 256 : dim / 32;
    uint8_t* arow = act + (int64_t)row * nb * act_block_bytes(VDT);
    if (VDT == kQ8K) wave_quantize_q8k<false>(v, lane, arow + (size_t)c * sizeof(ActQ8K), rec ? rec + c : nullptr, row);
    else wave_quantize_q8_0<false>(v, lane, c * 8 + (lane >> 3) < nb, arow + (size_t)c * 8 * sizeof(ActQ8_0));
}

// ---------------------------------------------------- QK-RMSNorm + RoPE + KV-cache append
// One head by one wave: optional per-head RMSNorm (QK-norm) then RoPE, src -> dst
// (hd <= 256).  Pairs: interleaved (2i, 2i+1) or rotate-half (i, i + hd/2); lane i
// owns pairs i and i + 64.  cos_row/sin_row: the RoPE tables at this position.
SXQ_DEV void wave_norm_rope(const float* src, const float* nw, float eps, float inv_hd, int hd, int interleaved,
                            const float* cos_row, const float* sin_row, float* dst, int lane) {
    constexpr int MAXP = 2;  // hd <= 256
    const int half = hd / 2;
    float a[MAXP], b[MAXP];
    int ia[MAXP], ib[MAXP];
    float ss = 0.0f;
#pragma unroll
    for (int t = 0; t < MAXP; ++t) {
        const int i = lane + 64 * t;
        ia[t] = interleaved ? 2 * i : i;
        ib[t] = interleaved ? 2 * i + 1 : i + half;
        a[t] = b[t] = 0.0f;
        if (i < half) {
            a[t] = src[ia[t]];
            b[t] = src[ib[t]];
            ss += a[t] * a[t] + b[t] * b[t];
        }
    }
    if (nw) {
        ss = wave_sum_f32(ss);
        const float den = sqrtf((ss * inv_hd + 0.0f) * 1.0f + eps);
#pragma unroll
        for (int t = 0; t < MAXP; ++t) {
            if (lane + 64 * t < half) {
                a[t] = (a[t] / den) * nw[ia[t]];
                b[t] = (b[t] / den) * nw[ib[t]];
            }
        }
    }
#pragma unroll
    for (int t = 0; t < MAXP; ++t) {
        const int i = lane + 64 * t;
        if (i < half) {
            const float c = cos_row[i], sn = sin_row[i];
            dst[ia[t]] = a[t] * c - b[t] * sn;
            dst[ib[t]] = b[t] * c + a[t] * sn;
        }
    }
}

// grid (B, n_heads + 2 * n_kv), one wave per head of the fused qkv row
// [q (nh*hd) | k (nkv*hd) | v (nkv*hd)]: queries -> qout, keys and values -> the cache
// at the stream's current length.
__global__ __launch_bounds__(64) void k_qk_rope_append(const float* __restrict__ qkv, int qkv_n, int nh, int nkv,
                                                       int hd, const float* __restrict__ qn,
                                                       const float* __restrict__ kn, float eps, float inv_hd,
                                                       int interleaved, const float* __restrict__ cos_t,
                                                       const float* __restrict__ sin_t, const int* __restrict__ len,
                                                       float* __restrict__ qout, float* __restrict__ kc,
                                                       float* __restrict__ vc, int64_t kv_stream_stride,
                                                       int max_seq) {
    const int s = blockIdx.x, hid = blockIdx.y, lane = threadIdx.x;
    const int pos = len[s];
    const float* src = qkv + (int64_t)s * qkv_n + (int64_t)hid * hd;
    const int half = hd / 2;
    const bool is_q = hid < nh, is_k = !is_q && hid < nh + nkv;
    if (!is_q && !is_k) {  // V: stored as projected
        const int g = hid - nh - nkv;
        float* dst = vc + (int64_t)s * kv_stream_stride + ((int64_t)g * max_seq + pos) * hd;
        for (int d = lane; d < hd; d += 64) dst[d] = src[d];
        return;
    }
    float* dst = is_q ? qout + ((int64_t)s * nh + hid) * hd
                      : kc + (int64_t)s * kv_stream_stride + ((int64_t)(hid - nh) * max_seq + pos) * hd;
    wave_norm_rope(src, is_q ? qn : kn, eps, inv_hd, hd, interleaved, cos_t + (int64_t)pos * half,
                   sin_t + (int64_t)pos * half, dst, lane);
}

// Split merge of one stream's attention partials part_s [nh][max_splits][hd + 4]
// (record {m, l, 0, 0, acc[hd]}, 16-byte aligned):
//   ctx = sum_i exp(m_i - M) acc_i / sum_i exp(m_i - M) l_i,  M = max_i m_i.
// merge_weights (one wave per head, 4 waves) fills wts[hh][i] = exp(m_i - M) and
// lsum[hh] for heads h0 .. h0 + nhc - 1; merge_elem then gives one context element.
SXQ_DEV void merge_weights(const float* part_s, int h0, int nhc, int nsp, int hd, int max_splits, float* wts,
                           float* lsum) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int hh = wave; hh < nhc; hh += 4) {
        const float* ph = part_s + (int64_t)(h0 + hh) * max_splits * (hd + 4);
        float M = -INFINITY;
        for (int i = lane; i < nsp; i += 64) M = fmaxf(M, ph[i * (hd + 4)]);
        M = wave_max_f32(M);
        float Ls = 0.0f;
        for (int i = lane; i < nsp; i += 64) {
            const float w = expf(ph[i * (hd + 4)] - M);
            wts[hh * kMaxSplits + i] = w;
            Ls += ph[i * (hd + 4) + 1] * w;
        }
        Ls = wave_sum_f32(Ls);
        if (lane == 0) lsum[hh] = Ls;
    }
}
SXQ_DEV float merge_elem(const float* part_s, int h, int hh, int d, int nsp, int hd, int max_splits, const float* wts,
                         const float* lsum) {
    const float* ph = part_s + (int64_t)h * max_splits * (hd + 4) + 4 + d;
    float acc = 0.0f;
    for (int i = 0; i < nsp; ++i) acc += ph[i * (hd + 4)] * wts[hh * kMaxSplits + i];
    return acc / lsum[hh];
}

// ------------------------------------------------------------- split-K decode attention
// One workgroup takes P consecutive cached positions of one KV head for all G = nh/nkv
// query heads sharing it (GQA without materialising repeat_kv) and writes per-head
// partials {m, l, 0, 0, acc[hd]} (records of hd + 4 floats):
//   m = max_j s_j, l = sum_j exp(s_j - m), acc = sum_j exp(s_j - m) v_j,
// with s_j = (q . k_j) * scale.  attn_tile_partials does that from LDS tiles: qs [G][hd],
// kt/vt [P][hd + 4] (np valid rows), scratch sc [G][P]; pm points at head 0's partial of
// this split, head_stride floats apart.  256 threads, all of which must call it.
SXQ_DEV void attn_tile_partials(const float* qs, const float* kt, const float* vt, float* sc, int G, int P, int np,
                                int hd, float scale, float* pm, int64_t head_stride) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, hdp = hd + 4;
    // scores: a lane pair per (head, position), each lane half of the head dim
    for (int base = 0; base < 2 * G * P; base += 256) {
        const int i = base + tid;
        const int pair = i >> 1, half = i & 1;
        const int h = pair / P, p = pair - h * P;
        float acc = 0.0f;
        if (i < 2 * G * P && p < np) {
            const float* qh = qs + h * hd + half * (hd / 2);
            const float* kr = kt + p * hdp + half * (hd / 2);
            for (int d = 0; d < hd / 2; d += 4) {
                const float4 kv = *(const float4*)(kr + d);
                const float4 qv = *(const float4*)(qh + d);
                acc += qv.x * kv.x;
                acc += qv.y * kv.y;
                acc += qv.z * kv.z;
                acc += qv.w * kv.w;
            }
        }
        acc += __shfl_xor(acc, 1, 64);
        if (i < 2 * G * P && half == 0 && p < np) sc[h * P + p] = acc * scale + 0.0f;
    }
    __syncthreads();
    for (int h = wave; h < G; h += 4) {
        float mx = -INFINITY;
        for (int p = lane; p < np; p += 64) mx = fmaxf(mx, sc[h * P + p]);
        mx = wave_max_f32(mx);
        float l = 0.0f;
        for (int p = lane; p < np; p += 64) {
            const float e = expf(sc[h * P + p] - mx);
            sc[h * P + p] = e;
            l += e;
        }
        l = wave_sum_f32(l);
        if (lane == 0) {
            store_agent(&pm[h * head_stride], mx);
            store_agent(&pm[h * head_stride + 1], l);
        }
    }
    __syncthreads();
    // Weighted values: a thread per 4 consecutive head-dim columns of a head (one 16-byte
    // LDS read of V per position feeds 4 independent sums), each summed over the
    // positions in order.
    for (int i = tid; i < G * hd / 4; i += 256) {
        const int h = (4 * i) / hd, d = 4 * i - h * hd;
        const float* e = sc + h * P;
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll 4
        for (int p = 0; p < np; ++p) {
            const float w = e[p];
            const float4 v = *(const float4*)(vt + p * hdp + d);
            acc.x += w * v.x;
            acc.y += w * v.y;
            acc.z += w * v.z;
            acc.w += w * v.w;
        }
        store_agent(&pm[h * head_stride + 4 + d], acc.x);
        store_agent(&pm[h * head_stride + 5 + d], acc.y);
        store_agent(&pm[h * head_stride + 6 + d], acc.z);
        store_agent(&pm[h * head_stride + 7 + d], acc.w);
    }
}

// grid (B, n_kv, max_splits), 256 threads: the partials of split z over the cache
// (keys/values already appended); k_attn_combine_quant merges the splits.
__global__ __launch_bounds__(256) void k_attn_partial(const float* __restrict__ q, const float* __restrict__ kc,
                                                      const float* __restrict__ vc, const int* __restrict__ len,
                                                      int nh, int nkv, int hd, int max_seq,
                                                      int64_t kv_stream_stride, int P, float scale,
                                                      float* __restrict__ part, int max_splits) {
    extern __shared__ float4 smem4[];  // float4: 16-byte aligned after any static LDS
    float* smem = (float*)smem4;
    const int s = blockIdx.x, g = blockIdx.y, sp = blockIdx.z;
    const int L = len[s] + 1;  // the token appended this step is attended too
    const int p0 = sp * P;
    if (p0 >= L) return;
    const int np = min(P, L - p0);
    const int G = nh / nkv, hdp = hd + 4;
    float* qs = smem;               // [G][hd]
    float* kt = qs + G * hd;        // [P][hd + 4]
    float* vt = kt + P * hdp;       // [P][hd + 4]
    float* sc = vt + P * hdp;       // [G][P]
    const int tid = threadIdx.x;
    const int64_t off = (int64_t)s * kv_stream_stride + ((int64_t)g * max_seq + p0) * hd;
    const float* kb = kc + off;
    const float* vb = vc + off;
    for (int i = tid; i < G * hd; i += 256) qs[i] = q[((int64_t)s * nh + g * G) * hd + i];
    load_kv_tile(kt, vt, kb, vb, np, hd);
    __syncthreads();
    float* pm = part + (((int64_t)s * nh + g * G) * max_splits + sp) * (hd + 4);
    attn_tile_partials(qs, kt, vt, sc, G, P, np, hd, scale, pm, (int64_t)max_splits * (hd + 4));
}

// The per-launch kernel: grid (B, n_kv, ceil(max_seq / kAttnSplitFused)), kAttnThreads threads.
// At least six waves per SIMD (at most 80 VGPRs): three workgroups per CU, as the LDS
// allows.  GC: the query heads per KV head as a compile-time constant, or 0 (read at
// run time).
template <int VDT, int HD, int GC>
__global__ __launch_bounds__(kAttnThreads) __attribute__((amdgpu_waves_per_eu(6, 8))) void k_attn_decode(AttnArgs A) {
    static_assert(kAttnThreads / 8 == kAttnSplitFused, "a split is one position per 8 lanes");
    extern __shared__ float4 smem4[];  // float4: 16-byte aligned after any static LDS
    __shared__ bool last;
    attn_decode_body<VDT, HD, kAttnThreads, GC>(A, blockIdx.x, blockIdx.y, blockIdx.z, (float*)smem4, &last);
}

// grid (B, ceil(nh*hd/256)), 256 threads: merge the splits of the heads covering
// context elements [c*256, c*256 + 256), then quantize that chunk for the O projection.
template <int VDT>
__global__ __launch_bounds__(256) void k_attn_combine_quant(const float* __restrict__ part, const int* __restrict__ len,
                                                            int nh, int hd, int P, int max_splits,
                                                            uint8_t* __restrict__ act, float* __restrict__ ctx_out) {
    __shared__ float xs[256];
    __shared__ float wts[8 * kMaxSplits];
    __shared__ float lsum[8];
    const int s = blockIdx.x, c = blockIdx.y, tid = threadIdx.x;
    const int dim = nh * hd;
    const int L = len[s] + 1;
    const int nsp = (L + P - 1) / P;
    const int h0 = (c * 256) / hd;
    const int nhc = min((256 + hd - 1) / hd, nh - h0);  // heads touching this chunk (<= 8)
    const float* part_s = part + (int64_t)s * nh * max_splits * (hd + 4);
    merge_weights(part_s, h0, nhc, nsp, hd, max_splits, wts, lsum);
    __syncthreads();
    const int e = c * 256 + tid;
    float v = 0.0f;
    if (e < dim) {
        const int h = e / hd, d = e - h * hd;
        v = merge_elem(part_s, h, h - h0, d, nsp, hd, max_splits, wts, lsum);
        if (ctx_out) ctx_out[(int64_t)s * dim + e] = v;
    }
    xs[tid] = v;
    __syncthreads();
    if (tid < 64) {
        const int nb = VDT == kQ8K ? dim / 256 : dim / 32;
        uint8_t* arow = act + (int64_t)s * nb * act_block_bytes(VDT);
        quantize_chunk<VDT>(xs, c, dim, tid, arow);
    }
}

// ------------------------------------------------------------------------ SwiGLU glue
// gu row = [gate (I) | up (I)]; a = silu(g) * u with silu(g) = g / (1 + exp(-g)).
template <int VDT>
__global__ __launch_bounds__(64) void k_silu_mul_quant(const float* __restrict__ gu, int I, uint8_t* __restrict__ act,
                                                       float* __restrict__ act_f32, MmaRec* __restrict__ rec) {
    const int s = blockIdx.x, c = blockIdx.y, lane = threadIdx.x;
    const float* g = gu + (int64_t)s * 2 * I;
    const float* u = g + I;
    const int e0 = c * 256 + 4 * lane;
    float a[4] = {0.f, 0.f, 0.f, 0.f};
    if (e0 < I) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float gv = g[e0 + r];
            a[r] = (gv / (1.0f + expf(-gv))) * u[e0 + r];
            if (act_f32) act_f32[(int64_t)s * I + e0 + r] = a[r];
        }
    }
    const float4 v = make_float4(a[0], a[1], a[2], a[3]);
    const int nb = VDT == kQ8K ? I / 256 : I / 32;
    uint8_t* arow = act + (int64_t)s * nb * act_block_bytes(VDT);
    if (VDT == kQ8K) wave_quantize_q8k<false>(v, lane, arow + (size_t)c * sizeof(ActQ8K), rec ? rec + c : nullptr, s);
    else wave_quantize_q8_0<false>(v, lane, c * 8 + (lane >> 3) < nb, arow + (size_t)c * 8 * sizeof(ActQ8_0));
}

// ------------------------------------------------------------------------ embeddings
// Element e of row `r` of a quantized weight in the device layout, exactly to_float.
SXQ_DEV float weight_elem(const QWeight& w, int64_t r, int e) {
    if (w.dtype == kQ4K) {
        const int b = e >> 8, i = e & 255;
        const int64_t blk = r * w.nb + b;
        const uint8_t* hb = w.hdr + blk * 16;
        const int c = i >> 6, hi = (i >> 5) & 1, l32 = i & 31;
        const int j = 2 * c + hi;
        int sc, m;
        const uint8_t* q = hb + 4;
        if (j < 4) {
            sc = q[j] & 63;
            m = q[j + 4] & 63;
        } else {
            sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
            m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
        }
        const float d = f16_bits_to_f32((uint16_t)(hb[0] | (hb[1] << 8)));
        const float dmin = f16_bits_to_f32((uint16_t)(hb[2] | (hb[3] << 8)));
        const int l = l32 & 7, t = l32 >> 3;
        const uint8_t byte = w.qs[blk * 128 + 4 * (4 * l + c) + t];
        const int qv = hi ? (byte >> 4) : (byte & 0xF);
        return (d * (float)sc) * (float)qv - dmin * (float)m;
    }
    const int b = e >> 5, i = e & 31;
    const int64_t blk = r * w.nb + b;
    const float d = f16_bits_to_f32((uint16_t)(w.hdr[2 * blk] | (w.hdr[2 * blk + 1] << 8)));
    if (w.dtype == kQ8_0) return (float)(int8_t)w.qs[blk * 32 + i] * d;
    const uint8_t byte = w.qs[blk * 16 + (i & 15)];
    return (float)((i < 16 ? (byte & 0xF) : (byte >> 4)) - 8) * d;
}

// Fish MCF (slow_ar.rs:101-161):
//   x = (E[tok] + sum_i C[code_i + i*cb]) * 1/sqrt(n_cb + 1)   on semantic positions,
//   x = E[tok] + 0 * (...)                                      otherwise,
// with E the dense embeddings.weight table when given (`table`, [rows][dim], the gather
// of :117), else the dequantized rows of the tied head w (rows = w.n).  Without codebooks
// (n_cb = 0) this is the plain gather E[tok].  Ids outside the table (token >= rows,
// code >= cb_size, negatives) read nothing: their rows count as zero.
// The step's RoPE row (RopeRow): workgroup (0, 0)'s first 2 * half threads, beside their
// embedding element.
SXQ_DEV void rope_row_copy(const RopeRow& rr) {
    if (rr.out && blockIdx.x == 0 && blockIdx.y == 0 && (int)threadIdx.x < 2 * rr.half) {
        const int t = threadIdx.x, i = t < rr.half ? t : t - rr.half;
        rr.out[t] = (t < rr.half ? rr.cos_t : rr.sin_t)[(int64_t)rr.len[0] * rr.half + i];
    }
}

__global__ __launch_bounds__(256) void k_embed_mcf(const int* __restrict__ ids, int ids_per,
                                                   const float* __restrict__ table, int64_t rows, QWeight w, int dim,
                                                   const float* __restrict__ cb, int n_cb, int cb_size,
                                                   int sem_begin, int sem_end, float inv_scale,
                                                   float* __restrict__ h, RopeRow rr) {
    rope_row_copy(rr);
    const int s = blockIdx.x;
    const int* fr = ids + (int64_t)s * ids_per;
    const int tok = fr[0];
    const bool tok_ok = tok >= 0 && (int64_t)tok < rows;
    const bool sem = tok >= sem_begin && tok <= sem_end;
    const int e = blockIdx.y * 256 + threadIdx.x;  // grid (B, ceil(dim / 256))
    if (e < dim) {
        float x = !tok_ok ? 0.0f : table ? table[(int64_t)tok * dim + e] : weight_elem(w, tok, e);
        if (n_cb > 0) {
            // the codebooks' values are loaded kCbBatch at a time (all in flight together),
            // then added in codebook order
            constexpr int kCbBatch = 16;
            float vq = 0.0f;
            for (int i0 = 0; i0 < n_cb; i0 += kCbBatch) {
                float v[kCbBatch];
#pragma unroll
                for (int j = 0; j < kCbBatch; ++j) {
                    const int i = i0 + j;
                    const int code = i < n_cb ? fr[1 + i] : -1;
                    v[j] = (code >= 0 && code < cb_size) ? cb[((int64_t)code + (int64_t)i * cb_size) * dim + e] : 0.0f;
                }
#pragma unroll
                for (int j = 0; j < kCbBatch; ++j)
                    if (i0 + j < n_cb) vq = i0 + j == 0 ? v[j] : vq + v[j];
            }
            x = (x + vq * (sem ? 1.0f : 0.0f)) * (sem ? inv_scale : 1.0f);
        }
        h[(int64_t)s * dim + e] = x;
    }
}

__global__ __launch_bounds__(256) void k_embed_dense(const int* __restrict__ ids, int ids_per,
                                                     const float* __restrict__ table, int rows, int dim,
                                                     float* __restrict__ h, RopeRow rr) {
    rope_row_copy(rr);
    const int s = blockIdx.x;
    const int tok = ids[(int64_t)s * ids_per];
    const bool ok = tok >= 0 && tok < rows;
    const int e = blockIdx.y * 256 + threadIdx.x;  // grid (B, ceil(dim / 256))
    if (e < dim) h[(int64_t)s * dim + e] = ok ? table[(int64_t)tok * dim + e] : 0.0f;
}

// ------------------------------------------------------------------------ argmax / length
// First index of the largest logit (NaN never wins); written to ids[s * ids_per].
// grid (B, kArgmaxSlices): workgroup b reduces slice b of the row and publishes
// (value, index); the last workgroup of a stream to finish (a per-stream counter) folds
// the partials in slice order -- so ties keep the first index -- writes the id, bumps
// the stream's cached length (the step is complete) and resets the counter for the
// next step.
SXQ_DEV void argmax_merge(float& best, int& idx, float ov, int oi) {
    if (ov > best || (ov == best && oi < idx)) { best = ov; idx = oi; }
}
__global__ __launch_bounds__(256) void k_argmax(const float* __restrict__ logits, int vocab, int* __restrict__ ids,
                                                int ids_per, int* __restrict__ out_ids, int* __restrict__ len,
                                                float* __restrict__ pval, int* __restrict__ pidx,
                                                unsigned* __restrict__ counter, int cstride) {
    __shared__ float bv[4];
    __shared__ int bi[4];
    __shared__ bool last;
    const int s = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int slice = (vocab + kArgmaxSlices - 1) / kArgmaxSlices;
    const int lo = b * slice, hi = min(vocab, lo + slice);
    const float* x = logits + (int64_t)s * vocab;
    float best = -INFINITY;
    int idx = 0x7FFFFFFF;
    // a thread's loads issued together (kArgmaxBatch at a time), then compared in index
    // order: per-thread indices rise, so the first max is kept
    constexpr int kArgmaxBatch = 16;
    for (int i0 = lo + tid; i0 < hi; i0 += kArgmaxBatch * 256) {
        float v[kArgmaxBatch];
#pragma unroll
        for (int j = 0; j < kArgmaxBatch; ++j) {
            const int i = i0 + j * 256;
            v[j] = i < hi ? x[i] : -INFINITY;
        }
#pragma unroll
        for (int j = 0; j < kArgmaxBatch; ++j)
            if (v[j] > best) { best = v[j]; idx = i0 + j * 256; }
    }
    for (int o = 32; o >= 1; o >>= 1) argmax_merge(best, idx, __shfl_xor(best, o, 64), __shfl_xor(idx, o, 64));
    if (lane == 0) { bv[wave] = best; bi[wave] = idx; }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 4; ++w) argmax_merge(best, idx, bv[w], bi[w]);
        store_agent(&pval[s * kArgmaxSlices + b], best);
        store_agent(&pidx[s * kArgmaxSlices + b], idx);
    }
    if (!publish_and_count(&counter[s * cstride], kArgmaxSlices, &last)) return;
    if (wave == 0) {
        best = load_agent(&pval[s * kArgmaxSlices + lane]);
        idx = load_agent(&pidx[s * kArgmaxSlices + lane]);
        for (int o = 32; o >= 1; o >>= 1) argmax_merge(best, idx, __shfl_xor(best, o, 64), __shfl_xor(idx, o, 64));
        if (lane == 0) {
            if (idx == 0x7FFFFFFF) idx = 0;
            ids[(int64_t)s * ids_per] = idx;
            if (out_ids) out_ids[s] = idx;
            if (len) len[s] += 1;
            __hip_atomic_store(&counter[s * cstride], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

__global__ void k_fill_value(float* __restrict__ y, int64_t n, float v) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = v;
}

__global__ void k_fill_int(int* __restrict__ y, int n, int v) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = v;
}

// ------------------------------------------------------------------------ launchers
hipError_t launch_rmsnorm_quant(int vdt, const float* h, int rows, int dim, const float* w, float eps, uint8_t* act,
                                float* normed, hipStream_t s, MmaRec* rec) {
    if (rec && (vdt != kQ8K || rows > 16)) return hipErrorInvalidValue;
    const float inv_n = (float)(1.0 / (double)dim);
    const dim3 grid(rows, (dim + 255) / 256);
    if (vdt == kQ8K)
        hipLaunchKernelGGL((k_rmsnorm_quant<kQ8K>), grid, dim3(1024), 0, s, h, dim, w, inv_n, eps, act, normed, rec);
    else
        hipLaunchKernelGGL((k_rmsnorm_quant<kQ8_0>), grid, dim3(1024), 0, s, h, dim, w, inv_n, eps, act, normed, rec);
    return hipGetLastError();
}

hipError_t launch_qk_rope_append(const float* qkv, int B, int qkv_n, int nh, int nkv, int hd, const float* qn,
                                 const float* kn, float eps, int interleaved, const float* cos_t, const float* sin_t,
                                 const int* len, float* qout, float* kc, float* vc, int64_t kv_stream_stride,
                                 int max_seq, hipStream_t s) {
    const float inv_hd = (float)(1.0 / (double)hd);
    hipLaunchKernelGGL(k_qk_rope_append, dim3(B, nh + 2 * nkv), dim3(64), 0, s, qkv, qkv_n, nh, nkv, hd, qn, kn, eps,
                       inv_hd, interleaved, cos_t, sin_t, len, qout, kc, vc, kv_stream_stride, max_seq);
    return hipGetLastError();
}

size_t attn_partial_lds(int nh, int nkv, int hd, int P) {
    const int G = nh / nkv;
    return sizeof(float) * ((size_t)G * hd + 2 * (size_t)P * (hd + 4) + (size_t)G * P);
}

hipError_t launch_attention(int vdt, const float* q, const float* kc, const float* vc, const int* len, int B, int nh,
                            int nkv, int hd, int max_seq, int64_t kv_stream_stride, int P, int max_splits,
                            float* part, uint8_t* act, float* ctx_out, hipStream_t s) {
    const float scale = (float)(1.0 / sqrt((double)hd));
    hipLaunchKernelGGL(k_attn_partial, dim3(B, nkv, max_splits), dim3(256), attn_partial_lds(nh, nkv, hd, P), s, q, kc,
                       vc, len, nh, nkv, hd, max_seq, kv_stream_stride, P, scale, part, max_splits);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int chunks = (nh * hd + 255) / 256;
    if (vdt == kQ8K) hipLaunchKernelGGL((k_attn_combine_quant<kQ8K>), dim3(B, chunks), dim3(256), 0, s, part, len, nh, hd, P, max_splits, act, ctx_out);
    else hipLaunchKernelGGL((k_attn_combine_quant<kQ8_0>), dim3(B, chunks), dim3(256), 0, s, part, len, nh, hd, P, max_splits, act, ctx_out);
    return hipGetLastError();
}

// Fused attention LDS (P = kAttnThreads/8 positions per split): the partial phase's
// tiles, or the merge phase's split weights and per-set sums, whichever is larger (the
// partial phase, at the decode shapes).
static size_t attn_decode_lds(int nh, int nkv, int hd, int max_splits) {
    const size_t G = nh / nkv, gd = G * hd, nq = kAttnThreads / (gd / 4), P = kAttnThreads / 8;
    const size_t nspf = (size_t)max_splits < (size_t)kMaxSplitsFused ? max_splits : kMaxSplitsFused;
    const size_t partial = P * hd + hd + G * P + (nq > 1 ? nq - 1 : 1) * gd;  // the queries share the sums' space
    const size_t merge = ((G * nspf + G + 3) & ~(size_t)3) + nq * gd;
    return sizeof(float) * (partial > merge ? partial : merge);
}

bool attn_decode_fits(int vdt, int nh, int nkv, int hd, int max_splits) {
    const int G = nh / nkv;
    return (hd == 64 || hd == 128) && G >= 1 && G <= 8 && (G * hd) % (vdt == kQ8K ? 256 : 32) == 0 &&
           attn_decode_lds(nh, nkv, hd, max_splits) <= 160 * 1024;
}

// The instance for a head group: G = 4 at head_dim 128 (Qwen3-4B, 32/8 heads) and G = 7
// at head_dim 64 (Qwen2-0.5B, 14/2 heads) compiled for their G, any other group size
// through the run-time instance.
template <int VDT, int HD, int GC>
static const void* attn_decode_fn() {
    return (const void*)k_attn_decode<VDT, HD, GC>;
}
template <int VDT>
static const void* attn_decode_kernel_vdt(int hd, int G) {
    if (hd == 128) return G == 4 ? attn_decode_fn<VDT, 128, 4>() : attn_decode_fn<VDT, 128, 0>();
    return G == 7 ? attn_decode_fn<VDT, 64, 7>() : attn_decode_fn<VDT, 64, 0>();
}
static const void* attn_decode_kernel(int vdt, int hd, int G) {
    return vdt == kQ8K ? attn_decode_kernel_vdt<kQ8K>(hd, G) : attn_decode_kernel_vdt<kQ8_0>(hd, G);
}

hipError_t attn_decode_prepare(int vdt, int nh, int nkv, int hd, int max_splits) {
    const int lds = (int)attn_decode_lds(nh, nkv, hd, max_splits);
    return hipFuncSetAttribute(attn_decode_kernel(vdt, hd, nh / nkv), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
}

int ready_copies() {
    static const int copies = [] {
        const char* e = getenv("SXQ_READY_COPIES");
        const int v = e ? atoi(e) : kReadyCopies;
        return v < 1 ? 1 : (v > kReadyCopies ? kReadyCopies : v);
    }();
    return copies;
}

int counter_stride() {
    static const int stride = getenv("SXQ_COUNTERS_PACKED") ? 1 : kCounterStride;
    return stride;
}

hipError_t launch_attention_decode(int vdt, const float* qkv, int B, int qkv_n, int nh, int nkv, int hd, const float* qn,
                                   const float* kn, float eps, int interleaved, const float* cos_t, const float* sin_t,
                                   const int* len, float* kc, float* vc, int64_t kv_stream_stride, int max_seq,
                                   int max_splits, float* part, unsigned* counter, uint8_t* act, float* ctx_out,
                                   float* q_out, hipStream_t s, MmaRec* rec, int grid_splits) {
    if (!attn_decode_fits(vdt, nh, nkv, hd, max_splits) || max_seq > kMaxSplitsFused * kAttnSplitFused)
        return hipErrorInvalidValue;
    if (rec && (vdt != kQ8K || B > 16)) return hipErrorInvalidValue;
    AttnArgs A;
    A.qkv = qkv;
    A.qkv_n = qkv_n;
    A.nh = nh;
    A.nkv = nkv;
    A.qn = qn;
    A.kn = kn;
    A.eps = eps;
    A.inv_hd = (float)(1.0 / (double)hd);
    A.scale = (float)(1.0 / sqrt((double)hd));
    A.interleaved = interleaved;
    A.cos_t = cos_t;
    A.sin_t = sin_t;
    A.len = len;
    A.kc = kc;
    A.vc = vc;
    A.kv_stream_stride = kv_stream_stride;
    A.max_seq = max_seq;
    A.part = part;
    A.max_splits = max_splits;
    A.counter = counter;
    A.cstride = counter_stride();
    A.act = act;
    A.ctx_out = ctx_out;
    A.q_out = q_out;
    A.ready = nullptr;
    A.ready_copies = 0;
    A.rope_row = nullptr;
    A.pub_off = 0;
    A.rec = rec;
    const int all = (max_seq + kAttnSplitFused - 1) / kAttnSplitFused;  // partial records: max_splits per head
    const dim3 grid(B, nkv, grid_splits > 0 && grid_splits < all ? grid_splits : all);
    const size_t lds = attn_decode_lds(nh, nkv, hd, max_splits);
    void* args[] = {&A};
    return hipLaunchKernel(attn_decode_kernel(vdt, hd, nh / nkv), grid, dim3(kAttnThreads), args, lds, s);
}

// ---- batch-1 decode attention + O projection as one launch ---------------------------
// Workgroups [0, n_attn) are k_attn_decode's (split sp = id / n_kv of head group
// g = id % n_kv), publishing their quantized context slices (attn_emit_context, PUB); the
// rest each own R rows of the O projection (512 threads; k_gemv2_q4k's tile for Q4_K,
// k_gemv2_q80's tasks for Q8_0 / Q4_0): they issue their weight loads and the residual
// load at once, then one thread waits for the n_kv slices (a bounded poll of the ready
// counter), the context row is staged into LDS with agent-coherent loads, and the tile's
// products and in-order fold follow -- the same arithmetic as the separate launches, bit
// for bit.  The wait cannot block the attention: the workgroups of a launch are
// dispatched in id order, so every attention workgroup holds its CU before the first
// projection workgroup does, and it never waits for one.  Should the poll run out anyway
// (about a second), the tile's outputs are NaN rather than stale.
struct WoArgs {
    const void* hdr;   // Q4_K block headers (16 B per block) or Q8_0 / Q4_0 f16 scales, [n][nb]
    const uint4* qs;   // quants: 128 / 32 / 16 B per block, [n][nb]
    int n, nb, R;      // output rows, blocks per row, rows per workgroup
    int n_attn;        // attention workgroups ahead of the projection's
    float* y;          // the residual stream row [n], updated in place: y = y + ctx . W^T
    unsigned* ready_next;
    unsigned need;  // slices in the context row (n_kv)
};
constexpr int kWoTm = 1;  // task rounds of a Q4_K projection tile: R * nb <= kWoTm * 128
constexpr int kWoPollCap = 1 << 22;
constexpr int kWoQ4K = 0, kWoQ8_0 = 1, kWoQ4_0 = 2;  // the O projection's weight type

// One thread polls the ready counter (bounded), then the context row (act_u4 16-byte
// pieces) is staged into LDS at the coherent level (this XCD's L2 may hold an earlier
// layer's row).  Returns false when the poll ran out.
SXQ_DEV bool wo_wait_stage(const AttnArgs& A, const WoArgs& W, int t, uint4* lds, int act_u4, bool* flag) {
    if (threadIdx.x == 0) {
        const unsigned* ready = A.ready + (t % A.ready_copies) * A.cstride;  // this tile's copy
        int it = 0;
        while (__hip_atomic_load(ready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < W.need && it < kWoPollCap) {
            __builtin_amdgcn_s_sleep(1);
            ++it;
        }
        *flag = it < kWoPollCap;
    }
    lds_barrier();  // (also: every thread's first-pass fold has read the products)
    const bool ok = *flag;
    const __amdgpu_buffer_rsrc_t ar = coherent_rsrc(A.act, (uint32_t)act_u4 * 16);
    for (int i = threadIdx.x; i < act_u4; i += kAttnThreads) {
        const float4 x = load16_coherent(ar, (uint32_t)i * 16);
        lds[i] = make_uint4(__float_as_uint(x.x), __float_as_uint(x.y), __float_as_uint(x.z), __float_as_uint(x.w));
    }
    lds_barrier();
    return ok;
}

// SPEC: the attention splits issue their loads before the length returns (A.rope_row).
template <int WT, int HD, int GC, int TM, bool SPEC>
__global__ __launch_bounds__(kAttnThreads) __attribute__((amdgpu_waves_per_eu(6, 8))) void k_attn_wo_decode(AttnArgs A,
                                                                                                          WoArgs W) {
    constexpr int NT = kAttnThreads;
    constexpr int VDT = WT == kWoQ4K ? kQ8K : kQ8_0;
    extern __shared__ float4 smem4[];
    __shared__ bool flag;
    const int id = blockIdx.x;
    if (id < W.n_attn) {
        attn_decode_body<VDT, HD, NT, GC, true, SPEC>(A, 0, id % A.nkv, id / A.nkv, (float*)smem4, &flag);
        return;
    }
    uint4* lds = (uint4*)smem4;
    const int tid = threadIdx.x, t = id - W.n_attn;
    const int nb = W.nb, row0 = t * W.R, rows = min(W.R, W.n - row0), tasks = rows * nb;
    if constexpr (WT == kWoQ4K) {
        uint4 q[TM][kQ4kCpl], h[TM];
        q4k_tile_load<NT, TM>((const uint4*)W.hdr, W.qs, (uint32_t)row0 * (uint32_t)nb, tasks, q, h);
        const int r = tid >> 3, l = tid & 7;
        const float res = W.y[row0 + min(r, rows - 1)];  // clamped, unconditional; used by lane class 0 of rows < rows
        issue_point();
        if (tid < A.ready_copies && t == 0)
            __hip_atomic_store(W.ready_next + tid * A.cstride, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int act_u4 = nb * (int)(sizeof(ActQ8K) / 16);
        float* pr = (float*)(lds + act_u4);  // product chains [R + 1][9][CS]
        bool ok = true;
        float v = 0.0f;
        // Two passes over the same code: the first, on whatever the LDS holds, runs while
        // the attention does and leaves the products' and the fold's instructions in the
        // instruction cache (their first fetch would otherwise sit on the critical path);
        // the second waits for the context and computes the result.
#pragma nounroll
        for (int pass = 0; pass < 2; ++pass) {
            if (pass == 1) ok = wo_wait_stage(A, W, t, lds, act_u4, &flag);
            q4k_tile_products<1, NT, TM>(q, h, (const ActQ8K*)lds, nb, 1, rows, W.R, pr);
            __syncthreads();
            v = q4k_tile_fold(pr, nb, W.R, 0, rows);
        }
        if (r < rows && l == 0) W.y[row0 + r] = ok ? res + v : __builtin_nanf("");
    } else {
        // k_gemv2_q80's tasks for one activation row: a lane pair per Q8_0 task, one lane
        // per Q4_0 task; products ((float)isum * d_w) * d_a in task slots, each row's
        // blocks then added in order by one thread
        constexpr bool Q4 = WT == kWoQ4_0;
        constexpr int LPT = Q4 ? 1 : 2, TPI = NT / LPT, QU4 = Q4 ? 1 : 2;
        const uint16_t* dw16 = (const uint16_t*)W.hdr;
        const int half = Q4 ? 0 : (tid & 1), slot = tid / LPT;
        const int64_t base = (int64_t)row0 * nb;
        uint4 w[TM];
        float dw[TM];
#pragma unroll
        for (int u = 0; u < TM; ++u) {
            const int tt = min(u * TPI + slot, tasks - 1);
            w[u] = W.qs[(base + tt) * QU4 + half];
            dw[u] = h2f(dw16[base + tt]);
        }
        const float res = W.y[row0 + min(tid, rows - 1)];  // clamped, unconditional; used by threads < rows
        issue_point();
        if (tid < A.ready_copies && t == 0)
            __hip_atomic_store(W.ready_next + tid * A.cstride, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int act_u4 = nb * (int)(sizeof(ActQ8_0) / 16);
        const ActQ8_0* la = (const ActQ8_0*)lds;
        float* pr = (float*)(lds + act_u4);  // product slots [TM * TPI]
        bool ok = true;
        float v = 0.0f;
#pragma nounroll
        for (int pass = 0; pass < 2; ++pass) {  // as for Q4_K: a warm-up pass, then the real one
            if (pass == 1) ok = wo_wait_stage(A, W, t, lds, act_u4, &flag);
#pragma unroll
            for (int u = 0; u < TM; ++u) {
                if (u * TPI >= tasks) break;
                const ActQ8_0& a = la[(u * TPI + slot) % nb];
                int isum;
                if (Q4) {
                    const uint4 A0 = ((const uint4*)a.qs)[0], A1 = ((const uint4*)a.qs)[1];
                    const uint32_t wd[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
                    const int Alo[4] = {(int)A0.x, (int)A0.y, (int)A0.z, (int)A0.w};
                    const int Ahi[4] = {(int)A1.x, (int)A1.y, (int)A1.z, (int)A1.w};
                    isum = -8 * a.asum;
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        isum = __builtin_amdgcn_sdot4((int)(wd[k] & 0x0F0F0F0Fu), Alo[k], isum, false);
                        isum = __builtin_amdgcn_sdot4((int)((wd[k] >> 4) & 0x0F0F0F0Fu), Ahi[k], isum, false);
                    }
                } else {
                    const uint4 Av = ((const uint4*)a.qs)[half];
                    int sd = __builtin_amdgcn_sdot4((int)w[u].x, (int)Av.x, 0, false);
                    sd = __builtin_amdgcn_sdot4((int)w[u].y, (int)Av.y, sd, false);
                    sd = __builtin_amdgcn_sdot4((int)w[u].z, (int)Av.z, sd, false);
                    sd = __builtin_amdgcn_sdot4((int)w[u].w, (int)Av.w, sd, false);
                    isum = sd + dpp_xor1(sd);
                }
                pr[u * TPI + slot] = ((float)isum * dw[u]) * a.d;
            }
            __syncthreads();
            if (tid < rows) {
                const float* p = pr + tid * nb;
                float sumf = 0.0f;
                for (int b = 0; b < nb; ++b) sumf += p[b];
                v = sumf;
            }
            __syncthreads();  // the next pass rewrites the slots
        }
        if (tid < rows) W.y[row0 + tid] = ok ? res + v : __builtin_nanf("");
    }
}

static int wo_rows(int nb) { return max(1, min(kAttnThreads / 8, kWoTm * (kAttnThreads / kQ4kLanes) / nb)); }
// Q8_0 / Q4_0 tiles: the fewest task rounds (1, 2 or 4) that keep the projection within
// 320 workgroups; R rows of nb tasks each fill them.
static int wo_tasks_per_round(int dtype) { return dtype == kQ4_0 ? kAttnThreads : kAttnThreads / 2; }
static int wo_tm_q80(int n, int nb, int dtype) {
    for (int tm : {1, 2, 4}) {
        const int R = min(64, tm * wo_tasks_per_round(dtype) / nb);
        if (R >= 1 && (n + R - 1) / R <= 320) return tm;
    }
    return 4;
}
static int wo_rows_q80(int n, int nb, int dtype) {
    return max(1, min(64, wo_tm_q80(n, nb, dtype) * wo_tasks_per_round(dtype) / nb));
}
static size_t wo_pub_off(int nh, int nkv, int hd, int max_splits) {
    return (attn_decode_lds(nh, nkv, hd, max_splits) + 15) & ~(size_t)15;
}
static size_t attn_wo_lds(int nh, int nkv, int hd, int max_splits, const QWeight& wo) {
    const size_t G = nh / nkv, nb = (size_t)wo.nb;
    size_t attn = wo_pub_off(nh, nkv, hd, max_splits), proj;
    if (wo.dtype == kQ4K) {
        attn += (G * hd / 256) * sizeof(ActQ8K);
        proj = nb * sizeof(ActQ8K) + (size_t)(wo_rows((int)nb) + 1) * 9 * q4k_chain_stride((int)nb) * sizeof(float);
    } else {
        attn += (G * hd / 32) * sizeof(ActQ8_0);
        proj = nb * sizeof(ActQ8_0) +
               (size_t)wo_tm_q80((int)wo.n, (int)nb, wo.dtype) * wo_tasks_per_round(wo.dtype) * sizeof(float);
    }
    return attn > proj ? attn : proj;
}
template <int WT, int TM, bool SPEC>
static const void* attn_wo_kernel_g(int hd, int G) {
    if (hd == 128)
        return G == 4 ? (const void*)k_attn_wo_decode<WT, 128, 4, TM, SPEC> : (const void*)k_attn_wo_decode<WT, 128, 0, TM, SPEC>;
    return G == 7 ? (const void*)k_attn_wo_decode<WT, 64, 7, TM, SPEC> : (const void*)k_attn_wo_decode<WT, 64, 0, TM, SPEC>;
}
template <int WT, bool SPEC>
static const void* attn_wo_kernel_tm(int hd, int G, int tm) {
    if (tm == 4) return attn_wo_kernel_g<WT, 4, SPEC>(hd, G);
    if (tm == 2) return attn_wo_kernel_g<WT, 2, SPEC>(hd, G);
    return attn_wo_kernel_g<WT, 1, SPEC>(hd, G);
}
template <bool SPEC>
static const void* attn_wo_kernel_s(int hd, int G, const QWeight& wo) {
    if (wo.dtype == kQ4K) {
        if (hd == 128)
            return G == 4 ? (const void*)k_attn_wo_decode<kWoQ4K, 128, 4, kWoTm, SPEC>
                          : (const void*)k_attn_wo_decode<kWoQ4K, 128, 0, kWoTm, SPEC>;
        return (const void*)k_attn_wo_decode<kWoQ4K, 64, 0, kWoTm, SPEC>;
    }
    const int tm = wo_tm_q80((int)wo.n, (int)wo.nb, wo.dtype);
    return wo.dtype == kQ8_0 ? attn_wo_kernel_tm<kWoQ8_0, SPEC>(hd, G, tm) : attn_wo_kernel_tm<kWoQ4_0, SPEC>(hd, G, tm);
}
static const void* attn_wo_kernel(int hd, int G, const QWeight& wo, bool spec) {
    return spec ? attn_wo_kernel_s<true>(hd, G, wo) : attn_wo_kernel_s<false>(hd, G, wo);
}

bool attn_wo_decode_fits(int vdt, int nh, int nkv, int hd, int max_splits, const QWeight& wo, int dim) {
    if (!attn_decode_fits(vdt, nh, nkv, hd, max_splits) || wo.k != (int64_t)nh * hd || wo.n != dim || wo.nb < 1)
        return false;
    if (vdt == kQ8K && wo.dtype == kQ4K) {
        if (wo.nb > kWoTm * (kAttnThreads / kQ4kLanes)) return false;
    } else if (vdt == kQ8_0 && (wo.dtype == kQ8_0 || wo.dtype == kQ4_0)) {
        if (wo.nb > 4 * wo_tasks_per_round(wo.dtype)) return false;
    } else {
        return false;
    }
    return attn_wo_lds(nh, nkv, hd, max_splits, wo) <= 160 * 1024;
}

hipError_t attn_wo_decode_prepare(int vdt, int nh, int nkv, int hd, int max_splits, const QWeight& wo) {
    (void)vdt;
    const int lds = (int)attn_wo_lds(nh, nkv, hd, max_splits, wo);
    hipError_t e = hipFuncSetAttribute(attn_wo_kernel(hd, nh / nkv, wo, false), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e == hipSuccess)
        e = hipFuncSetAttribute(attn_wo_kernel(hd, nh / nkv, wo, true), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    return e;
}

hipError_t launch_attention_wo_decode(int vdt, const float* qkv, int qkv_n, int nh, int nkv, int hd, const float* qn,
                                      const float* kn, float eps, int interleaved, const float* cos_t,
                                      const float* sin_t, const int* len, float* kc, float* vc, int max_seq,
                                      int max_splits, float* part, unsigned* counter, uint8_t* act, const QWeight& wo,
                                      float* y, unsigned* ready, unsigned* ready_next, float* ctx_out, float* q_out,
                                      hipStream_t s, int grid_splits, const float* rope_row) {
    if (!attn_wo_decode_fits(vdt, nh, nkv, hd, max_splits, wo, (int)wo.n) ||
        max_seq > kMaxSplitsFused * kAttnSplitFused || ready == ready_next)
        return hipErrorInvalidValue;
    AttnArgs A;
    A.qkv = qkv;
    A.qkv_n = qkv_n;
    A.nh = nh;
    A.nkv = nkv;
    A.qn = qn;
    A.kn = kn;
    A.eps = eps;
    A.inv_hd = (float)(1.0 / (double)hd);
    A.scale = (float)(1.0 / sqrt((double)hd));
    A.interleaved = interleaved;
    A.cos_t = cos_t;
    A.sin_t = sin_t;
    A.len = len;
    A.kc = kc;
    A.vc = vc;
    A.kv_stream_stride = (int64_t)nkv * max_seq * hd;  // one stream: unused
    A.max_seq = max_seq;
    A.part = part;
    A.max_splits = max_splits;
    A.counter = counter;
    A.cstride = counter_stride();
    A.act = act;
    A.ctx_out = ctx_out;
    A.q_out = q_out;
    A.ready = ready;
    A.ready_copies = ready_copies();
    A.rope_row = rope_row;
    A.pub_off = (uint32_t)wo_pub_off(nh, nkv, hd, max_splits);
    A.rec = nullptr;
    WoArgs W;
    W.hdr = wo.hdr;
    W.qs = (const uint4*)wo.qs;
    W.n = (int)wo.n;
    W.nb = (int)wo.nb;
    W.R = wo.dtype == kQ4K ? wo_rows(W.nb) : wo_rows_q80(W.n, W.nb, wo.dtype);
    const int all = (max_seq + kAttnSplitFused - 1) / kAttnSplitFused;
    W.n_attn = nkv * (grid_splits > 0 && grid_splits < all ? grid_splits : all);
    W.y = y;
    W.ready_next = ready_next;
    W.need = (unsigned)nkv;
    const int n_wo = (W.n + W.R - 1) / W.R;
    const size_t lds = attn_wo_lds(nh, nkv, hd, max_splits, wo);
    void* args[] = {&A, &W};
    return hipLaunchKernel(attn_wo_kernel(hd, nh / nkv, wo, rope_row != nullptr), dim3(W.n_attn + n_wo), dim3(kAttnThreads),
                           args, lds, s);
}

hipError_t launch_silu_mul_quant(int vdt, const float* gu, int B, int I, uint8_t* act, float* act_f32, hipStream_t s,
                                 MmaRec* rec) {
    if (rec && (vdt != kQ8K || B > 16)) return hipErrorInvalidValue;
    const dim3 grid(B, (I + 255) / 256);
    if (vdt == kQ8K) hipLaunchKernelGGL((k_silu_mul_quant<kQ8K>), grid, dim3(64), 0, s, gu, I, act, act_f32, rec);
    else hipLaunchKernelGGL((k_silu_mul_quant<kQ8_0>), grid, dim3(64), 0, s, gu, I, act, act_f32, rec);
    return hipGetLastError();
}

hipError_t launch_embed_mcf(const int* ids, int ids_per, int B, const float* table, int64_t table_rows,
                            const QWeight& w, int dim, const float* cb, int n_cb, int cb_size, int sem_begin,
                            int sem_end, float* h, hipStream_t s, const RopeRow& rr) {
    if (rr.out && (rr.half < 1 || rr.half > 128 || !rr.len || !rr.cos_t || !rr.sin_t)) return hipErrorInvalidValue;
    const float inv_scale = 1.0f / sqrtf((float)n_cb + 1.0f);
    const int64_t rows = table ? table_rows : w.n;
    hipLaunchKernelGGL(k_embed_mcf, dim3(B, (dim + 255) / 256), dim3(256), 0, s, ids, ids_per, table, rows, w, dim, cb,
                       n_cb, cb_size, sem_begin, sem_end, inv_scale, h, rr);
    return hipGetLastError();
}

hipError_t launch_embed_dense(const int* ids, int ids_per, int B, const float* table, int rows, int dim, float* h,
                              hipStream_t s, const RopeRow& rr) {
    if (rr.out && (rr.half < 1 || rr.half > 128 || !rr.len || !rr.cos_t || !rr.sin_t)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_embed_dense, dim3(B, (dim + 255) / 256), dim3(256), 0, s, ids, ids_per, table, rows, dim, h,
                       rr);
    return hipGetLastError();
}

hipError_t launch_argmax(const float* logits, int B, int vocab, int* ids, int ids_per, int* out_ids, int* len,
                         float* pval, int* pidx, unsigned* counter, hipStream_t s) {
    hipLaunchKernelGGL(k_argmax, dim3(B, kArgmaxSlices), dim3(256), 0, s, logits, vocab, ids, ids_per, out_ids, len,
                       pval, pidx, counter, counter_stride());
    return hipGetLastError();
}

hipError_t launch_fill_int(int* y, int n, int v, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_fill_int, dim3((n + 255) / 256), dim3(256), 0, s, y, n, v);
    return hipGetLastError();
}

hipError_t launch_fill_value(float* y, int64_t n, float v, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_fill_value, dim3((n + 255) / 256), dim3(256), 0, s, y, n, v);
    return hipGetLastError();
}

}  // namespace sxq
