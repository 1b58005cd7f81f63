// sxq_prefill.hip -- the glue of a prompt (many tokens per stream) through the decoder:
// per-token QK-RMSNorm + RoPE + KV-cache write, and causal GQA attention of the prompt's
// queries over each stream's cache.
//
// Reference: SlowAr::prefill / prefill_batch (crates/syrinx-fish/src/s2/slow_ar.rs:250-256,
// 404-454) and Qwen2Lm::forward_hidden_cached (crates/syrinx-lm/src/cv2/mod.rs:261-286):
// the new tokens sit at positions cache.len() .. cache.len() + t_new, each query attends
// its own stream's keys up to its own position (causal_mask_at, s2/nn.rs:208-218,
// cv2/attention.rs:120-141), scores (q . k) / sqrt(head_dim), softmax in f32.
#include "sxq_attn_dev.h"
#include "sxq_decoder.h"

namespace sxq {

// grid (T, n_heads + 2 * n_kv), one wave per head of token t's fused qkv row: the same
// per-head arithmetic (rope_load / rope_pair) as the fused decode attention, at the
// token's own stream and position (tok[t] = {stream, position}).
template <int HD>
__global__ __launch_bounds__(64) void k_prefill_rope_kv(const float* __restrict__ qkv, int qkv_n, int nh, int nkv,
                                                        const float* __restrict__ qn, const float* __restrict__ kn,
                                                        float eps, float inv_hd, int interleaved,
                                                        const float* __restrict__ cos_t, const float* __restrict__ sin_t,
                                                        const int2* __restrict__ tok, float* __restrict__ qout,
                                                        float* __restrict__ kc, float* __restrict__ vc,
                                                        int64_t kv_stream_stride, int max_seq) {
    const int t = blockIdx.x, hid = blockIdx.y, lane = threadIdx.x;
    const int2 sp = tok[t];
    const int s = sp.x, pos = sp.y;
    const float* src = qkv + (int64_t)t * qkv_n + (int64_t)hid * HD;
    const bool is_q = hid < nh, is_k = !is_q && hid < nh + nkv;
    if (!is_q && !is_k) {  // V: stored as projected
        const int g = hid - nh - nkv;
        float* dst = vc + (int64_t)s * kv_stream_stride + ((int64_t)g * max_seq + pos) * HD;
        for (int d = lane; d < HD; d += 64) dst[d] = src[d];
        return;
    }
    float* dst = is_q ? qout + ((int64_t)t * nh + hid) * HD
                      : kc + (int64_t)s * kv_stream_stride + ((int64_t)(hid - nh) * max_seq + pos) * HD;
    const float* nw = is_q ? qn : kn;
    const RopeIn ri = rope_load<HD>(src, nw, interleaved, cos_t + (int64_t)pos * (HD / 2),
                                    sin_t + (int64_t)pos * (HD / 2), lane);
    rope_store<HD>(rope_pair<HD>(ri, nw != nullptr, eps, inv_hd, lane), interleaved, dst, nullptr, lane);
}

constexpr int kPfRows = 64;  // query rows (tokens x heads of one KV group) per workgroup
constexpr int kPfKeys = 32;  // key positions per LDS block

size_t prefill_attn_lds(int hd) {
    return sizeof(float) * ((size_t)(kPfRows + 2 * kPfKeys) * (hd + 4) + (size_t)kPfRows * (kPfKeys + 1));
}

// One workgroup (256 threads) per (tile, KV group): a tile is up to kPfRows / G
// consecutive prompt tokens of one stream (tile = {stream, first token row t0, count,
// position p0 of token t0}); its rows are r = i * G + hh (token i, query head g * G + hh).
// Keys stream through LDS in blocks of kPfKeys positions (0 .. p0 + count - 1); every row
// keeps an online softmax (running max m, sum l, rescaled accumulator), masking keys past
// its own position.  Thread (r, qd) = (tid / 4, tid % 4) scores keys 8 qd .. 8 qd + 7 of a
// block for row r and accumulates head dims qd * HD/4 .. +HD/4 - 1 of that row.
template <int HD>
__global__ __launch_bounds__(256) void k_prefill_attn(const float* __restrict__ q, const float* __restrict__ kc,
                                                      const float* __restrict__ vc, const int4* __restrict__ tiles,
                                                      int nh, int nkv, int max_seq, int64_t kv_stream_stride,
                                                      float scale, float* __restrict__ ctx) {
    extern __shared__ float4 smem4[];
    constexpr int hdp = HD + 4, DPT = HD / 4;
    const int4 tl = tiles[blockIdx.x];
    const int s = tl.x, t0 = tl.y, cnt = tl.z, p0 = tl.w;
    const int g = blockIdx.y, G = nh / nkv, R = cnt * G;
    float* qs = (float*)smem4;          // [kPfRows][hdp]
    float* kt = qs + kPfRows * hdp;     // [kPfKeys][hdp]
    float* vt = kt + kPfKeys * hdp;     // [kPfKeys][hdp]
    float* pr = vt + kPfKeys * hdp;     // [kPfRows][kPfKeys + 1] probabilities of the block
    const int tid = threadIdx.x, r = tid >> 2, qd = tid & 3;
    const int qrow = nh * HD;  // floats per token row of q and ctx
    for (int e = tid; e < kPfRows * HD; e += 256) {
        const int rr = e / HD, d = e - rr * HD;
        float v = 0.0f;
        if (rr < R) v = q[(int64_t)(t0 + rr / G) * qrow + (g * G + rr % G) * HD + d];
        qs[rr * hdp + d] = v;
    }
    const bool live = r < R;
    const int qpos = live ? p0 + r / G : -1;
    float m = -INFINITY, l = 0.0f, acc[DPT];
#pragma unroll
    for (int i = 0; i < DPT; ++i) acc[i] = 0.0f;
    const int64_t koff = (int64_t)s * kv_stream_stride + (int64_t)g * max_seq * HD;
    const int kend = p0 + cnt;
    for (int j0 = 0; j0 < kend; j0 += kPfKeys) {
        const int nk = min(kPfKeys, kend - j0);
        __syncthreads();  // the previous block's K, V and P are no longer read
        load_kv_tile(kt, vt, kc + koff + (int64_t)j0 * HD, vc + koff + (int64_t)j0 * HD, nk, HD);
        __syncthreads();
        float sc[8];
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) sc[jj] = 0.0f;
        const float* qr = qs + r * hdp;
        for (int d = 0; d < HD; d += 4) {
            const float4 qv = *(const float4*)(qr + d);
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
                const float4 kv = *(const float4*)(kt + (8 * qd + jj) * hdp + d);
                sc[jj] += qv.x * kv.x;
                sc[jj] += qv.y * kv.y;
                sc[jj] += qv.z * kv.z;
                sc[jj] += qv.w * kv.w;
            }
        }
        float bm = -INFINITY;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
            const int j = 8 * qd + jj;
            const bool ok = live && j < nk && j0 + j <= qpos;
            sc[jj] = ok ? sc[jj] * scale + 0.0f : -INFINITY;
            bm = fmaxf(bm, sc[jj]);
        }
        bm = fmaxf(bm, __shfl_xor(bm, 1, 64));
        bm = fmaxf(bm, __shfl_xor(bm, 2, 64));
        const float mn = fmaxf(m, bm);
        const float corr = mn == -INFINITY ? 1.0f : expf(m - mn);
        float ps = 0.0f;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
            const float p = sc[jj] == -INFINITY ? 0.0f : expf(sc[jj] - mn);
            pr[r * (kPfKeys + 1) + 8 * qd + jj] = p;
            ps += p;
        }
        ps += __shfl_xor(ps, 1, 64);
        ps += __shfl_xor(ps, 2, 64);
        l = l * corr + ps;
        m = mn;
        __syncthreads();  // the row's probabilities (written by its four threads) are visible
#pragma unroll
        for (int i = 0; i < DPT; ++i) acc[i] *= corr;
        const float* prow = pr + r * (kPfKeys + 1);
        for (int j = 0; j < nk; ++j) {
            const float p = prow[j];
            const float* vr = vt + j * hdp + qd * DPT;
#pragma unroll
            for (int i = 0; i < DPT; i += 4) {
                const float4 v = *(const float4*)(vr + i);
                acc[i] += p * v.x;
                acc[i + 1] += p * v.y;
                acc[i + 2] += p * v.z;
                acc[i + 3] += p * v.w;
            }
        }
    }
    if (!live) return;
    float* out = ctx + (int64_t)(t0 + r / G) * qrow + (g * G + r % G) * HD + qd * DPT;
#pragma unroll
    for (int i = 0; i < DPT; i += 4)
        *(float4*)(out + i) = make_float4(acc[i] / l, acc[i + 1] / l, acc[i + 2] / l, acc[i + 3] / l);
}

// One thread per token t (and per tile index): stream-major order, stream s's tokens at
// rows base_s .. base_s + counts[s] - 1 and positions lens[s] .. lens[s] + counts[s] - 1.
__global__ __launch_bounds__(256) void k_prefill_tables(PrefillMeta pm, int T, int2* __restrict__ tok,
                                                        int4* __restrict__ tiles, int* __restrict__ last) {
    const int t = blockIdx.x * 256 + threadIdx.x;
    int base = 0, tbase = 0;
    for (int s = 0; s < pm.n; ++s) {
        const int c = pm.counts[s], nt = (c + pm.tile_tokens - 1) / pm.tile_tokens;
        if (t >= base && t < base + c) tok[t] = make_int2(s, pm.lens[s] + (t - base));
        if (t >= tbase && t < tbase + nt) {
            const int i0 = (t - tbase) * pm.tile_tokens;
            tiles[t] = make_int4(s, base + i0, min(pm.tile_tokens, c - i0), pm.lens[s] + i0);
        }
        if (t == 0) last[s] = c > 0 ? base + c - 1 : -1;
        base += c;
        tbase += nt;
    }
    (void)T;
}

__global__ void k_prefill_advance(PrefillMeta pm, int* __restrict__ len) {
    const int s = threadIdx.x;
    if (s < pm.n) len[s] += pm.counts[s];
}

hipError_t launch_prefill_tables(const PrefillMeta& pm, int T, int* tok, int* tiles, int* last, hipStream_t s) {
    const int n_items = T + pm.n;  // tokens, and at most T + n tiles
    hipLaunchKernelGGL(k_prefill_tables, dim3((n_items + 255) / 256), dim3(256), 0, s, pm, T, (int2*)tok, (int4*)tiles,
                       last);
    return hipGetLastError();
}

hipError_t launch_prefill_advance(const PrefillMeta& pm, int* len, hipStream_t s) {
    hipLaunchKernelGGL(k_prefill_advance, dim3(1), dim3(64), 0, s, pm, len);
    return hipGetLastError();
}

// rows[i] = src[idx[i]] for n rows of `cols` floats (each stream's last prompt row).
__global__ __launch_bounds__(256) void k_gather_rows(const float* __restrict__ src, const int* __restrict__ idx,
                                                     int cols, float* __restrict__ dst) {
    const int i = blockIdx.x;
    const float* a = src + (int64_t)idx[i] * cols;
    for (int c = threadIdx.x; c < cols; c += 256) dst[(int64_t)i * cols + c] = a[c];
}

hipError_t launch_prefill_rope_kv(const float* qkv, int T, int qkv_n, int nh, int nkv, int hd, const float* qn,
                                  const float* kn, float eps, int interleaved, const float* cos_t, const float* sin_t,
                                  const int* tok, float* qout, float* kc, float* vc, int64_t kv_stream_stride,
                                  int max_seq, hipStream_t s) {
    if (hd != 64 && hd != 128) return hipErrorInvalidValue;
    const dim3 grid(T, nh + 2 * nkv);
    if (hd == 128)
        hipLaunchKernelGGL(k_prefill_rope_kv<128>, grid, dim3(64), 0, s, qkv, qkv_n, nh, nkv, qn, kn, eps,
                           1.0f / (float)hd, interleaved, cos_t, sin_t, (const int2*)tok, qout, kc, vc,
                           kv_stream_stride, max_seq);
    else
        hipLaunchKernelGGL(k_prefill_rope_kv<64>, grid, dim3(64), 0, s, qkv, qkv_n, nh, nkv, qn, kn, eps,
                           1.0f / (float)hd, interleaved, cos_t, sin_t, (const int2*)tok, qout, kc, vc,
                           kv_stream_stride, max_seq);
    return hipGetLastError();
}

bool prefill_attn_supported(int nh, int nkv, int hd) { return (hd == 64 || hd == 128) && nh / nkv <= kPfRows; }
int prefill_tile_tokens(int nh, int nkv) { return kPfRows / (nh / nkv); }

hipError_t launch_prefill_attn(const float* q, const float* kc, const float* vc, const int* tiles, int n_tiles, int nh,
                               int nkv, int hd, int max_seq, int64_t kv_stream_stride, float* ctx, hipStream_t s) {
    if (!prefill_attn_supported(nh, nkv, hd)) return hipErrorInvalidValue;
    if (n_tiles == 0) return hipSuccess;
    const size_t lds = prefill_attn_lds(hd);
    const float scale = (float)(1.0 / sqrt((double)hd));
    if (hd == 128) {
        static const hipError_t a = hipFuncSetAttribute((const void*)k_prefill_attn<128>,
                                                        hipFuncAttributeMaxDynamicSharedMemorySize, (int)prefill_attn_lds(128));
        if (a != hipSuccess) return a;
        hipLaunchKernelGGL(k_prefill_attn<128>, dim3(n_tiles, nkv), dim3(256), lds, s, q, kc, vc, (const int4*)tiles,
                           nh, nkv, max_seq, kv_stream_stride, scale, ctx);
    } else {
        static const hipError_t a = hipFuncSetAttribute((const void*)k_prefill_attn<64>,
                                                        hipFuncAttributeMaxDynamicSharedMemorySize, (int)prefill_attn_lds(64));
        if (a != hipSuccess) return a;
        hipLaunchKernelGGL(k_prefill_attn<64>, dim3(n_tiles, nkv), dim3(256), lds, s, q, kc, vc, (const int4*)tiles,
                           nh, nkv, max_seq, kv_stream_stride, scale, ctx);
    }
    return hipGetLastError();
}

hipError_t launch_gather_rows(const float* src, const int* idx, int n, int cols, float* dst, hipStream_t s) {
    hipLaunchKernelGGL(k_gather_rows, dim3(n), dim3(256), 0, s, src, idx, cols, dst);
    return hipGetLastError();
}

}  // namespace sxq
