// sxq_gemm.hip -- prefill (many-row) QMatMul over Q4_K weights on CDNA4 MFMA.
//
// For m rows well beyond the decode GEMV (QMatMul::forward with M = prompt length; the
// reference calls it at crates/syrinx-lm/src/cv2/mod.rs:197 and, for the Fish slow AR
// prefill, through Weights::linear at crates/syrinx-fish/src/s2/nn.rs:61-74) the
// contraction is a real GEMM.  Weight tiles are dequantized into LDS exactly as Candle's
// to_float computes them in f32, (d*sc)*q - dmin*m, then rounded once to f16; the
// activations are rounded to f16; v_mfma_f32_32x32x16_f16 accumulates in f32.  (f16
// rather than bf16: the same MFMA rate on gfx950, with 3 more mantissa bits.)  The
// result therefore differs from Candle's integer Q8_K vec-dot by the f16 rounding of
// both operands, bounded by 2^-10 * sum_k |w_k x_k| per output.
//
// K order.  Inside each 256-element block the GEMM runs over K in the byte order of the
// Q4_K device layout (sxq_common.h): byte B = 16*l + 4*c + t of the class-major qs holds
// elements 64c + l + 8t (low nibble) and 64c + 32 + l + 8t (high nibble), which go to
// GEMM positions 2B and 2B + 1.  So one 16-byte weight segment dequantizes to 32
// consecutive f16 in LDS.  The activations are converted to f16 with the same
// permutation (k_x_to_f16_perm); a dot product does not depend on the order of its
// terms beyond rounding.
#include <stdlib.h>

#include "sxq_kernels.h"

namespace sxq {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

// GEMM position p (0..255) inside a block -> element index of the canonical order.
SXQ_HD int q4k_perm_elem(int p) {
    const int B = p >> 1, h = p & 1;
    const int l = B >> 4, c = (B >> 2) & 3, t = B & 3;
    return 64 * c + 32 * h + l + 8 * t;
}

// x f32 [m][k] (row stride ldx) -> xh f16 [m][k] with every 256-block permuted to the
// GEMM K order: xh[r][256b + p] = f16(x[r][256b + q4k_perm_elem(p)]).
__global__ __launch_bounds__(256) void k_x_to_f16_perm(const float* __restrict__ x, int64_t ldx, int m, int k,
                                                       _Float16* __restrict__ xh) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)m * k) return;
    const int64_t r = i / k;
    const int col = (int)(i - r * k);
    const int blk = col >> 8, p = col & 255;
    xh[i] = (_Float16)x[r * ldx + (blk << 8) + q4k_perm_elem(p)];
}

constexpr int kGemmBM = 128, kGemmBN = 128, kGemmBK = 256;
constexpr int kGemmLd = kGemmBK + 8;  // LDS row stride in halfs: 16 B of padding against bank conflicts

size_t gemm_q4k_lds() { return 2 * (size_t)kGemmBM * kGemmLd * sizeof(_Float16); }

// y[m][n] = x[m] . W[n] (+ bias[n], then res[m][n] + that), W Q4_K [n][k] in the device
// layout, xh from k_x_to_f16_perm.  Grid (ceil(N/128), ceil(M/128)), 256 threads: wave w
// owns the 64 x 64 sub-tile (w/2, w%2) as 2 x 2 MFMA tiles of 32 x 32.
__global__ __launch_bounds__(256) void k_gemm_q4k(const _Float16* __restrict__ xh, int M, int K,
                                                  const uint4* __restrict__ hdr, const uint4* __restrict__ qs, int N,
                                                  float* __restrict__ y, int64_t ldy, const float* __restrict__ bias,
                                                  const float* res, int64_t ldr) {
    extern __shared__ uint4 lds[];
    _Float16* As = (_Float16*)lds;              // [BM][kGemmLd] activations
    _Float16* Bs = As + kGemmBM * kGemmLd;      // [BN][kGemmLd] dequantized weights
    const int n0 = blockIdx.x * kGemmBN, m0 = blockIdx.y * kGemmBM;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int nb = K / 256;
    floatx16 acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[a][b][i] = 0.0f;

    for (int blk = 0; blk < nb; ++blk) {
        // activations: 128 rows x 32 uint4 (8 halfs each) = 16 uint4 per thread
        uint4 av[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int idx = j * 256 + tid, r = idx >> 5, c = idx & 31;
            const int row = min(m0 + r, M - 1);  // rows past M load row M-1; never stored
            av[j] = ((const uint4*)(xh + (int64_t)row * K + blk * 256))[c];
        }
        // weights: 128 rows x 8 segments of 16 B = 4 segments per thread
        uint4 wq[4], wh[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int idx = j * 256 + tid, r = idx >> 3, l = idx & 7;
            const int64_t b = (int64_t)min(n0 + r, N - 1) * nb + blk;  // rows past N: never stored
            wq[j] = qs[b * 8 + l];
            wh[j] = hdr[b];
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int idx = j * 256 + tid, r = idx >> 5, c = idx & 31;
            *(uint4*)(As + r * kGemmLd + c * 8) = av[j];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int idx = j * 256 + tid, r = idx >> 3, l = idx & 7;
            const uint4 h = wh[j];
            const float d = f16_bits_to_f32((uint16_t)(h.x & 0xFFFF)), dmin = f16_bits_to_f32((uint16_t)(h.x >> 16));
            const uint8_t* sc = (const uint8_t*)&h + 4;  // scales[12]
            const uint32_t qd[4] = {wq[j].x, wq[j].y, wq[j].z, wq[j].w};
            _Float16 out[32];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                // sub-blocks 2c (low nibbles) and 2c + 1 (high nibbles): get_scale_min_k4
                float s[2], mn[2];
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const int jb = 2 * c + hh;
                    int scv, mv;
                    if (jb < 4) {
                        scv = sc[jb] & 63;
                        mv = sc[jb + 4] & 63;
                    } else {
                        scv = (sc[jb + 4] & 0xF) | ((sc[jb - 4] >> 6) << 4);
                        mv = (sc[jb + 4] >> 4) | ((sc[jb] >> 6) << 4);
                    }
                    s[hh] = d * (float)scv;
                    mn[hh] = dmin * (float)mv;
                }
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const uint32_t byte = (qd[c] >> (8 * t)) & 0xFF;
                    out[8 * c + 2 * t] = (_Float16)(s[0] * (float)(byte & 0xF) - mn[0]);
                    out[8 * c + 2 * t + 1] = (_Float16)(s[1] * (float)(byte >> 4) - mn[1]);
                }
            }
            uint4* dst = (uint4*)(Bs + r * kGemmLd + 32 * l);
#pragma unroll
            for (int v = 0; v < 4; ++v) dst[v] = *(const uint4*)&out[8 * v];
        }
        __syncthreads();
#pragma unroll 4
        for (int kk = 0; kk < kGemmBK; kk += 16) {
            half8 a[2], b[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                a[t] = *(const half8*)(As + (wm + 32 * t + (lane & 31)) * kGemmLd + kk + 8 * (lane >> 5));
                b[t] = *(const half8*)(Bs + (wn + 32 * t + (lane & 31)) * kGemmLd + kk + 8 * (lane >> 5));
            }
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int nt = 0; nt < 2; ++nt)
                    acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[mt], b[nt], acc[mt][nt], 0, 0, 0);
        }
        __syncthreads();
    }
    // D layout: acc[i] = D[8*(i/4) + 4*(lane/32) + i%4][lane%32]
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            const int col = n0 + wn + 32 * nt + (lane & 31);
            if (col >= N) continue;
            const float bv = bias ? bias[col] : 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int row = m0 + wm + 32 * mt + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
                if (row < M) {
                    float v = acc[mt][nt][i];
                    if (bias) v = v + bv;
                    if (res) v = res[(int64_t)row * ldr + col] + v;
                    y[(int64_t)row * ldy + col] = v;
                }
            }
        }
}

hipError_t launch_x_to_f16_perm(const float* x, int64_t ldx, int m, int k, void* xh, hipStream_t s) {
    const int64_t total = (int64_t)m * k;
    hipLaunchKernelGGL(k_x_to_f16_perm, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, x, ldx, m, k,
                       (_Float16*)xh);
    return hipGetLastError();
}

hipError_t launch_gemm_q4k(const QWeight& w, const void* xh, int m, float* y, int64_t ldy, const float* bias,
                           const float* res, int64_t ldr, hipStream_t s) {
    if (w.dtype != kQ4K) return hipErrorInvalidValue;
    static const hipError_t attr = hipFuncSetAttribute((const void*)k_gemm_q4k,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)gemm_q4k_lds());
    if (attr != hipSuccess) return attr;
    const dim3 grid((unsigned)((w.n + kGemmBN - 1) / kGemmBN), (unsigned)((m + kGemmBM - 1) / kGemmBM));
    hipLaunchKernelGGL(k_gemm_q4k, grid, dim3(256), gemm_q4k_lds(), s, (const _Float16*)xh, m, (int)w.k,
                       (const uint4*)w.hdr, (const uint4*)w.qs, (int)w.n, y, ldy, bias, res, ldr);
    return hipGetLastError();
}

}  // namespace sxq
