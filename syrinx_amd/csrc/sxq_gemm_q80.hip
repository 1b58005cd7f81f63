// sxq_gemm_q80.hip -- many-row QMatMul over Q8_0 / Q4_0 weights on the int8 matrix cores,
// bit-identical to Candle's vec-dot.
//
// A prompt's projections (QMatMul::forward with M = prompt rows; the reference calls it at
// crates/syrinx-lm/src/cv2/mod.rs:197, whose weights load as Q4_0 at
// crates/syrinx-lm/src/cv2/load.rs:101-104) are a GEMM.  Candle computes every output as
// sum over blocks b of ((f32)S_b * d_w) * d_a, where S_b is the integer dot of one
// 32-element block of the weight row (int8 Q8_0 quants, or Q4_0 nibbles minus 8) with the
// Q8_0-quantized activation row, added block after block in f32.  One
// v_mfma_i32_32x32x32_i8 is exactly that integer dot for a 32 x 32 tile of (row, weight
// row) pairs over one block: its K depth is one block, and integer sums are exact in any
// order.  Each lane then folds its 16 results into its f32 sums in block order with
// Candle's two multiplies and one add, so the outputs are Candle's bits at every row
// count, unlike an f16 GEMM (which rounds both operands).  The float fold is 4 VALU
// instructions per output per block against 1/16 of an MFMA, so the kernel is bound by
// VALU issue, not by the matrix cores.
#include "sxq_kernels.h"

namespace sxq {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kQBM = 64;   // activation rows per workgroup tile
constexpr int kQBN = 128;  // weight rows per workgroup tile
constexpr int kQKC = 16;   // blocks whose activation scales are staged in LDS at a time

// The 16 weight bytes lane half h multiplies with activation elements 16h .. 16h+15 of
// block b: Q8_0 quants as stored; Q4_0 element j is the low nibble of byte j and element
// j + 16 the high nibble, as a signed int8 (q - 8): per byte (q + 0x78) ^ 0x80 (q <= 15,
// so the add never carries into the next byte).
template <bool Q4>
SXQ_DEV v4i weight_frag(const uint8_t* row, int b, int h) {
    if (!Q4) return *(const v4i*)(row + (size_t)b * 32 + 16 * h);
    const v4i w = *(const v4i*)(row + (size_t)b * 16);
    v4i r;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const uint32_t q = (h ? ((uint32_t)w[t] >> 4) : (uint32_t)w[t]) & 0x0F0F0F0Fu;
        r[t] = (int)((q + 0x78787878u) ^ 0x80808080u);
    }
    return r;
}

// y[m][n] = sum_b ((f32)S_b[m][n] * d_w[n][b]) * d_a[m][b] (+ bias[n], then res[m][n] + that).
// act: the Q8_0 activation blocks [M][nb] (ActQ8_0: quants, f32 d).  Weight device layout:
// wd[n * nb + b] f16 scales, wqs the quants (32 B per Q8_0 block, 16 B per Q4_0 block).
// One workgroup of 256 threads per 64 x 128 tile; wave w covers rows 32 (w & 1) .. +31 and
// weight rows 64 (w >> 1) .. +63 as two 32 x 32 MFMA tiles.  Lane (l, h) of a tile: A row l
// and B weight row l, elements 16h .. 16h+15 of the block; result i of the D layout is row
// 8 (i / 4) + 4 h + i % 4, weight row l.  Workgroups are numbered so that every row tile of
// one weight tile lands on the same XCD (id mod 8), whose L2 then serves its re-reads.
template <bool Q4>
__global__ __launch_bounds__(256) void k_gemm_q80(const ActQ8_0* __restrict__ act, int M, int nb,
                                                  const uint16_t* __restrict__ wd, const uint8_t* __restrict__ wqs,
                                                  int N, int tiles_m, int tiles_n, float* __restrict__ y, int64_t ldy,
                                                  const float* __restrict__ bias, const float* res, int64_t ldr) {
    __shared__ float4 sda4[kQKC][kQBM / 4];  // activation scales of the chunk, [block][row]
    const int id = blockIdx.x;
    const int xcd = id & 7, slot = id >> 3;
    const int nt = (slot / tiles_m) * 8 + xcd, mt = slot % tiles_m;
    if (nt >= tiles_n) return;  // uniform: padding of the weight tiles to a multiple of 8
    const int m0 = mt * kQBM, n0 = nt * kQBN;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;
    const int l31 = lane & 31, h = lane >> 5;
    constexpr int qsb = Q4 ? 16 : 32;
    // Loads use clamped rows (results past M or N are never stored).
    const ActQ8_0* arow = act + (int64_t)min(m0 + 32 * wm + l31, M - 1) * nb;
    const uint8_t* brow[2];
    const uint16_t* drow[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int n = min(n0 + 64 * wn + 32 * j + l31, N - 1);
        brow[j] = wqs + (int64_t)n * nb * qsb;
        drow[j] = wd + (int64_t)n * nb;
    }
    float acc[2][16];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[j][i] = 0.0f;
    const v16i zero = {};
    const float* sda = (const float*)sda4;

    for (int c0 = 0; c0 < nb; c0 += kQKC) {
        const int kc = min(kQKC, nb - c0);
        __syncthreads();  // the previous chunk's scale reads are done
        for (int e = tid; e < kQKC * kQBM; e += 256) {
            const int kb = e / kQBM, r = e % kQBM, m = m0 + r;
            ((float*)sda4)[e] = (kb < kc && m < M) ? act[(int64_t)m * nb + c0 + kb].d : 0.0f;
        }
        __syncthreads();
        // fragments of the chunk's first block; each iteration loads the next one ahead
        v4i a = *(const v4i*)((const int8_t*)(arow + c0) + 16 * h);
        v4i bw0 = weight_frag<Q4>(brow[0], c0, h), bw1 = weight_frag<Q4>(brow[1], c0, h);
        float dw0 = f16_bits_to_f32(drow[0][c0]), dw1 = f16_bits_to_f32(drow[1][c0]);
        for (int kb = 0; kb < kc; ++kb) {
            const int b = c0 + kb;
            const v16i s0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bw0, zero, 0, 0, 0);
            const v16i s1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bw1, zero, 0, 0, 0);
            const float cw0 = dw0, cw1 = dw1;
            if (kb + 1 < kc) {
                a = *(const v4i*)((const int8_t*)(arow + b + 1) + 16 * h);
                bw0 = weight_frag<Q4>(brow[0], b + 1, h);
                bw1 = weight_frag<Q4>(brow[1], b + 1, h);
                dw0 = f16_bits_to_f32(drow[0][b + 1]);
                dw1 = f16_bits_to_f32(drow[1][b + 1]);
            }
            float da[16];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 v = sda4[kb][(32 * wm + 8 * q + 4 * h) >> 2];
                da[4 * q] = v.x;
                da[4 * q + 1] = v.y;
                da[4 * q + 2] = v.z;
                da[4 * q + 3] = v.w;
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[0][i] = acc[0][i] + ((float)s0[i] * cw0) * da[i];
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[1][i] = acc[1][i] + ((float)s1[i] * cw1) * da[i];
        }
    }
    (void)sda;

#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int n = n0 + 64 * wn + 32 * j + l31;
        if (n >= N) continue;
        const float bv = bias ? bias[n] : 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int m = m0 + 32 * wm + 8 * (i >> 2) + 4 * h + (i & 3);
            if (m >= M) continue;
            float v = bias ? acc[j][i] + bv : acc[j][i];
            if (res) v = res[(int64_t)m * ldr + n] + v;
            y[(int64_t)m * ldy + n] = v;
        }
    }
}

hipError_t launch_gemm_q80(const QWeight& w, const void* act, int m, float* y, int64_t ldy, const float* bias,
                           const float* res, int64_t ldr, hipStream_t s) {
    if ((w.dtype != kQ8_0 && w.dtype != kQ4_0) || m <= 0) return hipErrorInvalidValue;
    const int tiles_m = (m + kQBM - 1) / kQBM;
    const int tiles_n = (int)((w.n + kQBN - 1) / kQBN);
    const int grid = (tiles_n + 7) / 8 * 8 * tiles_m;
    if (w.dtype == kQ8_0)
        hipLaunchKernelGGL(k_gemm_q80<false>, dim3((unsigned)grid), dim3(256), 0, s, (const ActQ8_0*)act, m,
                           (int)w.nb, (const uint16_t*)w.hdr, w.qs, (int)w.n, tiles_m, tiles_n, y, ldy, bias, res, ldr);
    else
        hipLaunchKernelGGL(k_gemm_q80<true>, dim3((unsigned)grid), dim3(256), 0, s, (const ActQ8_0*)act, m,
                           (int)w.nb, (const uint16_t*)w.hdr, w.qs, (int)w.n, tiles_m, tiles_n, y, ldy, bias, res, ldr);
    return hipGetLastError();
}

}  // namespace sxq
