// sxq_gemv.hip -- decode GEMV (m = 1..16) over quantized weights for gfx950.
//
// y[r][row] = vec_dot(W[row], act[r]) exactly as candle-core 0.8's generic CPU
// vec-dot computes it (k_quants.rs vec_dot_unopt), bit for bit:
//   * the integer part of each block's dot product is exact in any order;
//   * the float part is replayed in Candle's order: Q8_0/Q4_0 fold
//     `sumf += (f32)isum * d_w * d_a` block by block; Q4_K keeps eight lane sums
//     `sums[l] += (d_w*d_a) * (f32)aux32[l]` (l = element index mod 8), a separate
//     `sumf -= (dmin_w*d_a) * (f32)sumi`, and returns sumf + (-0.0 + sums[0] + ... + sums[7]).
//
// Work split: an 8-lane group streams one weight row, block after block, so each row's
// float chain runs in block order inside one group.  For Q4_K lane l of the group
// loads the 16 bytes holding class l (elements = l mod 8) of all four 32-byte chunks
// (see the device layout in sxq_common.h) and produces aux32[l] directly; for Q8_0 and
// Q4_0 lane l takes block b0 + l and the group folds the eight block terms in order.
// Activations are copied from their quantized device layout into LDS once per
// workgroup (in K chunks when m * K does not fit).
#include "sxq_kernels.h"

namespace sxq {

static constexpr int kLdsBudget = 48 * 1024;

SXQ_DEV float h2f(uint32_t bits16) { return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16); }

// Copy act blocks [m][c0, c0+cb) (global, row stride nb blocks) into LDS [m][cb].
template <int ABYTES>
SXQ_DEV void stage_act(uint4* lds, const uint8_t* __restrict__ act, int m, int nb, int c0, int cb) {
    constexpr int U4 = ABYTES / 16;
    const int per_row = cb * U4;
    const int total = m * per_row;
    for (int i = threadIdx.x; i < total; i += blockDim.x) {
        const int r = i / per_row, rem = i - r * per_row;
        lds[i] = ((const uint4*)(act + ((int64_t)r * nb + c0) * ABYTES))[rem];
    }
}

// ------------------------------------------------------------------------- Q4_K x Q8_K
template <int MMAX, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void k_gemv_q4k(const uint4* __restrict__ hdr, const uint4* __restrict__ qs,
                                                         int n, int nb, const uint8_t* __restrict__ act, int m,
                                                         int cbmax, float* __restrict__ y, int64_t ldy,
                                                         const float* __restrict__ bias) {
    extern __shared__ uint4 lds[];
    const ActQ8K* la = (const ActQ8K*)lds;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l = lane & 7, grp = lane >> 3;
    const int row = (blockIdx.x * WAVES + wave) * 8 + grp;
    const bool active = row < n;
    const int rowc = active ? row : n - 1;

    float sums[MMAX], sumf[MMAX];
#pragma unroll
    for (int r = 0; r < MMAX; ++r) sums[r] = sumf[r] = 0.0f;

    for (int c0 = 0; c0 < nb; c0 += cbmax) {
        const int cb = min(cbmax, nb - c0);
        if (c0) __syncthreads();
        stage_act<sizeof(ActQ8K)>(lds, act, m, nb, c0, cb);
        __syncthreads();
        const uint4* hrow = hdr + (int64_t)rowc * nb + c0;
        const uint4* qrow = qs + ((int64_t)rowc * nb + c0) * 8 + l;
        for (int b = 0; b < cb; ++b) {
            const uint4 q = qrow[(int64_t)b * 8];
            const uint4 h = hrow[b];
            // 6-bit scales/mins of the 8 sub-blocks, packed four per dword
            const uint32_t sc_lo = h.y & 0x3F3F3F3Fu;
            const uint32_t sc_hi = (h.w & 0x0F0F0F0Fu) | (((h.y >> 6) & 0x03030303u) << 4);
            const uint32_t mn_lo = h.z & 0x3F3F3F3Fu;
            const uint32_t mn_hi = ((h.w >> 4) & 0x0F0F0F0Fu) | (((h.z >> 6) & 0x03030303u) << 4);
            const int ml = (int)(((l < 4 ? mn_lo : mn_hi) >> (8 * (l & 3))) & 0xFF);
            const uint32_t w4[8] = {q.x & 0x0F0F0F0Fu, (q.x >> 4) & 0x0F0F0F0Fu, q.y & 0x0F0F0F0Fu,
                                    (q.y >> 4) & 0x0F0F0F0Fu, q.z & 0x0F0F0F0Fu, (q.z >> 4) & 0x0F0F0F0Fu,
                                    q.w & 0x0F0F0F0Fu, (q.w >> 4) & 0x0F0F0F0Fu};
            int sc[8];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                sc[j] = (int)((sc_lo >> (8 * j)) & 0xFF);
                sc[4 + j] = (int)((sc_hi >> (8 * j)) & 0xFF);
            }
            const float dw = h2f(h.x & 0xFFFF), dminw = h2f(h.x >> 16);
#pragma unroll
            for (int r = 0; r < MMAX; ++r) {
                if (r < m) {
                    const ActQ8K& a = la[r * cb + b];
                    const uint4 A0 = ((const uint4*)a.qs)[2 * l];
                    const uint4 A1 = ((const uint4*)a.qs)[2 * l + 1];
                    const int Aj[8] = {(int)A0.x, (int)A0.y, (int)A0.z, (int)A0.w,
                                       (int)A1.x, (int)A1.y, (int)A1.z, (int)A1.w};
                    int aux = 0;
#pragma unroll
                    for (int j = 0; j < 8; ++j) aux += __mul24(__builtin_amdgcn_sdot4((int)w4[j], Aj[j], 0, false), sc[j]);
                    const int sumi = sum8_i32(__mul24(ml, a.bs2[l]));
                    const float ad = a.d;
                    const float dd = dw * ad;
                    sums[r] += dd * (float)aux;
                    const float dm = dminw * ad;
                    sumf[r] -= dm * (float)sumi;
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < MMAX; ++r) {
        if (r < m) {
            float tot = -0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) tot += __shfl(sums[r], grp * 8 + i, 64);
            float v = sumf[r] + tot;
            if (active && l == 0) {
                if (bias) v = v + bias[row];
                y[(int64_t)r * ldy + row] = v;
            }
        }
    }
}

// ----------------------------------------------------------------- Q8_0 / Q4_0 x Q8_0
template <int MMAX, int WAVES, bool Q4>
__global__ __launch_bounds__(64 * WAVES) void k_gemv_q80(const uint16_t* __restrict__ dw16, const uint4* __restrict__ qs,
                                                         int n, int nb, const uint8_t* __restrict__ act, int m,
                                                         int cbmax, float* __restrict__ y, int64_t ldy,
                                                         const float* __restrict__ bias) {
    extern __shared__ uint4 lds[];
    const ActQ8_0* la = (const ActQ8_0*)lds;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l = lane & 7, grp = lane >> 3;
    const int row = (blockIdx.x * WAVES + wave) * 8 + grp;
    const bool active = row < n;
    const int rowc = active ? row : n - 1;
    constexpr int QU4 = Q4 ? 1 : 2;  // uint4 per weight block

    float sumf[MMAX];
#pragma unroll
    for (int r = 0; r < MMAX; ++r) sumf[r] = 0.0f;

    for (int c0 = 0; c0 < nb; c0 += cbmax) {
        const int cb = min(cbmax, nb - c0);
        if (c0) __syncthreads();
        stage_act<sizeof(ActQ8_0)>(lds, act, m, nb, c0, cb);
        __syncthreads();
        for (int b0 = 0; b0 < cb; b0 += 8) {
            const int b = b0 + l;
            const bool valid = b < cb;
            const int bc = valid ? b : cb - 1;
            const int64_t blk = (int64_t)rowc * nb + c0 + bc;
            uint4 w0 = qs[blk * QU4];
            uint4 w1 = Q4 ? make_uint4(0, 0, 0, 0) : qs[blk * QU4 + 1];
            const float dw = h2f(dw16[blk]);
            const int nvalid = min(8, cb - b0);
#pragma unroll
            for (int r = 0; r < MMAX; ++r) {
                if (r < m) {
                    const ActQ8_0& a = la[r * cb + bc];
                    const uint4 A0 = ((const uint4*)a.qs)[0];
                    const uint4 A1 = ((const uint4*)a.qs)[1];
                    int isum;
                    if (Q4) {
                        const uint32_t wd[4] = {w0.x, w0.y, w0.z, w0.w};
                        const int Alo[4] = {(int)A0.x, (int)A0.y, (int)A0.z, (int)A0.w};
                        const int Ahi[4] = {(int)A1.x, (int)A1.y, (int)A1.z, (int)A1.w};
                        isum = -8 * a.asum;
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            isum = __builtin_amdgcn_sdot4((int)(wd[i] & 0x0F0F0F0Fu), Alo[i], isum, false);
                            isum = __builtin_amdgcn_sdot4((int)((wd[i] >> 4) & 0x0F0F0F0Fu), Ahi[i], isum, false);
                        }
                    } else {
                        isum = __builtin_amdgcn_sdot4((int)w0.x, (int)A0.x, 0, false);
                        isum = __builtin_amdgcn_sdot4((int)w0.y, (int)A0.y, isum, false);
                        isum = __builtin_amdgcn_sdot4((int)w0.z, (int)A0.z, isum, false);
                        isum = __builtin_amdgcn_sdot4((int)w0.w, (int)A0.w, isum, false);
                        isum = __builtin_amdgcn_sdot4((int)w1.x, (int)A1.x, isum, false);
                        isum = __builtin_amdgcn_sdot4((int)w1.y, (int)A1.y, isum, false);
                        isum = __builtin_amdgcn_sdot4((int)w1.z, (int)A1.z, isum, false);
                        isum = __builtin_amdgcn_sdot4((int)w1.w, (int)A1.w, isum, false);
                    }
                    const float t = ((float)isum * dw) * a.d;
                    // fold the group's block terms into sumf in block order
                    float acc = sumf[r];
                    for (int i = 0; i < nvalid; ++i) acc += __shfl(t, grp * 8 + i, 64);
                    sumf[r] = acc;
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < MMAX; ++r) {
        if (r < m && active && l == 0) {
            float v = sumf[r];
            if (bias) v = v + bias[row];
            y[(int64_t)r * ldy + row] = v;
        }
    }
}

template <int MMAX>
static hipError_t gemv_dispatch(const QWeight& w, const void* act, int m, float* y, int64_t ldy, const float* bias,
                                hipStream_t s) {
    const int n = (int)w.n, nb = (int)w.nb;
    const int groups = (n + 7) / 8;
    // Four waves per workgroup once there are enough rows to fill the chip that way.
    const bool wide = groups >= 4 * 1024;
    const int waves = wide ? 4 : 1;
    const dim3 grid((groups + waves - 1) / waves), block(64 * waves);
    const size_t ab = act_block_bytes(vec_dot_type(w.dtype));
    int cbmax = (int)(kLdsBudget / (ab * (size_t)m));
    if (cbmax < 1) cbmax = 1;
    if (cbmax > nb) cbmax = nb;
    const size_t lds = ab * (size_t)m * (size_t)cbmax;
    const uint8_t* a = (const uint8_t*)act;
    if (w.dtype == kQ4K) {
        if (wide) hipLaunchKernelGGL((k_gemv_q4k<MMAX, 4>), grid, block, lds, s, (const uint4*)w.hdr, (const uint4*)w.qs, n, nb, a, m, cbmax, y, ldy, bias);
        else hipLaunchKernelGGL((k_gemv_q4k<MMAX, 1>), grid, block, lds, s, (const uint4*)w.hdr, (const uint4*)w.qs, n, nb, a, m, cbmax, y, ldy, bias);
    } else if (w.dtype == kQ8_0) {
        if (wide) hipLaunchKernelGGL((k_gemv_q80<MMAX, 4, false>), grid, block, lds, s, (const uint16_t*)w.hdr, (const uint4*)w.qs, n, nb, a, m, cbmax, y, ldy, bias);
        else hipLaunchKernelGGL((k_gemv_q80<MMAX, 1, false>), grid, block, lds, s, (const uint16_t*)w.hdr, (const uint4*)w.qs, n, nb, a, m, cbmax, y, ldy, bias);
    } else if (w.dtype == kQ4_0) {
        if (wide) hipLaunchKernelGGL((k_gemv_q80<MMAX, 4, true>), grid, block, lds, s, (const uint16_t*)w.hdr, (const uint4*)w.qs, n, nb, a, m, cbmax, y, ldy, bias);
        else hipLaunchKernelGGL((k_gemv_q80<MMAX, 1, true>), grid, block, lds, s, (const uint16_t*)w.hdr, (const uint4*)w.qs, n, nb, a, m, cbmax, y, ldy, bias);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_gemv(const QWeight& w, const void* act, int m, float* y, int64_t ldy, const float* bias,
                       hipStream_t s) {
    if (m <= 0 || w.n <= 0) return hipSuccess;
    if (m == 1) return gemv_dispatch<1>(w, act, m, y, ldy, bias, s);
    if (m == 2) return gemv_dispatch<2>(w, act, m, y, ldy, bias, s);
    if (m <= 4) return gemv_dispatch<4>(w, act, m, y, ldy, bias, s);
    if (m <= 8) return gemv_dispatch<8>(w, act, m, y, ldy, bias, s);
    if (m <= 16) return gemv_dispatch<16>(w, act, m, y, ldy, bias, s);
    return hipErrorInvalidValue;
}

}  // namespace sxq
