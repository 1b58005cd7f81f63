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
#include <stddef.h>
#include <stdlib.h>

#include <atomic>
#include <type_traits>

#include "sxq_decoder.h"
#include "sxq_gemv_dev.h"
#include "sxq_kernels.h"

namespace sxq {

static constexpr int kLdsBudget = 48 * 1024;

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
                                                         int cbmax, float* y, int64_t ldy,
                                                         const float* __restrict__ bias, const float* res, int64_t ldr) {
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
                if (res) v = res[(int64_t)r * ldr + row] + v;  // residual: `r + a`
                y[(int64_t)r * ldy + row] = v;
            }
        }
    }
}

// ----------------------------------------------------------------- Q8_0 / Q4_0 x Q8_0
template <int MMAX, int WAVES, bool Q4>
__global__ __launch_bounds__(64 * WAVES) void k_gemv_q80(const uint16_t* __restrict__ dw16, const uint4* __restrict__ qs,
                                                         int n, int nb, const uint8_t* __restrict__ act, int m,
                                                         int cbmax, float* y, int64_t ldy,
                                                         const float* __restrict__ bias, const float* res, int64_t ldr) {
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
            if (res) v = res[(int64_t)r * ldr + row] + v;  // residual: `r + a`
            y[(int64_t)r * ldy + row] = v;
        }
    }
}

// ---------------------------------------------------------------------------------
// Task-split GEMV (m = 1..4).  A 256-thread workgroup owns R consecutive rows; their
// R*nb (row, block) tasks are dealt round-robin to 256/kQ4kLanes lane groups (Q4_K), 128
// lane pairs (Q8_0) or 256 lanes (Q4_0), at most TMAX tasks each.  Every group first
// issues the weight loads of all its tasks (clamped, unconditional), then the
// activation loads into LDS, so a wave has up to 2*TMAX 16-byte loads in flight and
// the compute that follows is branch-free.  Each task leaves Candle's per-block float
// product(s) in LDS: Q4_K the eight lane terms (d_w*d_a)*(f32)aux32[l] and the min term
// (dmin_w*d_a)*(f32)sumi; Q8_0/Q4_0 the term ((f32)isum*d_w)*d_a.  The epilogue folds
// them in block order per (row, lane) -- the only order-dependent part -- so results
// stay bit-identical to Candle's generic vec-dot.  The Q4_K tile (loads, products,
// fold) is in sxq_gemv_dev.h.

// Activation staging in two halves so the caller can put its weight loads between
// them: act_fetch issues a thread's first 16-byte loads (clamped, so all are
// unconditional and in flight together); act_store writes them to LDS and copies any
// remainder (only when m * nb blocks exceed kPer * NT uint4).
template <int NT, int MMAX>
struct Stage {
    // 16 KB first; 16 KB per activation row for 1024 threads, whose multi-row launches
    // stage up to 46 KB
    static constexpr int kPer = NT == 1024 ? MMAX : 1024 / NT;
};
template <int NT, int MMAX, int KP = Stage<NT, MMAX>::kPer>
SXQ_DEV void act_fetch(uint4 (&v)[KP], const uint8_t* __restrict__ act, int total_u4) {
#pragma unroll
    for (int k = 0; k < KP; ++k)
        v[k] = ld_global((const uint4*)opaque_ptr(act) + min(k * NT + (int)threadIdx.x, total_u4 - 1));
    issue_point();  // keep these loads ahead of the weight loads
}
template <int NT, int MMAX, int KP = Stage<NT, MMAX>::kPer>
SXQ_DEV void act_store(const uint4 (&v)[KP], uint4* lds, const uint8_t* __restrict__ act, int total_u4) {
    // clamped like the loads: out-of-range threads rewrite the last element with its own value
#pragma unroll
    for (int k = 0; k < KP; ++k) lds[min(k * NT + (int)threadIdx.x, total_u4 - 1)] = v[k];
    for (int i = KP * NT + threadIdx.x; i < total_u4; i += NT) lds[i] = ((const uint4*)act)[i];
}

// Q4_K task-split GEMV, NT threads (256 or 1024) per workgroup: NT/kQ4kLanes lane groups,
// TM rounds of tasks (the launch's tiles need no more; a round that held no task would
// still issue its loads, and the epilogue would wait for them before reusing their
// registers).
template <int MMAX, bool NORM, int NT, int TM>
__global__ __launch_bounds__(NT) void k_gemv2_q4k(const uint4* __restrict__ hdr, const uint4* __restrict__ qs, int n,
                                                  int nb, const uint8_t* __restrict__ act, int m, int R, float* y,
                                                  int64_t ldy, const float* __restrict__ bias, const float* res,
                                                  int64_t ldr, NormIn ni) {
    static_assert(!NORM || (NT == 1024 && MMAX == 1), "the fused RMSNorm prologue is for one row, 1024 threads");
    constexpr int SLOTS = NT / kQ4kLanes;  // lane groups = tasks per round
    extern __shared__ uint4 lds[];
    const ActQ8K* la = (const ActQ8K*)lds;
    const int row0 = blockIdx.x * R;
    const int rows = min(R, n - row0);
    const int tasks = rows * nb;
    float* pr = (float*)(lds + (size_t)m * nb * (sizeof(ActQ8K) / 16));  // product chains [m][R + 1][9][CS]
    const uint32_t blk0 = (uint32_t)row0 * (uint32_t)nb;
    const int act_u4 = m * nb * (int)(sizeof(ActQ8K) / 16);
    uint4 av[Stage<NT, MMAX>::kPer];
    float4 xv, wv;
    if constexpr (NORM) norm_fetch(xv, wv, ni, nb * 256);
    else act_fetch<NT, MMAX>(av, act, act_u4);
    uint4 q[TM][kQ4kCpl], h[TM];
    q4k_tile_load<NT, TM>(hdr, qs, blk0, tasks, q, h);
    if constexpr (NORM) {
        __shared__ float red[16];
        norm_quant_store<kQ8K>(xv, wv, ni, nb * 256, (uint8_t*)lds, red);
    } else {
        act_store<NT, MMAX>(av, lds, act, act_u4);
    }
    // The activations are in LDS; the weight loads may still be in flight: each round of
    // products waits only for its own.
    lds_barrier();
    q4k_tile_products<MMAX, NT, TM>(q, h, la, nb, m, rows, R, pr);
    __syncthreads();
    // epilogue: thread (row r, lane class l) folds its chain in block order
    const int r = threadIdx.x >> 3, l = threadIdx.x & 7;
    for (int rr = 0; rr < m; ++rr) {
        const float v0 = q4k_tile_fold(pr, nb, R, rr, rows);
        if (r < rows && l == 0) {
            const int row = row0 + r;
            float v = v0;
            if (bias) v = v + bias[row];
            if (res) v = res[(int64_t)rr * ldr + row] + v;
            y[(int64_t)rr * ldy + row] = v;
        }
    }
}

// ------------------------------------------------- SwiGLU pair around the down projection
// One decode row (m = 1, 1024 threads), Q4_K weights.  k_gemv2_q4k_swiglu is the fused
// RMSNorm GEMV of the gate|up weight [2I][nb] (gate rows 0..I-1, up rows I..2I-1) whose
// tile t holds gate rows [tB, tB + Bt) and the same up rows [I + tB, I + tB + Bt), so its
// epilogue has both halves of each pair: it stores gu (both halves, canonical order) and
// a = silu(g) * u -- k_silu_mul_quant's arithmetic -- as f32.  k_gemv2_q4k_quant is the
// down projection whose prologue quantizes that f32 row to Q8_K in LDS (chunk c by wave
// c mod 16, the quantizer of k_silu_mul_quant), so the two leave the same bits as the
// GEMV + SiLU*mul kernel + GEMV sequence, one launch and one quantized row fewer.
template <int TM>
__global__ __launch_bounds__(1024) void k_gemv2_q4k_swiglu(const uint4* __restrict__ hdr, const uint4* __restrict__ qs,
                                                           int I, int nb, int B, NormIn ni, float* __restrict__ gu,
                                                           float* __restrict__ act_f32) {
    constexpr int NT = 1024;
    extern __shared__ uint4 lds[];
    __shared__ float sw[NT / 8];  // the tile's row results: gate [0, Bt), up [Bt, 2Bt)
    __shared__ float red[16];
    const ActQ8K* la = (const ActQ8K*)lds;
    const int t = blockIdx.x, g0 = t * B, Bt = min(B, I - g0);
    const int rows = 2 * Bt, tasks = rows * nb, seg = Bt * nb;
    float* pr = (float*)(lds + (size_t)nb * (sizeof(ActQ8K) / 16));  // product chains [2B + 1][9][CS]
    float4 xv, wv;
    norm_fetch(xv, wv, ni, nb * 256);
    uint4 q[TM][kQ4kCpl], h[TM];
    q4k_tile_load2<NT, TM>(hdr, qs, (uint32_t)g0 * (uint32_t)nb, (uint32_t)(I + g0) * (uint32_t)nb, seg, tasks, q, h);
    norm_quant_store<kQ8K>(xv, wv, ni, nb * 256, (uint8_t*)lds, red);
    lds_barrier();
    q4k_tile_products<1, NT, TM>(q, h, la, nb, 1, rows, 2 * B, pr);
    __syncthreads();
    const int r = threadIdx.x >> 3, l = threadIdx.x & 7;
    const float v = q4k_tile_fold(pr, nb, 2 * B, 0, rows);
    if (r < rows && l == 0) {
        sw[r] = v;
        gu[r < Bt ? g0 + r : I + g0 + (r - Bt)] = v;
    }
    __syncthreads();
    if (threadIdx.x < Bt) {
        const float gv = sw[threadIdx.x], uv = sw[Bt + threadIdx.x];
        act_f32[g0 + threadIdx.x] = (gv / (1.0f + expf(-gv))) * uv;
    }
}

template <int TM>
__global__ __launch_bounds__(1024) void k_gemv2_q4k_quant(const uint4* __restrict__ hdr, const uint4* __restrict__ qs,
                                                          int n, int nb, int R, const float* __restrict__ x,
                                                          float* y, const float* res) {
    constexpr int NT = 1024, J = 3;
    extern __shared__ uint4 lds[];
    ActQ8K* la = (ActQ8K*)lds;
    const int row0 = blockIdx.x * R, rows = min(R, n - row0), tasks = rows * nb;
    float* pr = (float*)(lds + (size_t)nb * (sizeof(ActQ8K) / 16));  // product chains [R + 1][9][CS]
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // wave w quantizes chunks w, w + 16, w + 32 (nb <= 48); their loads go ahead of the
    // weight loads, which return after them
    float4 v[J];
    void* out[J];
    bool valid[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int c = wave + 16 * j, cc = min(c, nb - 1);
        valid[j] = c < nb;
        out[j] = la + cc;
        v[j] = ld_global((const float4*)(opaque_ptr(x) + cc * 256 + 4 * lane));
    }
    issue_point();
    uint4 q[TM][kQ4kCpl], h[TM];
    q4k_tile_load<NT, TM>(hdr, qs, (uint32_t)row0 * (uint32_t)nb, tasks, q, h);
    // Called by every wave (a wave past the last chunk writes nothing): under a branch the
    // compiler would sink the loads above into it, behind the weight loads.
    wave_quantize_q8k_n<J, false>(v, lane, out, valid);
    lds_barrier();
    q4k_tile_products<1, NT, TM>(q, h, la, nb, 1, rows, R, pr);
    __syncthreads();
    const int r = threadIdx.x >> 3, l = threadIdx.x & 7;
    const float v0 = q4k_tile_fold(pr, nb, R, 0, rows);
    if (r < rows && l == 0) {
        const int row = row0 + r;
        float v = v0;
        if (res) v = res[row] + v;
        y[row] = v;
    }
}

// Q8_0 / Q4_0 task-split GEMV: a lane pair per Q8_0 task (16 bytes each), one lane per
// Q4_0 task; NT threads per workgroup.  PRO selects the activation prologue:
//   kProStage  the Q8_0 activation blocks `act` [m][nb], staged into LDS;
//   kProNorm   one row: RMSNorm + the Q8_0 quantizer of ni.x in the prologue;
//   kProPair   kProNorm on the gate|up weight [2n][nb] as a SwiGLU pair: tile t holds gate
//              rows [tR, tR + Rt) and the same up rows [n + tR, n + tR + Rt); the epilogue
//              stores both halves into y (= gu [2n]) and a = silu(g) * u -- k_silu_mul_quant's
//              arithmetic -- into act_out [n];
//   kProQuant  one row: the f32 row ni.x [nb * 32] quantized to Q8_0 in LDS (chunk c of 256
//              by wave c mod 16, the quantizer of k_silu_mul_quant and k_quantize_act; past
//              the row's end a chunk reads zeros), the down projection of the pair and the
//              one-row QMatMul forward.
// The pair leaves the bits of the GEMV + SiLU*mul kernel + GEMV sequence.
constexpr int kProStage = 0, kProNorm = 1, kProPair = 2, kProQuant = 3;
template <int MMAX, bool Q4, int PRO, int NT, int TM>
__global__ __launch_bounds__(NT) void k_gemv2_q80(const uint16_t* __restrict__ dw16, const uint4* __restrict__ qs,
                                                  int n, int nb, const uint8_t* __restrict__ act, int m, int R,
                                                  float* y, int64_t ldy, const float* __restrict__ bias,
                                                  const float* res, int64_t ldr, NormIn ni, float* act_out) {
    static_assert(PRO == kProStage || (MMAX == 1 && (NT == 1024 || PRO == kProQuant)),
                  "the fused prologues are for one row, the RMSNorm ones with 1024 threads");
    constexpr bool NORM = PRO == kProNorm || PRO == kProPair;
    extern __shared__ uint4 lds[];
    const ActQ8_0* la = (const ActQ8_0*)lds;
    const int row0 = blockIdx.x * R;
    // a pair tile: Rt gate rows, then the same up rows, n rows apart (tasks seg.. skip ahead)
    const int Rt = min(R, n - row0);
    const int rows = PRO == kProPair ? 2 * Rt : Rt;
    const int tasks = rows * nb;
    const int seg = PRO == kProPair ? Rt * nb : tasks;
    const int64_t skip = PRO == kProPair ? (int64_t)(n - Rt) * nb : 0;
    constexpr int LPT = Q4 ? 1 : 2, TPI = NT / LPT, QU4 = Q4 ? 1 : 2;
    const int TS = (tasks + TPI - 1) / TPI * TPI;  // product slots: whole rounds
    float* pr = (float*)(lds + (size_t)m * nb * (sizeof(ActQ8_0) / 16));  // [m][TS]
    const int half = Q4 ? 0 : (threadIdx.x & 1);
    const int slot = threadIdx.x / LPT;
    const int64_t base = (int64_t)row0 * nb;
    const int act_u4 = m * nb * (int)(sizeof(ActQ8_0) / 16);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    constexpr int J = 3, NWV = NT / 64;  // kProQuant: chunks per wave (nb <= J * NWV * 8), waves
    uint4 av[PRO == kProStage ? Stage<NT, MMAX>::kPer : 1];
    float4 xv, wv, qv[J];
    if constexpr (NORM) {
        norm_fetch(xv, wv, ni, nb * 32);
    } else if constexpr (PRO == kProQuant) {
        // the row's loads go ahead of the weight loads, which return after them
        const int nch = (nb + 7) >> 3;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int cc = min(wave + NWV * j, nch - 1), e = cc * 256 + 4 * lane;
            qv[j] = e < nb * 32 ? ld_global((const float4*)(opaque_ptr(ni.x) + e)) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        issue_point();
    } else {
        act_fetch<NT, MMAX>(av, act, act_u4);
    }
    uint4 w[TM];
    float dw[TM];
#pragma unroll
    for (int u = 0; u < TM; ++u) {
        const int t = min(u * TPI + slot, tasks - 1);
        const int64_t wt = base + t + (t >= seg ? skip : 0);
        w[u] = qs[wt * QU4 + half];
        dw[u] = h2f(dw16[wt]);
    }
    if constexpr (NORM) {
        __shared__ float red[16];
        norm_quant_store<kQ8_0>(xv, wv, ni, nb * 32, (uint8_t*)lds, red);
    } else if constexpr (PRO == kProQuant) {
        // every wave calls the quantizer (a chunk past the row writes nothing)
        const int nch = (nb + 7) >> 3;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int c = wave + NWV * j;
            wave_quantize_q8_0<false>(qv[j], lane, c < nch && c * 8 + (lane >> 3) < nb,
                                      (uint8_t*)lds + (size_t)min(c, nch - 1) * 8 * sizeof(ActQ8_0));
        }
    } else {
        act_store<NT, MMAX>(av, lds, act, act_u4);
    }
    __syncthreads();
    // Block index of task u*TPI + slot, stepped by TPI mod nb each round; tasks past the
    // end write spare slots that the epilogue never reads.
    const uint32_t step = (uint32_t)TPI % (uint32_t)nb;
    uint32_t b = (uint32_t)slot % (uint32_t)nb;
#pragma unroll
    for (int u = 0; u < TM; ++u) {
        if (u * TPI >= tasks) break;
#pragma unroll
        for (int r = 0; r < MMAX; ++r) {
            if (r < m) {
                const ActQ8_0& a = la[r * nb + (int)b];
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
                    const uint4 A = ((const uint4*)a.qs)[half];
                    int s = __builtin_amdgcn_sdot4((int)w[u].x, (int)A.x, 0, false);
                    s = __builtin_amdgcn_sdot4((int)w[u].y, (int)A.y, s, false);
                    s = __builtin_amdgcn_sdot4((int)w[u].z, (int)A.z, s, false);
                    s = __builtin_amdgcn_sdot4((int)w[u].w, (int)A.w, s, false);
                    isum = s + dpp_xor1(s);
                }
                // Q8_0: both lanes of the pair hold the full isum and write the same value
                pr[r * TS + u * TPI + slot] = ((float)isum * dw[u]) * a.d;
            }
        }
        b += step;
        b = min(b, b - (uint32_t)nb);  // unsigned: subtracts nb only when b >= nb
    }
    __syncthreads();
    if constexpr (PRO == kProPair) {
        __shared__ float sw[NT / 2];  // the tile's row results: gate [0, Rt), up [Rt, 2Rt)
        for (int i = threadIdx.x; i < rows; i += NT) {
            const float* p = pr + i * nb;
            float sumf = 0.0f;
            for (int b = 0; b < nb; ++b) sumf += p[b];
            sw[i] = sumf;
            y[i < Rt ? row0 + i : n + row0 + (i - Rt)] = sumf;
        }
        __syncthreads();
        if (threadIdx.x < Rt) {
            const float gv = sw[threadIdx.x], uv = sw[Rt + threadIdx.x];
            act_out[row0 + threadIdx.x] = (gv / (1.0f + expf(-gv))) * uv;
        }
        return;
    }
    for (int i = threadIdx.x; i < rows * m; i += NT) {
        const int r = i / m, rr = i - r * m;
        const float* p = pr + rr * TS + r * nb;
        float sumf = 0.0f;
        for (int b = 0; b < nb; ++b) sumf += p[b];
        const int row = row0 + r;
        if (bias) sumf = sumf + bias[row];
        if (res) sumf = res[(int64_t)rr * ldr + row] + sumf;
        y[(int64_t)rr * ldy + row] = sumf;
    }
}

// Task-split sizing for NT threads per workgroup.  Rows per workgroup R: spread the
// rows over one full wave of workgroups -- 256 (one 1024-thread workgroup per CU) or
// 1024 (four 256-thread workgroups per CU), overridable with SXQ_GEMV_WG -- capped so
// every lane group holds at most kTmax tasks, the epilogue has a thread per (row, lane
// class), and LDS fits the workgroup's share of a CU's 160 KB: 60 KB for 256 threads,
// 144 KB for 1024 (one workgroup per CU).
static int tasks_per_round(int dtype, int nt) { return dtype == kQ4K ? nt / kQ4kLanes : (dtype == kQ8_0 ? nt / 2 : nt); }
// Q4_K rounds of a 1024-thread workgroup: at most 7 (eight rounds of 12 weight registers
// would not fit the 128 VGPRs of 1024 threads); kTmax elsewhere.
constexpr int kTmaxQ4k1024 = 7;
static int round_cap(int dtype, int nt) { return dtype == kQ4K && nt == 1024 ? kTmaxQ4k1024 : kTmax; }

size_t gemv2_lds(int nb, int m, int R, int dtype, int nt) {
    const size_t ab = act_block_bytes(vec_dot_type(dtype));
    if (dtype == kQ4K) return (size_t)m * nb * ab + (size_t)m * (R + 1) * 9 * q4k_chain_stride(nb) * 4;
    const int tpi = tasks_per_round(dtype, nt);
    const size_t slots = ((size_t)R * nb + tpi - 1) / tpi * tpi;
    return (size_t)m * nb * ab + slots * m * 4;
}

static size_t gemv2_lds_cap(int nt) { return nt == 1024 ? 144 * 1024 : 60 * 1024; }

int gemv2_rows(int n, int nb, int m, int dtype, int nt) {
    static const int env_wg = [] {
        const char* e = getenv("SXQ_GEMV_WG");
        return e ? atoi(e) : 0;
    }();
    const int target_wg = env_wg > 0 ? env_wg : (nt == 1024 ? 256 : 1024);
    int R = (n + target_wg - 1) / target_wg;
    R = min(R, nt / 8);
    R = min(R, max(1, tasks_per_round(dtype, nt) * round_cap(dtype, nt) / nb));
    while (R > 1 && gemv2_lds(nb, m, R, dtype, nt) > gemv2_lds_cap(nt)) --R;
    return max(R, 1);
}

// Whether the task-split kernel with NT threads covers this shape: one row's tasks
// within kTmax rounds and LDS within the cap; for NT = 1024 and one activation row also
// no more workgroups than the one-per-CU target (otherwise the 256-thread kernel is the
// better fit; with more rows the larger LDS share wins at any workgroup count).
bool gemv2_fits(int n, int nb, int m, int dtype, int nt) {
    if (nb > tasks_per_round(dtype, nt) * round_cap(dtype, nt) || gemv2_lds(nb, m, 1, dtype, nt) > gemv2_lds_cap(nt))
        return false;
    if (nt == 256 || m > 1) return true;
    const int R = gemv2_rows(n, nb, m, dtype, nt);
    return (n + R - 1) / R <= 256;
}

// Threads per workgroup.  One activation row: 256 (measured at least as fast as 1024 at
// every decode shape, and faster for w1|w3).  Two or more rows: 1024 where it fits --
// every workgroup stages all m rows of activation blocks in LDS, and with 256 threads
// the LDS cap leaves so few weight rows per workgroup that the staging outweighs the
// weights (the 9728-wide down projection at m = 4: one row per workgroup, 2560
// workgroups each staging 46 KB).  SXQ_GEMV_NT=256 or 1024 forces one size where it fits.
// The fused RMSNorm prologue always runs with 1024 threads, so the row is normalised
// and quantized once per CU rather than four times.
static int gemv2_nt(int n, int nb, int m, int dtype) {
    static const int env_nt = [] {
        const char* e = getenv("SXQ_GEMV_NT");
        return e ? atoi(e) : 0;
    }();
    const bool wide = env_nt ? env_nt == 1024 : m >= 2;
    return wide && gemv2_fits(n, nb, m, dtype, 1024) ? 1024 : 256;
}

// A launch with more than 64 KB of dynamic LDS needs the kernel's limit raised first;
// raised once per kernel, to the largest cap any launch of it asks for.
template <auto K>
static hipError_t allow_lds(size_t lds) {
    if (lds <= 64 * 1024) return hipSuccess;
    static const hipError_t e =
        hipFuncSetAttribute((const void*)K, hipFuncAttributeMaxDynamicSharedMemorySize, (int)gemv2_lds_cap(1024));
    return e;
}

// Calls f(std::integral_constant<int, TM>()) for TM = rounds (1 .. kTmax).
template <typename F>
static hipError_t with_rounds(int rounds, F&& f) {
    switch (rounds) {
        case 1: return f(std::integral_constant<int, 1>());
        case 2: return f(std::integral_constant<int, 2>());
        case 3: return f(std::integral_constant<int, 3>());
        case 4: return f(std::integral_constant<int, 4>());
        case 5: return f(std::integral_constant<int, 5>());
        case 6: return f(std::integral_constant<int, 6>());
        case 7: return f(std::integral_constant<int, 7>());
        case 8: return f(std::integral_constant<int, 8>());
        default: return hipErrorInvalidValue;
    }
}
static_assert(kTmax == 8, "with_rounds covers 1 .. kTmax");

template <int MMAX, bool NORM, int NT>
static hipError_t gemv2_launch(const QWeight& w, const void* act, int m, float* y, int64_t ldy, const float* bias,
                               const float* res, int64_t ldr, hipStream_t s, const NormIn& ni) {
    const int n = (int)w.n, nb = (int)w.nb;
    const int R = gemv2_rows(n, nb, m, w.dtype, NT);
    const size_t lds = gemv2_lds(nb, m, R, w.dtype, NT);
    const dim3 grid((n + R - 1) / R), block(NT);
    const uint8_t* a = (const uint8_t*)act;
    const int tpr = tasks_per_round(w.dtype, NT);
    const int rounds = (R * nb + tpr - 1) / tpr;
    const hipError_t e = with_rounds(rounds, [&](auto tmc) -> hipError_t {
        constexpr int TM = decltype(tmc)::value;
        if (w.dtype == kQ4K) {
            if constexpr (NT == 1024 && TM > kTmaxQ4k1024) {
                return hipErrorInvalidValue;  // (gemv2_rows never asks for it)
            } else {
                if (const hipError_t e_ = allow_lds<k_gemv2_q4k<MMAX, NORM, NT, TM>>(lds); e_ != hipSuccess) return e_;
                hipLaunchKernelGGL((k_gemv2_q4k<MMAX, NORM, NT, TM>), grid, block, lds, s, (const uint4*)w.hdr,
                                   (const uint4*)w.qs, n, nb, a, m, R, y, ldy, bias, res, ldr, ni);
            }
        } else if (w.dtype == kQ8_0) {
            if (const hipError_t e_ = allow_lds<k_gemv2_q80<MMAX, false, NORM, NT, TM>>(lds); e_ != hipSuccess) return e_;
            hipLaunchKernelGGL((k_gemv2_q80<MMAX, false, NORM, NT, TM>), grid, block, lds, s, (const uint16_t*)w.hdr, (const uint4*)w.qs, n, nb, a, m, R, y, ldy, bias, res, ldr, ni, (float*)nullptr);
        } else if (w.dtype == kQ4_0) {
            if (const hipError_t e_ = allow_lds<k_gemv2_q80<MMAX, true, NORM, NT, TM>>(lds); e_ != hipSuccess) return e_;
            hipLaunchKernelGGL((k_gemv2_q80<MMAX, true, NORM, NT, TM>), grid, block, lds, s, (const uint16_t*)w.hdr, (const uint4*)w.qs, n, nb, a, m, R, y, ldy, bias, res, ldr, ni, (float*)nullptr);
        } else {
            return hipErrorInvalidValue;
        }
        return hipSuccess;
    });
    if (e != hipSuccess) return e;
    return hipGetLastError();
}

template <int MMAX>
static hipError_t gemv2_dispatch(const QWeight& w, const void* act, int m, float* y, int64_t ldy, const float* bias,
                                 const float* res, int64_t ldr, hipStream_t s) {
    if (gemv2_nt((int)w.n, (int)w.nb, m, w.dtype) == 1024)
        return gemv2_launch<MMAX, false, 1024>(w, act, m, y, ldy, bias, res, ldr, s, NormIn());
    return gemv2_launch<MMAX, false, 256>(w, act, m, y, ldy, bias, res, ldr, s, NormIn());
}

template <int MMAX>
static hipError_t gemv_dispatch(const QWeight& w, const void* act, int m, float* y, int64_t ldy, const float* bias,
                                const float* res, int64_t ldr, hipStream_t s) {
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
        if (wide) hipLaunchKernelGGL((k_gemv_q4k<MMAX, 4>), grid, block, lds, s, (const uint4*)w.hdr, (const uint4*)w.qs, n, nb, a, m, cbmax, y, ldy, bias, res, ldr);
        else hipLaunchKernelGGL((k_gemv_q4k<MMAX, 1>), grid, block, lds, s, (const uint4*)w.hdr, (const uint4*)w.qs, n, nb, a, m, cbmax, y, ldy, bias, res, ldr);
    } else if (w.dtype == kQ8_0) {
        if (wide) hipLaunchKernelGGL((k_gemv_q80<MMAX, 4, false>), grid, block, lds, s, (const uint16_t*)w.hdr, (const uint4*)w.qs, n, nb, a, m, cbmax, y, ldy, bias, res, ldr);
        else hipLaunchKernelGGL((k_gemv_q80<MMAX, 1, false>), grid, block, lds, s, (const uint16_t*)w.hdr, (const uint4*)w.qs, n, nb, a, m, cbmax, y, ldy, bias, res, ldr);
    } else if (w.dtype == kQ4_0) {
        if (wide) hipLaunchKernelGGL((k_gemv_q80<MMAX, 4, true>), grid, block, lds, s, (const uint16_t*)w.hdr, (const uint4*)w.qs, n, nb, a, m, cbmax, y, ldy, bias, res, ldr);
        else hipLaunchKernelGGL((k_gemv_q80<MMAX, 1, true>), grid, block, lds, s, (const uint16_t*)w.hdr, (const uint4*)w.qs, n, nb, a, m, cbmax, y, ldy, bias, res, ldr);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ----------------------------------------- skinny batch: Q4_K GEMV on f16 matrix cores
// 5..16 activation rows.  The integer part of Candle's Q4_K vec-dot, aux32[l] (class l =
// element index mod 8) = sum over the block's 32 class-l elements of sc_s * q4 * q8,
// runs on v_mfma_f32_16x16x32_f16 with exact operands: q8 in [-128, 127] and
// W' = sc_s * q4 <= 945 are integers that f16 holds exactly, every product and partial
// sum is an integer below 2^24, so the f32 accumulator holds aux32 exactly, in any
// order.  One MFMA per (class, block) gives 16 activation rows x 16 weight rows; the
// min term's sumi = sum_s mins_s * bs2_s (|bs2| <= 4096) runs on two
// v_mfma_f32_16x16x4_f32 the same way.  The float steps stay Candle's: per block
// sums[l] += (d_w * d_a) * aux32[l] and sumf -= (dmin_w * d_a) * sumi, chains in
// block order, then sumf + (-0.0 + sums[0] + ... + sums[7]).
//
// A workgroup of 8 waves owns 16 weight rows and all their blocks; wave w runs class w
// (wave 0 also the min term) over the blocks in order, so every chain
// stays in one lane's registers in block order, and only at the end do the eight class
// sums of each (activation row, weight row) meet in LDS, added in class order.  The
// operands go through LDS in chunks of four blocks, copied with contiguous 16-byte loads
// (whole cache lines; each lane's own pieces are 4- to 16-byte scraps of many lines)
// into row-padded tiles that the lanes then read without bank conflicts: weights
// 16 rows x 512 B (+16), headers decoded once per (block, lane group, row) into the
// f16 scale pairs of the W' FMA and d, dmin, mins as floats, and activations
// 16 rows x 4 x 304 B (+16); double-buffered, loaded one chunk ahead, one barrier per
// chunk (71 KB: two workgroups, 16 waves, per CU).  Activation rows past m and weight rows past n use clamped copies and are never
// stored.  MFMA k-slots: lane group g (lane / 16) of a class-l operand holds dword g of
// the weight's class-l 16 bytes (device layout: byte 16l + 4c + t holds elements
// 64c + l + 8t and 64c + 32 + l + 8t), as the eight values (t, nibble) = (0,lo) (2,lo)
// (1,lo) (3,lo) (0,hi) (2,hi) (1,hi) (3,hi); the activation operand holds the same
// elements, which sit at qs[32l + 8g + {0,2,1,3,4,6,5,7}] of the class-major Q8_K block.
constexpr int kMmaRows = 16;
constexpr int kMmaChunk = 4;                          // blocks per chunk
constexpr int kMmaWRow = kMmaChunk * 32 + 4;          // dwords per weight row of a chunk (padded)
constexpr int kMmaARow = kMmaChunk * 76 + 4;          // dwords per activation row of a chunk (padded)
constexpr int kMmaHdr = kMmaChunk * 4 * 16 * 8;     // decoded headers: [block][g][row] x 2 uint4
constexpr int kMmaBuf = 16 * kMmaWRow + kMmaHdr + 16 * kMmaARow;  // dwords per chunk buffer
constexpr size_t kMmaLds = 2 * (size_t)kMmaBuf * 4;
static_assert(kMmaBuf >= 9 * 256, "the final class sums reuse a chunk buffer");
static_assert(sizeof(ActQ8K) == 76 * 4, "activation rows are copied as 19 uint4 per block");

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// (1024 + hi16, 1024 + lo16) f16 pair of two 16-bit integers below 1024
SXQ_DEV half2_t mma_magic(uint32_t v) { return __builtin_bit_cast(half2_t, v | 0x64006400u); }

// one class dword of a weight block -> its eight W' = sc * q4 in slot order (sc0: low
// nibbles, sub-block 2g; sc1: high nibbles, sub-block 2g + 1); exact: (1024 + q) * sc
// - 1024 * sc rounds once, to the integer q * sc
SXQ_DEV half8_t mma_weight8(uint32_t v, half2_t sc0, half2_t ns0, half2_t sc1, half2_t ns1) {
    const half2_t x0 = __builtin_elementwise_fma(mma_magic(v & 0x000F000Fu), sc0, ns0);
    const half2_t x1 = __builtin_elementwise_fma(mma_magic((v >> 8) & 0x000F000Fu), sc0, ns0);
    const half2_t x2 = __builtin_elementwise_fma(mma_magic((v >> 4) & 0x000F000Fu), sc1, ns1);
    const half2_t x3 = __builtin_elementwise_fma(mma_magic((v >> 12) & 0x000F000Fu), sc1, ns1);
    return half8_t{x0.x, x0.y, x1.x, x1.y, x2.x, x2.y, x3.x, x3.y};
}

// eight int8 (two dwords) -> f16 in slot order {0,2,1,3,4,6,5,7}
SXQ_DEV half8_t mma_act8(uint2 v) {
    const half2_t off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    const uint32_t x0 = v.x ^ 0x80808080u, x1 = v.y ^ 0x80808080u;  // u = q + 128
    // byte select: (u0, 0x64, u2, 0x64) = f16 pair (1024 + u0, 1024 + u2)
    const half2_t p0 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, x0, 0x04020400u)) + off;
    const half2_t p1 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, x0, 0x04030401u)) + off;
    const half2_t p2 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, x1, 0x04020400u)) + off;
    const half2_t p3 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, x1, 0x04030401u)) + off;
    return half8_t{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

__global__ __launch_bounds__(512) void k_gemv_mma_q4k(const uint4* __restrict__ hdr, const uint4* __restrict__ qs,
                                                      int n, int nb, const uint8_t* __restrict__ act, int m, float* y,
                                                      int64_t ldy, const float* __restrict__ bias, const float* res,
                                                      int64_t ldr) {
    extern __shared__ uint4 lds[];
    uint32_t* l32 = (uint32_t*)lds;  // [2][kMmaBuf]: weights [16][kMmaWRow], headers [16][4] uint4, act [16][kMmaARow]
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, nl = lane & 15;
    const int row0 = blockIdx.x * kMmaRows;
    const int nc = (nb + kMmaChunk - 1) / kMmaChunk;

    // chunk copy: weight pieces u = tid, tid + 256 of (row u >> 5, 16-byte piece u & 31);
    // header (row tid >> 2, block tid & 3) for tid < 64; activation pieces u = tid + 256k
    // (k < 5, clamped to the 1216 pieces) of (row u / 76, piece u % 76)
    uint4 swq0, sh, sa0, sa1, sa2;  // the chunk in flight
#define SXQ_MMA_WQ(K, V)                                                                   \
    {                                                                                      \
        const int u = tid + 512 * (K), r = min(row0 + (u >> 5), n - 1), p = u & 31;        \
        const int b = min(cc * kMmaChunk + (p >> 3), nb - 1);                             \
        V = qs[((size_t)r * nb + b) * 8 + (p & 7)];                                        \
    }
#define SXQ_MMA_A(K, V)                                                                    \
    {                                                                                      \
        const int u = min(tid + 512 * (K), 16 * 76 - 1), r = min(u / 76, m - 1), p = u % 76; \
        const int b = min(cc * kMmaChunk + p / 19, nb - 1);                              \
        V = ((const uint4*)(act + ((size_t)r * nb + b) * sizeof(ActQ8K)))[p % 19];        \
    }
    auto stage_load = [&](int c) {  // unconditional loads (clamped)
        const int cc = min(c, nc - 1);
        SXQ_MMA_WQ(0, swq0)
        {  // header of (row tid & 15, block (tid >> 6) & 3), decoded for g = (tid >> 4) & 3
            const int r = min(row0 + (tid & 15), n - 1), b = min(cc * kMmaChunk + ((tid >> 6) & 3), nb - 1);
            sh = hdr[(size_t)r * nb + b];
        }
        SXQ_MMA_A(0, sa0) SXQ_MMA_A(1, sa1) SXQ_MMA_A(2, sa2)
    };
#undef SXQ_MMA_WQ
#undef SXQ_MMA_A
    auto stage_store = [&](int c) {
        uint32_t* bw = l32 + (c & 1) * kMmaBuf;
        *(uint4*)(bw + (tid >> 5) * kMmaWRow + (tid & 31) * 4) = swq0;
        if (tid < 256) {  // one decode per (block, g, row) for every wave: scales 2g, 2g + 1 as the
                          // f16 pairs of the W' FMA, d, dmin, mins g and g + 4
            const int gg = (tid >> 4) & 3;
            const uint32_t sc_lo = sh.y & 0x3F3F3F3Fu;
            const uint32_t sc_hi = (sh.w & 0x0F0F0F0Fu) | (((sh.y >> 6) & 0x03030303u) << 4);
            const uint32_t mn_lo = sh.z & 0x3F3F3F3Fu;
            const uint32_t mn_hi = ((sh.w >> 4) & 0x0F0F0F0Fu) | (((sh.z >> 6) & 0x03030303u) << 4);
            const uint32_t scw = (gg < 2 ? sc_lo : sc_hi) >> (16 * (gg & 1));
            const float f0 = (float)(scw & 0xFF), f1 = (float)((scw >> 8) & 0xFF);
            const half2_t sc0 = {(_Float16)f0, (_Float16)f0}, sc1 = {(_Float16)f1, (_Float16)f1};
            const half2_t ns0 = {(_Float16)(-1024.0f * f0), (_Float16)(-1024.0f * f0)};
            const half2_t ns1 = {(_Float16)(-1024.0f * f1), (_Float16)(-1024.0f * f1)};
            uint4* hd = (uint4*)(bw + 16 * kMmaWRow);
            hd[tid] = make_uint4(__builtin_bit_cast(uint32_t, sc0), __builtin_bit_cast(uint32_t, ns0),
                                 __builtin_bit_cast(uint32_t, sc1), __builtin_bit_cast(uint32_t, ns1));
            hd[256 + tid] = make_uint4(__builtin_bit_cast(uint32_t, h2f(sh.x & 0xFFFF)),
                                       __builtin_bit_cast(uint32_t, h2f(sh.x >> 16)),
                                       __builtin_bit_cast(uint32_t, (float)((mn_lo >> (8 * gg)) & 0xFF)),
                                       __builtin_bit_cast(uint32_t, (float)((mn_hi >> (8 * gg)) & 0xFF)));
        }
        uint32_t* ba = bw + 16 * kMmaWRow + kMmaHdr;
        const uint4 v[3] = {sa0, sa1, sa2};
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            const int u = min(tid + 512 * k, 16 * 76 - 1);
            *(uint4*)(ba + (u / 76) * kMmaARow + (u % 76) * 4) = v[k];
        }
    };

    // chains of lane (nl, g), accumulator element e: activation row 4g + e, weight row nl
    float s0c[4] = {0.f, 0.f, 0.f, 0.f}, sf[4] = {0.f, 0.f, 0.f, 0.f};
    stage_load(0);
    stage_store(0);
    stage_load(1);
    __syncthreads();
    for (int c = 0; c < nc; ++c) {
        const uint32_t* bw = l32 + (c & 1) * kMmaBuf;
        const uint4* bh = (const uint4*)(bw + 16 * kMmaWRow);
        const uint32_t* ba = bw + 16 * kMmaWRow + kMmaHdr;
        const int live = min(kMmaChunk, nb - c * kMmaChunk);
#pragma unroll
        for (int j = 0; j < kMmaChunk; ++j) {
            if (j < live) {  // uniform
                const uint4 ha = bh[j * 64 + lane], hb = bh[256 + j * 64 + lane];  // decoded header
                const half2_t sc0 = __builtin_bit_cast(half2_t, ha.x), ns0 = __builtin_bit_cast(half2_t, ha.y);
                const half2_t sc1 = __builtin_bit_cast(half2_t, ha.z), ns1 = __builtin_bit_cast(half2_t, ha.w);
                const uint32_t wq = bw[nl * kMmaWRow + j * 32 + 4 * w + g];             // class w dword g
                const uint2 aq = *(const uint2*)(ba + nl * kMmaARow + j * 76 + 8 * w + 2 * g);  // qs[32w + 8g]
                const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
                const f32x4_t c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    mma_act8(aq), mma_weight8(wq, sc0, ns0, sc1, ns1), z, 0, 0, 0);
                const float dw = __builtin_bit_cast(float, hb.x);
                float ad[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) ad[e] = __builtin_bit_cast(float, ba[(4 * g + e) * kMmaARow + j * 76 + 64]);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float d = dw * ad[e];
                    s0c[e] += d * c0[e];
                }
                if (w == 0) {  // the min term: mins g and g + 4 against bs2 of activation row nl
                    const int* bs = (const int*)(ba + nl * kMmaARow + j * 76 + 68);  // bs2 at byte 272
                    f32x4_t mi = z;
                    mi = __builtin_amdgcn_mfma_f32_16x16x4f32((float)bs[g], __builtin_bit_cast(float, hb.z), mi, 0, 0, 0);
                    mi = __builtin_amdgcn_mfma_f32_16x16x4f32((float)bs[g + 4], __builtin_bit_cast(float, hb.w), mi, 0, 0,
                                                              0);
                    const float dminw = __builtin_bit_cast(float, hb.y);
#pragma unroll
                    for (int e = 0; e < 4; ++e) sf[e] -= (dminw * ad[e]) * mi[e];
                }
            }
        }
        if (c + 1 < nc) stage_store(c + 1);
        stage_load(c + 2);
        __syncthreads();
    }
    // the class sums meet in LDS (chunk buffer 0: every read of it is behind the last
    // barrier): xb[chain][activation row][weight row], chain 0..7 = class, 8 = min
    float* xb = (float*)lds;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int i = (4 * g + e) * 16 + nl;
        xb[w * 256 + i] = s0c[e];
        if (w == 0) xb[8 * 256 + i] = sf[e];
    }
    __syncthreads();
    const int mr = tid >> 4, row = row0 + (tid & 15);
    if (tid < 256 && mr < m && row < n) {
        float tot = -0.0f;
#pragma unroll
        for (int cl = 0; cl < 8; ++cl) tot += xb[cl * 256 + tid];
        float v = xb[8 * 256 + tid] + tot;
        if (bias) v = v + bias[row];
        if (res) v = res[(int64_t)mr * ldr + row] + v;
        y[(int64_t)mr * ldy + row] = v;
    }
}

// The same product with the activation operands read from the quantizers' MmaRec
// records (f16 values already in operand order) instead of staged through LDS and
// converted by every workgroup: per block a wave loads its class's 16 bytes per lane
// from L2, a chunk ahead, into registers.  LDS holds the weights, the decoded headers
// and the records' d and bs of a chunk (double-buffered, 37 KB).  The high nibbles
// stay in place in the W' FMA ((1024 + 16 q) * (sc / 16) - 64 sc = q * sc, exact), and
// full chunks run as straight-line code with the min term in wave 0 only, so the
// scheduler overlaps the blocks.  Same float steps, same bits.
//
// The work is dealt in units: a 16-row tile, or with ks > 1 one of a tile's ks K-slices
// (cpu = ceil(nc / ks) chunks each, chunks past the row's blocks computing nothing).  Each
// workgroup takes the units blockIdx.x, blockIdx.x + gridDim.x, ... and runs their chunks
// as one sequence (step q: unit q / cpu, chunk q % cpu of it), so the loads of a unit's
// first chunks are in flight while the previous unit computes: a unit costs its chunks'
// compute, not a workgroup's start-up and load latency.  A unit's class sums go to LDS
// buffer (unit & 1) after its last chunk and are used after the next barrier; the next
// write to that buffer comes two units later, behind another barrier.  With ks = 1 they
// are added in class order and stored: Candle's chains, the same bits.  With ks > 1 (the
// tiles alone would leave compute units idle) each slice adds its own chains the same
// way into one partial per output, `part` [tile][slice][256], and the tile's last slice
// to arrive (a counter per tile, kCounterStride words apart, reset after use) adds the
// partials in slice order: the same terms in another association (float rounding
// only), in a fixed order (deterministic).
constexpr int kRecBuf = 16 * kMmaWRow + kMmaHdr + kMmaChunk * 128 + kMmaChunk * 16;  // dwords per chunk buffer
constexpr int kRecXb = 9 * 256;  // dwords of one tile's class sums: [chain][activation row][weight row]
constexpr size_t kRecLds = (2 * (size_t)kRecBuf + 2 * (size_t)kRecXb) * 4;

SXQ_DEV half8_t mma_weight8_hi(uint32_t v, half2_t sc0, half2_t ns0, half2_t sc1, half2_t ns1) {
    const uint32_t u = v >> 8;
    const half2_t x0 = __builtin_elementwise_fma(mma_magic(v & 0x000F000Fu), sc0, ns0);
    const half2_t x1 = __builtin_elementwise_fma(mma_magic(u & 0x000F000Fu), sc0, ns0);
    const half2_t x2 = __builtin_elementwise_fma(mma_magic(v & 0x00F000F0u), sc1, ns1);
    const half2_t x3 = __builtin_elementwise_fma(mma_magic(u & 0x00F000F0u), sc1, ns1);
    return half8_t{x0.x, x0.y, x1.x, x1.y, x2.x, x2.y, x3.x, x3.y};
}

constexpr int kRecMaxKs = kGemvRecMaxKs;

__global__ __launch_bounds__(512) void k_gemv_mma_q4k_rec(const uint4* __restrict__ hdr, const uint4* __restrict__ qs,
                                                          int n, int nb, const MmaRec* __restrict__ rec, int m, float* y,
                                                          int64_t ldy, const float* __restrict__ bias, const float* res,
                                                          int64_t ldr, int ks, float* part, unsigned* count) {
    extern __shared__ uint4 lds[];
    __shared__ bool last;
    uint32_t* l32 = (uint32_t*)lds;  // [2][kRecBuf]: weights [16][kMmaWRow], headers [2][256] uint4, bs [4][128], d [4][16]
    float* xbs = (float*)(l32 + 2 * kRecBuf);  // [2][kRecXb]: class sums of a finished unit
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, nl = lane & 15;
    const int nc = (nb + kMmaChunk - 1) / kMmaChunk;
    const int cpu = (nc + ks - 1) / ks;  // chunks per unit
    const int units = (n + kMmaRows - 1) / kMmaRows * ks;
    const int Q = (units - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x * cpu;  // this workgroup's steps
    // A step: the workgroup's unit count u (its parity picks the class-sum buffer), the
    // chunk c within the unit, the unit's tile and K-slice.  Steps advance by adds and
    // compares; the only divisions by cpu and ks are the ones above and here.  Steps
    // past the last one (loads issued ahead) point past the tiles, whose loads clamp.
    struct Step {
        int u, c, tile, sl;
    };
    const int gq = (int)gridDim.x / ks, gr = (int)gridDim.x % ks;
    auto adv = [&](Step s) {
        if (++s.c == cpu) {
            s.c = 0;
            ++s.u;
            s.tile += gq;
            s.sl += gr;
            if (s.sl >= ks) {
                s.sl -= ks;
                ++s.tile;
            }
        }
        return s;
    };
    auto chunk = [&](const Step& s) { return s.sl * cpu + s.c; };  // >= nc: past the row's blocks
    const uint8_t* rb = (const uint8_t*)rec;

    // chunk copy of step s (clamped, so every load is in bounds): weight piece tid (row
    // tid >> 5, 16-byte piece tid & 31); tid < 256: the header of (row tid & 15, block
    // (tid >> 6) & 3); tid 256..383: the records' bs (32 pieces per block); tid 384..399: their d
    uint4 swq0, sx;
    auto stage_load = [&](const Step& s) {
        const int cc = chunk(s), row0 = s.tile * kMmaRows;
        {
            const int r = min(row0 + (tid >> 5), n - 1), p = tid & 31;
            const int b = min(cc * kMmaChunk + (p >> 3), nb - 1);
            swq0 = qs[((size_t)r * nb + b) * 8 + (p & 7)];
        }
        if (tid < 256) {
            const int r = min(row0 + (tid & 15), n - 1), b = min(cc * kMmaChunk + ((tid >> 6) & 3), nb - 1);
            sx = hdr[(size_t)r * nb + b];
        } else if (tid < 384) {
            const int u = tid - 256, b = min(cc * kMmaChunk + (u >> 5), nb - 1);
            sx = ((const uint4*)(rb + (size_t)b * sizeof(MmaRec) + offsetof(MmaRec, bs)))[u & 31];
        } else if (tid < 400) {
            const int u = tid - 384, b = min(cc * kMmaChunk + (u >> 2), nb - 1);
            sx = ((const uint4*)(rb + (size_t)b * sizeof(MmaRec) + offsetof(MmaRec, d)))[u & 3];
        }
    };
    auto stage_store = [&](int q) {
        uint32_t* bw = l32 + (q & 1) * kRecBuf;
        *(uint4*)(bw + (tid >> 5) * kMmaWRow + (tid & 31) * 4) = swq0;
        if (tid < 256) {  // one decode per (block, g, row): scales 2g and 2g + 1 (the latter / 16), d, dmin, mins
            const uint4 sh = sx;
            const int gg = (tid >> 4) & 3;
            const uint32_t sc_lo = sh.y & 0x3F3F3F3Fu;
            const uint32_t sc_hi = (sh.w & 0x0F0F0F0Fu) | (((sh.y >> 6) & 0x03030303u) << 4);
            const uint32_t mn_lo = sh.z & 0x3F3F3F3Fu;
            const uint32_t mn_hi = ((sh.w >> 4) & 0x0F0F0F0Fu) | (((sh.z >> 6) & 0x03030303u) << 4);
            const uint32_t scw = (gg < 2 ? sc_lo : sc_hi) >> (16 * (gg & 1));
            const float f0 = (float)(scw & 0xFF), f1 = (float)((scw >> 8) & 0xFF);
            const half2_t sc0 = {(_Float16)f0, (_Float16)f0};
            const half2_t sc1 = {(_Float16)(f1 * 0.0625f), (_Float16)(f1 * 0.0625f)};  // exact: f1 < 64
            const half2_t ns0 = {(_Float16)(-1024.0f * f0), (_Float16)(-1024.0f * f0)};
            const half2_t ns1 = {(_Float16)(-64.0f * f1), (_Float16)(-64.0f * f1)};
            uint4* hd = (uint4*)(bw + 16 * kMmaWRow);
            hd[tid] = make_uint4(__builtin_bit_cast(uint32_t, sc0), __builtin_bit_cast(uint32_t, ns0),
                                 __builtin_bit_cast(uint32_t, sc1), __builtin_bit_cast(uint32_t, ns1));
            hd[256 + tid] = make_uint4(__builtin_bit_cast(uint32_t, h2f(sh.x & 0xFFFF)),
                                       __builtin_bit_cast(uint32_t, h2f(sh.x >> 16)),
                                       __builtin_bit_cast(uint32_t, (float)((mn_lo >> (8 * gg)) & 0xFF)),
                                       __builtin_bit_cast(uint32_t, (float)((mn_hi >> (8 * gg)) & 0xFF)));
        } else if (tid < 400) {
            ((uint4*)(bw + 16 * kMmaWRow + kMmaHdr))[tid - 256] = sx;  // bs [4][128] floats, then d [4][16]
        }
    };
    // this wave's activation operands of step q's chunk: block j, class w, row nl, slots 8g .. 8g + 7
    auto load_a = [&](const Step& s, half8_t (&A)[kMmaChunk]) {
        const int cc = chunk(s);
#pragma unroll
        for (int j = 0; j < kMmaChunk; ++j) {
            const int b = min(cc * kMmaChunk + j, nb - 1);
            A[j] = __builtin_bit_cast(half8_t, ld_global((const uint4*)&rec[b].q[w][nl][g][0]));
        }
    };
    // chains of lane (nl, g), accumulator element e: activation row 4g + e, weight row nl
    float s0c[4] = {0.f, 0.f, 0.f, 0.f}, sf[4] = {0.f, 0.f, 0.f, 0.f};
    const bool wave0 = __builtin_amdgcn_readfirstlane(w) == 0;
    auto body = [&](int q, const half8_t (&A)[kMmaChunk], int live, auto full, auto w0) {
        const uint32_t* bw = l32 + (q & 1) * kRecBuf;
        const uint4* bh = (const uint4*)(bw + 16 * kMmaWRow);
        const float* bsv = (const float*)(bw + 16 * kMmaWRow + kMmaHdr);
        const float* dv = bsv + kMmaChunk * 128;
#pragma unroll
        for (int j = 0; j < kMmaChunk; ++j) {
            if (decltype(full)::value || j < live) {
                const uint4 ha = bh[j * 64 + lane];
                const half2_t sc0 = __builtin_bit_cast(half2_t, ha.x), ns0 = __builtin_bit_cast(half2_t, ha.y);
                const half2_t sc1 = __builtin_bit_cast(half2_t, ha.z), ns1 = __builtin_bit_cast(half2_t, ha.w);
                const uint32_t wq = bw[nl * kMmaWRow + j * 32 + 4 * w + g];  // class w dword g
                const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
                const f32x4_t c0 =
                    __builtin_amdgcn_mfma_f32_16x16x32_f16(A[j], mma_weight8_hi(wq, sc0, ns0, sc1, ns1), z, 0, 0, 0);
                const float4 ad = *(const float4*)(dv + j * 16 + 4 * g);  // d of activation rows 4g .. 4g + 3
                const float adv[4] = {ad.x, ad.y, ad.z, ad.w};
                if constexpr (decltype(w0)::value) {
                    const uint4 hb = bh[256 + j * 64 + lane];
                    const float dw = __builtin_bit_cast(float, hb.x);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float d = dw * adv[e];
                        s0c[e] += d * c0[e];
                    }
                    // the min term: mins g and g + 4 against bs2 of activation row nl
                    f32x4_t mi = z;
                    mi = __builtin_amdgcn_mfma_f32_16x16x4f32(bsv[j * 128 + nl * 4 + g], __builtin_bit_cast(float, hb.z), mi,
                                                              0, 0, 0);
                    mi = __builtin_amdgcn_mfma_f32_16x16x4f32(bsv[j * 128 + 64 + nl * 4 + g],
                                                              __builtin_bit_cast(float, hb.w), mi, 0, 0, 0);
                    const float dminw = __builtin_bit_cast(float, hb.y);
#pragma unroll
                    for (int e = 0; e < 4; ++e) sf[e] -= (dminw * adv[e]) * mi[e];
                } else {
                    const float dw = ((const float*)(bh + 256 + j * 64 + lane))[0];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float d = dw * adv[e];
                        s0c[e] += d * c0[e];
                    }
                }
            }
        }
    };
    using Yes = std::integral_constant<bool, true>;
    using No = std::integral_constant<bool, false>;
    auto compute = [&](int q, const Step& s, const half8_t (&A)[kMmaChunk]) {
        const int live = min(kMmaChunk, nb - chunk(s) * kMmaChunk);  // <= 0: nothing to add
        if (live == kMmaChunk) {
            if (wave0) body(q, A, live, Yes{}, Yes{});
            else body(q, A, live, Yes{}, No{});
        } else {
            if (wave0) body(q, A, live, No{}, Yes{});
            else body(q, A, live, No{}, No{});
        }
        if (s.c == cpu - 1) {  // the unit's last chunk: its class sums to LDS, fresh chains
            float* xb = xbs + (s.u & 1) * kRecXb;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int i = (4 * g + e) * 16 + nl;
                xb[w * 256 + i] = s0c[e];
                if (w == 0) xb[8 * 256 + i] = sf[e];
                s0c[e] = 0.f;
                sf[e] = 0.f;
            }
        }
    };
    // after the barrier that follows a unit's last chunk (every thread calls it)
    auto finish = [&](const Step& s) {
        if (s.c != cpu - 1) return;
        const float* xb = xbs + (s.u & 1) * kRecXb;
        const int t = s.tile;
        const int mr = tid >> 4, row = t * kMmaRows + (tid & 15);
        const bool out = tid < 256 && mr < m && row < n;
        // the unit's class sums in class order, then the min chain
        float v = 0.0f;
        if (tid < 256) {
            float tot = -0.0f;
#pragma unroll
            for (int cl = 0; cl < 8; ++cl) tot += xb[cl * 256 + tid];
            v = xb[8 * 256 + tid] + tot;
        }
        if (ks > 1) {  // this slice's partials to part; the tile's last slice adds them in slice order
            if (tid < 256) store_agent(part + ((size_t)t * ks + s.sl) * 256 + tid, v);
            if (!publish_and_count(&count[t * kCounterStride], (unsigned)ks, &last)) return;
            if (out) {
                float pv[kRecMaxKs];
#pragma unroll
                for (int k = 0; k < kRecMaxKs; ++k)
                    if (k < ks) pv[k] = load_agent(part + ((size_t)t * ks + k) * 256 + tid);
                v = pv[0];
#pragma unroll
                for (int k = 1; k < kRecMaxKs; ++k)
                    if (k < ks) v += pv[k];
            }
            if (tid == 0) __hip_atomic_store(&count[t * kCounterStride], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (out) {
            if (bias) v = v + bias[row];
            if (res) v = res[(int64_t)mr * ldr + row] + v;
            y[(int64_t)mr * ldy + row] = v;
        }
    };
    // A0 / A1 alternate (the loop runs two steps per trip, so both stay in registers):
    // step q + 1's operands load while step q computes; the weights load two steps ahead
    half8_t A0[kMmaChunk], A1[kMmaChunk];
    Step s0 = {0, 0, (int)blockIdx.x / ks, (int)blockIdx.x % ks}, s1 = adv(s0);  // steps q, q + 1
    stage_load(s0);
    load_a(s0, A0);
    stage_store(0);
    stage_load(s1);
    __syncthreads();
    for (int q = 0; q < Q; q += 2) {
        const Step s2 = adv(s1), s3 = adv(s2);
        load_a(s1, A1);
        compute(q, s0, A0);
        if (q + 1 < Q) stage_store(q + 1);
        stage_load(s2);
        __syncthreads();
        finish(s0);
        if (q + 1 >= Q) break;
        load_a(s2, A0);
        compute(q + 1, s1, A1);
        if (q + 2 < Q) stage_store(q + 2);
        stage_load(s3);
        __syncthreads();
        finish(s1);
        s0 = s2;
        s1 = s3;
    }
}

static hipError_t gemv_mma_launch(const QWeight& w, const void* act, int m, float* y, int64_t ldy, const float* bias,
                                  const float* res, int64_t ldr, hipStream_t s) {
    static const hipError_t attr =
        hipFuncSetAttribute((const void*)k_gemv_mma_q4k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMmaLds);
    if (attr != hipSuccess) return attr;
    const int n = (int)w.n, nb = (int)w.nb;
    hipLaunchKernelGGL(k_gemv_mma_q4k, dim3((unsigned)((n + kMmaRows - 1) / kMmaRows)), dim3(512), kMmaLds, s,
                       (const uint4*)w.hdr, (const uint4*)w.qs, n, nb, (const uint8_t*)act, m, y, ldy, bias, res, ldr);
    return hipGetLastError();
}

static bool gemv_v1() {
    static const bool v1 = getenv("SXQ_GEMV_V1") != nullptr;
    return v1;
}
static bool gemv_mma_on() {
    static const bool mma = [] {
        const char* e = getenv("SXQ_GEMV_MMA");
        return !e || atoi(e) != 0;
    }();
    return mma;
}

// Compute units of the current device (cached per device).
static int gemv_device_cus() {
    static std::atomic<int> cus[64];  // 0 until first asked (threads may race to store the same value)
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int c = cus[dev].load(std::memory_order_relaxed);
    if (c == 0) {
        if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
        cus[dev].store(c, std::memory_order_relaxed);
    }
    return c;
}

bool gemv_rec_fits(const QWeight& w, int m) {
    return !gemv_v1() && gemv_mma_on() && w.dtype == kQ4K && m > 4 && m <= 16 && w.n > 0;
}

hipError_t launch_gemv_rec(const QWeight& w, const void* act, const MmaRec* rec, int m, float* y, int64_t ldy,
                           const float* bias, const float* res, int64_t ldr, hipStream_t s, const GemvRecWs* ws) {
    if (!rec || !gemv_rec_fits(w, m)) return launch_gemv(w, act, m, y, ldy, bias, res, ldr, s);
    static const hipError_t attr =
        hipFuncSetAttribute((const void*)k_gemv_mma_q4k_rec, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kRecLds);
    if (attr != hipSuccess) return attr;
    const int n = (int)w.n, nb = (int)w.nb;
    const int ntiles = (n + kMmaRows - 1) / kMmaRows, nc = (nb + kMmaChunk - 1) / kMmaChunk;
    // Workgroups: two per compute unit (the kernel's occupancy), the units dealt evenly
    // (the fewest workgroups that keep the most units per workgroup).  SXQ_GEMV_REC_WG
    // sets the target count for A/B measurement; 0 = one workgroup per unit.
    int target = 2 * gemv_device_cus();
    if (const char* e = getenv("SXQ_GEMV_REC_WG")) target = atoi(e);
    // K-slices: as many as the tiles leave workgroups for (2 for the 160-tile wo, 3 for
    // w2: 4077 tok/s on the 16-stream step against 4035 with 2 for both and 3804 with 4;
    // SXQ_GEMV_REC_KS sets the count for A/B).  SXQ_BIT_EXACT (read per call): one.
    int ks = 1;
    const char* exact = getenv("SXQ_BIT_EXACT");
    if (ws && ws->part && !(exact && exact[0] != '0') && ntiles <= kGemvRecMaxSplitTiles && target > 0 &&
        2 * ntiles <= target) {
        int want = min(min(kGemvRecMaxKs, nc), target / ntiles);
        if (const char* e = getenv("SXQ_GEMV_REC_KS")) want = min(min(kGemvRecMaxKs, nc), max(1, atoi(e)));
        const int cpu = (nc + want - 1) / want;
        ks = (nc + cpu - 1) / cpu;  // no slice without a chunk
    }
    const int units = ntiles * ks;
    int grid = units;
    if (target > 0 && target < units) {
        const int per = (units + target - 1) / target;
        grid = (units + per - 1) / per;
    }
    hipLaunchKernelGGL(k_gemv_mma_q4k_rec, dim3((unsigned)grid), dim3(512), kRecLds, s, (const uint4*)w.hdr,
                       (const uint4*)w.qs, n, nb, rec, m, y, ldy, bias, res, ldr, ks, ks > 1 ? ws->part : nullptr,
                       ks > 1 ? ws->count : nullptr);
    return hipGetLastError();
}

hipError_t launch_gemv(const QWeight& w, const void* act, int m, float* y, int64_t ldy, const float* bias,
                       const float* res, int64_t ldr, hipStream_t s) {
    if (m <= 0 || w.n <= 0) return hipSuccess;
    if (!gemv_v1()) {
        const int nb = (int)w.nb;
        const bool fits = gemv2_fits((int)w.n, nb, m, w.dtype, 256);
        if (fits && m == 1) return gemv2_dispatch<1>(w, act, m, y, ldy, bias, res, ldr, s);
        if (fits && m == 2) return gemv2_dispatch<2>(w, act, m, y, ldy, bias, res, ldr, s);
        if (fits && m <= 4) return gemv2_dispatch<4>(w, act, m, y, ldy, bias, res, ldr, s);
        // 5..16 rows of Q4_K: one pass over the weights on the matrix cores
        if (w.dtype == kQ4K && m <= 16 && gemv_mma_on()) return gemv_mma_launch(w, act, m, y, ldy, bias, res, ldr, s);
        // 5..16 rows: the task-split kernel four activation rows at a time (each launch
        // streams the weights again; per row this is still well ahead of the
        // one-group-per-row kernel, whose few waves leave most of the GPU idle).
        if (m <= 16 && gemv2_fits((int)w.n, nb, 4, w.dtype, 256)) {
            const size_t row_bytes = (size_t)nb * act_block_bytes(vec_dot_type(w.dtype));
            for (int r0 = 0; r0 < m; r0 += 4) {
                const int mc = min(4, m - r0);
                const void* a = (const uint8_t*)act + (size_t)r0 * row_bytes;
                float* yc = y + (int64_t)r0 * ldy;
                const float* rc = res ? res + (int64_t)r0 * ldr : nullptr;
                const hipError_t e = mc == 1   ? gemv2_dispatch<1>(w, a, mc, yc, ldy, bias, rc, ldr, s)
                                     : mc == 2 ? gemv2_dispatch<2>(w, a, mc, yc, ldy, bias, rc, ldr, s)
                                               : gemv2_dispatch<4>(w, a, mc, yc, ldy, bias, rc, ldr, s);
                if (e != hipSuccess) return e;
            }
            return hipSuccess;
        }
    }
    if (m == 1) return gemv_dispatch<1>(w, act, m, y, ldy, bias, res, ldr, s);
    if (m == 2) return gemv_dispatch<2>(w, act, m, y, ldy, bias, res, ldr, s);
    if (m <= 4) return gemv_dispatch<4>(w, act, m, y, ldy, bias, res, ldr, s);
    if (m <= 8) return gemv_dispatch<8>(w, act, m, y, ldy, bias, res, ldr, s);
    if (m <= 16) return gemv_dispatch<16>(w, act, m, y, ldy, bias, res, ldr, s);
    return hipErrorInvalidValue;
}

// SwiGLU pair sizing: B gate rows per tile so that the tiles spread over one
// workgroup per CU, within the tile limits (2B rows <= NT/8, 2B*nb tasks <= kTmaxQ4k1024 rounds).
static int swiglu_rows(int I, int nb) {
    int B = (I + 255) / 256;
    B = min(B, 1024 / 16);
    B = min(B, max(1, (1024 / kQ4kLanes) * kTmaxQ4k1024 / (2 * nb)));
    return max(B, 1);
}

// Q8_0 / Q4_0 pairs: gate|up tiles over one workgroup per CU, or over two when one per CU
// would take more than kTmax task rounds (w1|w3 19456 x 2560 in Q8_0: 12 rounds on 256
// workgroups, 6 on 512 -- two 1024-thread workgroups of <= 64 VGPRs share a CU; measured
// 539 against 522 tok/s for the Qwen3-4B-shape Q8_0 decode).
static int swiglu_rows_q80(int I, int nb, int dtype) {
    const int tpr = tasks_per_round(dtype, 1024);
    int B = (I + 255) / 256;
    if (2 * B * nb > tpr * kTmax) B = (I + 511) / 512;
    return max(min(B, 1024 / 16), 1);
}

bool swiglu_pair_fits(const QWeight& gate_up, const QWeight& down) {
    const int I = (int)(gate_up.n / 2), nb = (int)gate_up.nb;
    const int dt = gate_up.dtype;
    if (down.dtype != dt || gate_up.n != 2 * (int64_t)I || down.k != I || gate_up.k > kNormMaxDim || I % 256 != 0 ||
        I / 256 > 48 || !gemv2_fits((int)down.n, (int)down.nb, 1, dt, 1024))
        return false;
    if (dt == kQ4K) return 2 * swiglu_rows(I, nb) * nb <= (1024 / kQ4kLanes) * kTmaxQ4k1024;
    if (dt == kQ8_0 || dt == kQ4_0) {
        const int B = swiglu_rows_q80(I, nb, dt);
        return 2 * B * nb <= tasks_per_round(dt, 1024) * kTmax && gemv2_lds(nb, 1, 2 * B, dt, 1024) <= 64 * 1024;
    }
    return false;
}

// The Q8_0 / Q4_0 pair: k_gemv2_q80 with the kProPair prologue and epilogue over the
// gate|up weight, then with the kProQuant prologue over the down weight.
template <bool Q4>
static hipError_t swiglu_pair_q80(const QWeight& gate_up, const QWeight& down, const NormIn& ni, float* gu,
                                  float* act_f32, float* y, const float* res, hipStream_t s) {
    const int dt = gate_up.dtype;
    const int I = (int)(gate_up.n / 2), nb = (int)gate_up.nb;
    const int B = swiglu_rows_q80(I, nb, dt);
    const int tpr = tasks_per_round(dt, 1024);
    const size_t lds1 = gemv2_lds(nb, 1, 2 * B, dt, 1024);
    hipError_t e = with_rounds((2 * B * nb + tpr - 1) / tpr, [&](auto tmc) -> hipError_t {
        constexpr int TM = decltype(tmc)::value;
        if (const hipError_t e_ = allow_lds<k_gemv2_q80<1, Q4, kProPair, 1024, TM>>(lds1); e_ != hipSuccess) return e_;
        hipLaunchKernelGGL((k_gemv2_q80<1, Q4, kProPair, 1024, TM>), dim3((I + B - 1) / B), dim3(1024), lds1, s,
                           (const uint16_t*)gate_up.hdr, (const uint4*)gate_up.qs, I, nb, (const uint8_t*)nullptr, 1,
                           B, gu, (int64_t)0, (const float*)nullptr, (const float*)nullptr, (int64_t)0, ni, act_f32);
        return hipSuccess;
    });
    if (e == hipSuccess) e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int n = (int)down.n, nb2 = (int)down.nb;
    const int R = gemv2_rows(n, nb2, 1, dt, 1024);
    const size_t lds2 = gemv2_lds(nb2, 1, R, dt, 1024);
    NormIn q;
    q.x = act_f32;
    e = with_rounds((R * nb2 + tpr - 1) / tpr, [&](auto tmc) -> hipError_t {
        constexpr int TM = decltype(tmc)::value;
        if (const hipError_t e_ = allow_lds<k_gemv2_q80<1, Q4, kProQuant, 1024, TM>>(lds2); e_ != hipSuccess) return e_;
        hipLaunchKernelGGL((k_gemv2_q80<1, Q4, kProQuant, 1024, TM>), dim3((n + R - 1) / R), dim3(1024), lds2, s,
                           (const uint16_t*)down.hdr, (const uint4*)down.qs, n, nb2, (const uint8_t*)nullptr, 1, R, y,
                           (int64_t)0, (const float*)nullptr, res, (int64_t)0, q, (float*)nullptr);
        return hipSuccess;
    });
    if (e != hipSuccess) return e;
    return hipGetLastError();
}

hipError_t launch_swiglu_pair(const QWeight& gate_up, const QWeight& down, const NormIn& ni, float* gu, float* act_f32,
                              float* y, const float* res, hipStream_t s) {
    if (!swiglu_pair_fits(gate_up, down)) return hipErrorInvalidValue;
    if (gate_up.dtype == kQ8_0) return swiglu_pair_q80<false>(gate_up, down, ni, gu, act_f32, y, res, s);
    if (gate_up.dtype == kQ4_0) return swiglu_pair_q80<true>(gate_up, down, ni, gu, act_f32, y, res, s);
    const int I = (int)(gate_up.n / 2), nb = (int)gate_up.nb;
    const int B = swiglu_rows(I, nb);
    const size_t lds1 = gemv2_lds(nb, 1, 2 * B, kQ4K, 1024);
    const int tpr = tasks_per_round(kQ4K, 1024);
    hipError_t e = with_rounds((2 * B * nb + tpr - 1) / tpr, [&](auto tmc) -> hipError_t {
        constexpr int TM = decltype(tmc)::value;
        if constexpr (TM > kTmaxQ4k1024) {
            return hipErrorInvalidValue;  // (swiglu_rows never asks for it)
        } else {
            hipLaunchKernelGGL(k_gemv2_q4k_swiglu<TM>, dim3((I + B - 1) / B), dim3(1024), lds1, s,
                               (const uint4*)gate_up.hdr, (const uint4*)gate_up.qs, I, nb, B, ni, gu, act_f32);
            return hipSuccess;
        }
    });
    if (e == hipSuccess) e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int n = (int)down.n, nb2 = (int)down.nb;
    const int R = gemv2_rows(n, nb2, 1, kQ4K, 1024);
    const size_t lds2 = gemv2_lds(nb2, 1, R, kQ4K, 1024);
    e = with_rounds((R * nb2 + tpr - 1) / tpr, [&](auto tmc) -> hipError_t {
        constexpr int TM = decltype(tmc)::value;
        if constexpr (TM > kTmaxQ4k1024) {
            return hipErrorInvalidValue;  // (gemv2_rows never asks for it)
        } else {
            hipLaunchKernelGGL(k_gemv2_q4k_quant<TM>, dim3((n + R - 1) / R), dim3(1024), lds2, s,
                               (const uint4*)down.hdr, (const uint4*)down.qs, n, nb2, R, act_f32, y, res);
            return hipSuccess;
        }
    });
    if (e != hipSuccess) return e;
    return hipGetLastError();
}

// Threads per workgroup of the one-row quantizing GEMV: 1024 where it fits (one workgroup
// per CU quantizes the row once; [4864 x 896] Q8_0 per call 5.78 us against 5.97 for the
// quantizer + GEMV launches, 6.04 against 6.13 with 256 threads), else 256 when its four
// waves' three chunks each cover the row.
static int gemv_quant_nt(const QWeight& w) {
    const int n = (int)w.n, nb = (int)w.nb;
    if (nb <= 3 * 16 * 8 && gemv2_fits(n, nb, 1, w.dtype, 1024)) return 1024;
    if (nb <= 3 * 4 * 8 && gemv2_fits(n, nb, 1, w.dtype, 256)) return 256;
    return 0;
}

bool gemv_quant_fits(const QWeight& w) { return (w.dtype == kQ8_0 || w.dtype == kQ4_0) && gemv_quant_nt(w) > 0; }

template <int NT>
static hipError_t gemv_quant_launch(const QWeight& w, const float* x, float* y, const float* bias, const float* res,
                                    hipStream_t s) {
    const int n = (int)w.n, nb = (int)w.nb, dt = w.dtype;
    const int R = gemv2_rows(n, nb, 1, dt, NT);
    const size_t lds = gemv2_lds(nb, 1, R, dt, NT);
    const int tpr = tasks_per_round(dt, NT);
    NormIn q;
    q.x = x;
    const hipError_t e = with_rounds((R * nb + tpr - 1) / tpr, [&](auto tmc) -> hipError_t {
        constexpr int TM = decltype(tmc)::value;
        if (dt == kQ8_0) {
            if (const hipError_t e_ = allow_lds<k_gemv2_q80<1, false, kProQuant, NT, TM>>(lds); e_ != hipSuccess) return e_;
            hipLaunchKernelGGL((k_gemv2_q80<1, false, kProQuant, NT, TM>), dim3((n + R - 1) / R), dim3(NT), lds, s,
                               (const uint16_t*)w.hdr, (const uint4*)w.qs, n, nb, (const uint8_t*)nullptr, 1, R, y,
                               (int64_t)0, bias, res, (int64_t)0, q, (float*)nullptr);
        } else {
            if (const hipError_t e_ = allow_lds<k_gemv2_q80<1, true, kProQuant, NT, TM>>(lds); e_ != hipSuccess) return e_;
            hipLaunchKernelGGL((k_gemv2_q80<1, true, kProQuant, NT, TM>), dim3((n + R - 1) / R), dim3(NT), lds, s,
                               (const uint16_t*)w.hdr, (const uint4*)w.qs, n, nb, (const uint8_t*)nullptr, 1, R, y,
                               (int64_t)0, bias, res, (int64_t)0, q, (float*)nullptr);
        }
        return hipSuccess;
    });
    if (e != hipSuccess) return e;
    return hipGetLastError();
}

hipError_t launch_gemv_quant(const QWeight& w, const float* x, float* y, const float* bias, const float* res,
                             hipStream_t s) {
    if (!gemv_quant_fits(w)) return hipErrorInvalidValue;
    return gemv_quant_nt(w) == 256 ? gemv_quant_launch<256>(w, x, y, bias, res, s)
                                   : gemv_quant_launch<1024>(w, x, y, bias, res, s);
}

hipError_t launch_gemv_rmsnorm(const QWeight& w, const NormIn& ni, int m, uint8_t* act_scratch, float* y,
                               int64_t ldy, const float* bias, const float* res, int64_t ldr, hipStream_t s,
                               MmaRec* rec) {
    if (m <= 0 || w.n <= 0) return hipSuccess;
    const int k = (int)w.k;
    if (!gemv_v1() && m == 1 && k <= kNormMaxDim && gemv2_fits((int)w.n, (int)w.nb, 1, w.dtype, 1024))
        return gemv2_launch<1, true, 1024>(w, nullptr, 1, y, ldy, bias, res, ldr, s, ni);
    if (!gemv_rec_fits(w, m)) rec = nullptr;
    hipError_t e = launch_rmsnorm_quant(vec_dot_type(w.dtype), ni.x, m, k, ni.w, ni.eps, act_scratch, ni.normed, s, rec);
    if (e != hipSuccess) return e;
    return launch_gemv_rec(w, act_scratch, rec, m, y, ldy, bias, res, ldr, s);
}

}  // namespace sxq
