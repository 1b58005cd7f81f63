// sxq_gemv_dev.h -- one tile of the Q4_K x Q8_K task-split GEMV (k_gemv2_q4k,
// sxq_gemv.hip) as device functions: weight loads, per-task products, in-order fold.
// The results are Candle's vec-dot bit for bit.
//
// A tile is `rows` consecutive weight rows starting at block index blk0 (row-major,
// nb blocks per row); its rows*nb (row, block) tasks are dealt round-robin to the
// NT/kQ4kLanes lane groups of the workgroup, at most kTmax tasks each.  Lane c of a group
// loads the 16 kQ4kCpl bytes holding classes kQ4kCpl c .. (elements = l mod 8) of a
// block's four 32-byte chunks (the device layout of sxq_common.h: class l's 16 bytes at
// 16 l) and produces Candle's aux32[l] for them directly.
#pragma once
#include "sxq_kernels.h"
#include "sxq_quant_dev.h"
#include "sxq_sync_dev.h"

namespace sxq {

constexpr int kTmax = 8;
constexpr int kQ4kLanes = 4;            // lanes per (row, block) task
constexpr int kQ4kCpl = 8 / kQ4kLanes;  // classes per lane
static_assert(kQ4kLanes == 2 || kQ4kLanes == 4 || kQ4kLanes == 8, "a task's lanes share a DPP row");
SXQ_DEV float h2f(uint32_t bits16) { return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16); }

// The integer part of a Q4_K task, aux32[l] = sum_j sc_j * dot_j over the eight
// sub-blocks (exact in any order), as the instructions it should be: the compiler turns
// sdot4(w, a, 0) into an accumulating v_dot4c plus a move of 0 into its destination,
// and extracts each scale byte before multiplying.  Here: eight v_dot4_i32_i8 with c = 0,
// then eight 24-bit multiplies whose scale operand is an SDWA byte select of the packed
// scale word (scale j: byte j of slo for j < 4, byte j - 4 of shi).  One asm block, all
// dots ahead of all multiplies: a dot's result may be read only some cycles after it
// is written (the compiler pads with s_nop when it schedules them), and here each is
// read eight instructions later.  |dot_j| <= 4 * 15 * 128 < 2^23, scales < 2^6.
SXQ_DEV int q4k_aux(const int (&w)[8], const int (&a)[8], int slo, int shi) {
    int d0, d1, d2, d3, d4, d5, d6, d7;
    asm("v_dot4_i32_i8 %0, %8, %16, 0\n\t"
        "v_dot4_i32_i8 %1, %9, %17, 0\n\t"
        "v_dot4_i32_i8 %2, %10, %18, 0\n\t"
        "v_dot4_i32_i8 %3, %11, %19, 0\n\t"
        "v_dot4_i32_i8 %4, %12, %20, 0\n\t"
        "v_dot4_i32_i8 %5, %13, %21, 0\n\t"
        "v_dot4_i32_i8 %6, %14, %22, 0\n\t"
        "v_dot4_i32_i8 %7, %15, %23, 0\n\t"
        "v_mul_i32_i24_sdwa %0, %0, %24 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0\n\t"
        "v_mul_i32_i24_sdwa %1, %1, %24 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1\n\t"
        "v_mul_i32_i24_sdwa %2, %2, %24 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2\n\t"
        "v_mul_i32_i24_sdwa %3, %3, %24 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3\n\t"
        "v_mul_i32_i24_sdwa %4, %4, %25 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0\n\t"
        "v_mul_i32_i24_sdwa %5, %5, %25 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1\n\t"
        "v_mul_i32_i24_sdwa %6, %6, %25 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2\n\t"
        "v_mul_i32_i24_sdwa %7, %7, %25 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3"
        : "=&v"(d0), "=&v"(d1), "=&v"(d2), "=&v"(d3), "=&v"(d4), "=&v"(d5), "=&v"(d6), "=&v"(d7)
        : "v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3]), "v"(w[4]), "v"(w[5]), "v"(w[6]), "v"(w[7]), "v"(a[0]),
          "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5]), "v"(a[6]), "v"(a[7]), "v"(slo), "v"(shi));
    return ((d0 + d1) + (d2 + d3)) + ((d4 + d5) + (d6 + d7));
}

// Issue the weight loads of every task of this thread's group, TM rounds (clamped to
// the last task, so all TM loads are unconditional and in flight together; the tile
// must have at most TM * NT/8 tasks).
template <int NT, int TM = kTmax>
SXQ_DEV void q4k_tile_load(const uint4* __restrict__ hdr, const uint4* __restrict__ qs, uint32_t blk0, int tasks,
                           uint4 (&q)[TM][kQ4kCpl], uint4 (&h)[TM]) {
    constexpr int SLOTS = NT / kQ4kLanes;
    const int c = threadIdx.x % kQ4kLanes, grp = threadIdx.x / kQ4kLanes;
    const char* qbase = (const char*)opaque_ptr(qs) + c * 16 * kQ4kCpl;
    const char* hbase = (const char*)opaque_ptr(hdr);
#pragma unroll
    for (int u = 0; u < TM; ++u) {
        const uint32_t blk = blk0 + (uint32_t)min(u * SLOTS + grp, tasks - 1);
#pragma unroll
        for (int k = 0; k < kQ4kCpl; ++k) q[u][k] = ld_global((const uint4*)(qbase + (blk << 7) + 16 * k));
        h[u] = ld_global((const uint4*)(hbase + (blk << 4)));
    }
    // The weight loads are all issued here: a prologue's arithmetic on its own (earlier)
    // loads would otherwise make them wait, or they would sink behind it.
    issue_point();
}

// The same for a tile of two row segments: tasks [0, seg) are blocks blkA + t, tasks
// [seg, tasks) blocks blkB + (t - seg) (seg a whole number of rows: a multiple of nb,
// so a task's block index within its row is still t mod nb).
template <int NT, int TM = kTmax>
SXQ_DEV void q4k_tile_load2(const uint4* __restrict__ hdr, const uint4* __restrict__ qs, uint32_t blkA, uint32_t blkB,
                            int seg, int tasks, uint4 (&q)[TM][kQ4kCpl], uint4 (&h)[TM]) {
    constexpr int SLOTS = NT / kQ4kLanes;
    const int c = threadIdx.x % kQ4kLanes, grp = threadIdx.x / kQ4kLanes;
    const char* qbase = (const char*)opaque_ptr(qs) + c * 16 * kQ4kCpl;
    const char* hbase = (const char*)opaque_ptr(hdr);
#pragma unroll
    for (int u = 0; u < TM; ++u) {
        const int t = min(u * SLOTS + grp, tasks - 1);
        const uint32_t blk = t < seg ? blkA + (uint32_t)t : blkB + (uint32_t)(t - seg);
#pragma unroll
        for (int k = 0; k < kQ4kCpl; ++k) q[u][k] = ld_global((const uint4*)(qbase + (blk << 7) + 16 * k));
        h[u] = ld_global((const uint4*)(hbase + (blk << 4)));
    }
    issue_point();  // as in q4k_tile_load
}

// Layout of the per-block float products: one chain per (activation row rr, tile row
// r, lane class c = 0..7, plus c = 8 for the min terms), nb floats in block order, at
// pr + ((rr * (RC + 1) + r) * 9 + c) * CS (RC = the tile's row capacity; row RC of each
// activation row is a spare that takes the writes of tasks past the end).  The chain stride CS
// is nb rounded up to 4 floats and then to an odd number of 16-byte units, so that
// chains start 16-byte aligned (the fold reads them as float4) and the eight lane
// classes' writes of one task fall in eight different LDS banks.
SXQ_HD int q4k_chain_stride(int nb) {
    const int q = (nb + 3) >> 2;
    return 4 * (q | 1);
}

// Per-task float products into the chains: the eight class terms (d_w*d_a)*(f32)aux32[l]
// (lane c: classes CPL c .. CPL c + CPL - 1) and the min term (dmin_w*d_a)*(f32)sumi of
// Candle's Q4_K vec-dot, against the LDS activation blocks la [m][nb].  sumi = sum_j
// m_j * bsum_j over the eight sub-blocks is an integer (exact in any order): lane c adds
// sub-blocks CPL c .. CPL c + CPL - 1, the task's lanes' parts meet by DPP.  Task t is tile row t / nb, block t % nb;
// tasks past the end (last round) compute on clamped loads and write into the spare row.
template <int MMAX, int NT, int TM = kTmax>
SXQ_DEV void q4k_tile_products(const uint4 (&q)[TM][kQ4kCpl], const uint4 (&h)[TM], const ActQ8K* la, int nb, int m,
                               int rows, int RC, float* pr) {
    constexpr int SLOTS = NT / kQ4kLanes, CPL = kQ4kCpl;
    const int c = threadIdx.x % kQ4kLanes, grp = threadIdx.x / kQ4kLanes;
    const int CS = q4k_chain_stride(nb), tasks = rows * nb;
    // Tile row and block of task u*SLOTS + grp, stepped by SLOTS each round.
    const uint32_t bstep = (uint32_t)SLOTS % (uint32_t)nb, rstep = (uint32_t)SLOTS / (uint32_t)nb;
    uint32_t b = (uint32_t)grp % (uint32_t)nb, row = (uint32_t)grp / (uint32_t)nb;
#pragma unroll
    for (int u = 0; u < TM; ++u) {
        if (u * SLOTS >= tasks) break;  // uniform: no group has a task in this round
        const uint32_t sc_lo = h[u].y & 0x3F3F3F3Fu;
        const uint32_t sc_hi = (h[u].w & 0x0F0F0F0Fu) | (((h[u].y >> 6) & 0x03030303u) << 4);
        const uint32_t mn_lo = h[u].z & 0x3F3F3F3Fu;
        const uint32_t mn_hi = ((h[u].w >> 4) & 0x0F0F0F0Fu) | (((h[u].z >> 6) & 0x03030303u) << 4);
        // the mins of this lane's sub-blocks j = CPL c + k: byte j of mn_lo (j < 4), j - 4 of mn_hi
        int mk[CPL];
#pragma unroll
        for (int k = 0; k < CPL; ++k) {
            const int j = CPL * c + k;
            mk[k] = (int)(((j < 4 ? mn_lo : mn_hi) >> (8 * (j & 3))) & 0xFF);
        }
        int w4[CPL][8];
#pragma unroll
        for (int k = 0; k < CPL; ++k) {
            const uint4 qq = q[u][k];
            w4[k][0] = (int)(qq.x & 0x0F0F0F0Fu);
            w4[k][1] = (int)((qq.x >> 4) & 0x0F0F0F0Fu);
            w4[k][2] = (int)(qq.y & 0x0F0F0F0Fu);
            w4[k][3] = (int)((qq.y >> 4) & 0x0F0F0F0Fu);
            w4[k][4] = (int)(qq.z & 0x0F0F0F0Fu);
            w4[k][5] = (int)((qq.z >> 4) & 0x0F0F0F0Fu);
            w4[k][6] = (int)(qq.w & 0x0F0F0F0Fu);
            w4[k][7] = (int)((qq.w >> 4) & 0x0F0F0F0Fu);
        }
        const int slo = (int)sc_lo, shi = (int)sc_hi;  // scale of sub-block j: byte j of slo, j - 4 of shi
        const float dw = h2f(h[u].x & 0xFFFF), dminw = h2f(h[u].x >> 16);
        const bool live = row < (uint32_t)rows;
#pragma unroll
        for (int r = 0; r < MMAX; ++r) {
            if (r < m) {
                const ActQ8K& a = la[r * nb + (int)b];
                // a task past the end writes into the spare row RC (never folded)
                float* p = pr + ((r * (RC + 1) + (live ? (int)row : RC)) * 9) * CS + (int)b;
                const float ad = a.d;
#pragma unroll
                for (int k = 0; k < CPL; ++k) {
                    const int l = CPL * c + k;
                    const uint4 A0 = ((const uint4*)a.qs)[2 * l];
                    const uint4 A1 = ((const uint4*)a.qs)[2 * l + 1];
                    const int Aj[8] = {(int)A0.x, (int)A0.y, (int)A0.z, (int)A0.w,
                                       (int)A1.x, (int)A1.y, (int)A1.z, (int)A1.w};
                    const int aux = q4k_aux(w4[k], Aj, slo, shi);
                    p[l * CS] = (dw * ad) * (float)aux;
                }
                int sumi = 0;
#pragma unroll
                for (int k = 0; k < CPL; ++k) sumi += __mul24(mk[k], a.bs2[CPL * c + k]);
                // the task's lanes (adjacent, within one DPP row)
                if constexpr (kQ4kLanes >= 2) sumi += dpp_i32<0xB1>(sumi);
                if constexpr (kQ4kLanes >= 4) sumi += dpp_i32<0x4E>(sumi);
                if constexpr (kQ4kLanes >= 8) sumi += dpp_i32<0x141>(sumi);
                if (c == 0) p[8 * CS] = (dminw * ad) * (float)sumi;
            }
        }
        b += bstep;
        row += rstep;
        if (b >= (uint32_t)nb) {
            b -= (uint32_t)nb;
            row += 1;
        }
    }
}

// Fold of activation row rr: thread (tile row r = tid/8, lane class l) sums its lane
// chain in block order, and (every lane, the same values) the min terms; the eight lane
// sums are then added in Candle's order.  The chains are sequential float adds: each is
// read as float4s, sixteen blocks ahead of their adds, and the lane sums reach lane
// class 0 by DPP row shifts (lane j of the group -> lane 0) rather than LDS permutes.
// Blocks past nb in a chain's last step are added as +0.0: adding +0.0
// leaves both chains' bits unchanged (the lane chain starts at +0.0, and a
// round-to-nearest sum that starts at +0.0 is never -0.0; x - (+0.0) is x).  Every
// thread calls it; the result (sumf + (-0.0 + sums[0] + ... + sums[7])) is valid in lane
// class 0 of rows < rows.
SXQ_DEV float q4k_tile_fold(const float* pr, int nb, int RC, int rr, int rows) {
    const int l = threadIdx.x & 7, r = threadIdx.x >> 3;
    const int CS = q4k_chain_stride(nb), nv = (nb + 3) >> 2;
    float sl = 0.0f, sf = 0.0f;
    if (r < rows) {
        const float4* cl = (const float4*)(pr + ((rr * (RC + 1) + r) * 9 + l) * CS);
        const float4* cm = (const float4*)(pr + ((rr * (RC + 1) + r) * 9 + 8) * CS);
        // sixteen blocks per step; only a step that runs past nb needs its blocks masked
        for (int v0 = 0; v0 < nv; v0 += 4) {
            float ta[16], tm[16];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int v = min(v0 + j, nv - 1);  // clamped: read, not added
                const float4 x = cl[v], y = cm[v];
                ta[4 * j] = x.x, ta[4 * j + 1] = x.y, ta[4 * j + 2] = x.z, ta[4 * j + 3] = x.w;
                tm[4 * j] = y.x, tm[4 * j + 1] = y.y, tm[4 * j + 2] = y.z, tm[4 * j + 3] = y.w;
            }
            if (4 * v0 + 16 <= nb) {  // uniform
#pragma unroll
                for (int k = 0; k < 16; ++k) {
                    sl += ta[k];
                    sf -= tm[k];
                }
            } else {
#pragma unroll
                for (int k = 0; k < 16; ++k) {
                    const bool in = 4 * v0 + k < nb;  // uniform
                    sl += in ? ta[k] : 0.0f;
                    sf -= in ? tm[k] : 0.0f;
                }
            }
        }
    }
    float tot = -0.0f + sl;
    tot += dpp_f32<0x101>(sl);  // row_shl:j -- lane i reads lane i + j of its row of 16
    tot += dpp_f32<0x102>(sl);
    tot += dpp_f32<0x103>(sl);
    tot += dpp_f32<0x104>(sl);
    tot += dpp_f32<0x105>(sl);
    tot += dpp_f32<0x106>(sl);
    tot += dpp_f32<0x107>(sl);
    return sf + tot;
}

// RMSNorm + activation quantization as the prologue of a 1024-thread GEMV (one row of
// dim <= 4096): thread t holds float4 t of the row and of the norm weight, i.e. lane
// t%64's share of 256-element chunk t/64, so wave w normalises and quantizes chunk w
// straight from registers into the LDS activation blocks.  The row's sum of squares is
// rmsnorm_sumsq_1024 -- the same function and order as k_rmsnorm_quant -- so both paths
// produce the same bits.
SXQ_DEV void norm_fetch(float4& xv, float4& wv, const NormIn& ni, int dim) {
    const int i = min((int)threadIdx.x, dim / 4 - 1);  // clamped: every load in bounds
    xv = ld_global((const float4*)opaque_ptr(ni.x) + i);
    wv = ld_global((const float4*)opaque_ptr(ni.w) + i);
    issue_point();  // keep these loads ahead of the weight loads
}
template <int VDT>
SXQ_DEV void norm_quant_store(const float4& xv, const float4& wv, const NormIn& ni, int dim, uint8_t* lds_act,
                              float* red) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool mine = tid < dim / 4;
    float ss = 0.0f;
    if (mine) {
        ss += xv.x * xv.x;
        ss += xv.y * xv.y;
        ss += xv.z * xv.z;
        ss += xv.w * xv.w;
    }
    ss = rmsnorm_sumsq_1024(ss, red);
    const float var = ss * (float)(1.0 / (double)dim) + 0.0f;
    const float den = sqrtf(var * 1.0f + ni.eps);
    const int nchunks = (dim + 255) / 256;
    if (wave >= nchunks) return;  // uniform per wave
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (mine) {
        v.x = (xv.x / den) * wv.x;
        v.y = (xv.y / den) * wv.y;
        v.z = (xv.z / den) * wv.z;
        v.w = (xv.w / den) * wv.w;
        if (ni.normed && blockIdx.x == 0) ((float4*)ni.normed)[tid] = v;
    }
    if (VDT == kQ8K) {
        wave_quantize_q8k<false>(v, lane, lds_act + (size_t)wave * sizeof(ActQ8K));
    } else {
        wave_quantize_q8_0<false>(v, lane, wave * 8 + (lane >> 3) < dim / 32, lds_act + (size_t)wave * 8 * sizeof(ActQ8_0));
    }
}

}  // namespace sxq
