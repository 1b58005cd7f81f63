// sxq_quant_dev.h -- wave-level activation quantizers shared by the GEMV path and the
// decoder glue kernels (device code, header-only).
//
// They restate candle-core 0.8 k_quants.rs BlockQ8K::from_float and
// BlockQ8_0::from_float (the activation quantization QMatMul performs before its
// vec-dot; call site crates/syrinx-lm/src/cv2/mod.rs:197) operation for operation.
#pragma once
#include "sxq_common.h"

namespace sxq {

// ---------------------------------------------------------------------------------
// Wave-wide helpers (64 lanes).
SXQ_DEV float wave_max_f32(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
SXQ_DEV int wave_min_i32(int v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = min(v, __shfl_xor(v, o, 64));
    return v;
}

// Workgroup barrier that waits only for this wave's LDS accesses (lgkmcnt(0)), not for
// its global loads: __syncthreads() waits for every outstanding load, so a GEMV's
// weight loads issued ahead of it would all have to land before anything after it ran.
SXQ_DEV void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt not waited for
    asm volatile("s_barrier" ::: "memory");
}

// In-row DPP steps (lanes combine inside 16-lane rows): quad_perm xor1 = 0xB1,
// xor2 = 0x4E, row_half_mirror = 0x141 (i <-> 7-i), row_mirror = 0x140 (i <-> 15-i).
// After xor1 and xor2 every quad holds its quad total; the half mirror then pairs each
// lane with the other quad of its 8, and the row mirror with the other 8 of its 16, so
// for max/min/integer sums the four steps leave every lane with its 16-lane total.
template <int CTRL>
SXQ_DEV float dpp_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
SXQ_DEV int dpp_i32(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false); }

// Wave-wide sum / max through DPP (xor 1, xor 2, the other quad of 8, the other 8 of 16:
// every lane then holds its 16-lane row total) and the four row totals read as scalars,
// (r0 + r1) + (r2 + r3).  Every lane gets the same value; wave-uniform control flow only.
SXQ_DEV float row_total(float v, int r) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16 * r)); }
SXQ_DEV float wave_sum_rows(float v) {
    v += dpp_f32<0xB1>(v);
    v += dpp_f32<0x4E>(v);
    v += dpp_f32<0x141>(v);
    v += dpp_f32<0x140>(v);
    return (row_total(v, 0) + row_total(v, 1)) + (row_total(v, 2) + row_total(v, 3));
}
SXQ_DEV float wave_max_rows(float v) {
    v = fmaxf(v, dpp_f32<0xB1>(v));
    v = fmaxf(v, dpp_f32<0x4E>(v));
    v = fmaxf(v, dpp_f32<0x141>(v));
    v = fmaxf(v, dpp_f32<0x140>(v));
    return fmaxf(fmaxf(row_total(v, 0), row_total(v, 1)), fmaxf(row_total(v, 2), row_total(v, 3)));
}

// Sum of one f32 per thread over a 1024-thread workgroup, in a fixed order: each wave's
// sum as wave_sum_rows, then the sixteen wave sums as a balanced pairwise tree.  This
// is the RMSNorm sum of squares of every kernel here (fused GEMV prologue and the
// standalone RMSNorm), so they agree bit for bit.  `red`: 16 floats of LDS.  Every
// thread of the workgroup must call it (it synchronises, on LDS only).
SXQ_DEV float rmsnorm_sumsq_1024(float ss, float* red) {
    ss = wave_sum_rows(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    lds_barrier();
    float t[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) t[i] = red[2 * i] + red[2 * i + 1];
    return ((t[0] + t[1]) + (t[2] + t[3])) + ((t[4] + t[5]) + (t[6] + t[7]));
}

// Round half away from zero (Rust's f32::round) of a finite or NaN value.
SXQ_DEV float round_away(float t) { return roundf(t); }

// Quantize J chunks of 256 consecutive activations at once (lane i holds elements
// 4i..4i+3 of chunk j in v[j]) to Q8_K blocks: k_quants.rs BlockQ8K::from_float.  The
// chunks' steps are interleaved so their cross-lane latencies overlap; chunk j is
// written only if `valid[j]` (wave-uniform).  Writes the device layout (ActQ8K,
// class-major qs) or the canonical BlockQ8K.
//
// Candle's loop keeps the first element of largest magnitude (`amax < |x|`, so NaN is
// never taken and ties go to the lower index): here the magnitude maximum is a max
// over lanes (NaN-ignoring maxNum starting from 0, as amax starts at 0), and the first
// element reaching it is found by a ballot over lanes and an in-lane scan.  The
// quantized value is min(round(iscale * x), 127) (f32::min: NaN -> 127), which lies in
// [-128, 127] (|iscale * x| <= 128 up to rounding) and so converts without saturation.
//
// `rec` (optional, J pointers, each may be null): also write chunk j's values into row
// `rec_row` of its matrix-core operand record.
template <int J, bool CANON>
SXQ_DEV void wave_quantize_q8k_n(const float4 (&v)[J], int lane, void* const (&out)[J], const bool (&valid)[J],
                                 MmaRec* const* rec = nullptr, int rec_row = 0) {
    float x[J][4], am[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        x[j][0] = v[j].x; x[j][1] = v[j].y; x[j][2] = v[j].z; x[j][3] = v[j].w;
        am[j] = fmaxf(fmaxf(fmaxf(fmaxf(0.0f, fabsf(x[j][0])), fabsf(x[j][1])), fabsf(x[j][2])), fabsf(x[j][3]));
    }
    // wave maximum of |x|: DPP inside 16-lane rows, then the four row maxima as scalars
    // (am is a non-negative float, never NaN, so it orders like its bit pattern and the
    // steps are integer maxima, one DPP instruction each)
    uint32_t wm[J];
#pragma unroll
    for (int j = 0; j < J; ++j) wm[j] = __builtin_bit_cast(uint32_t, am[j]);
#pragma unroll
    for (int j = 0; j < J; ++j) wm[j] = max(wm[j], (uint32_t)dpp_i32<0xB1>((int)wm[j]));
#pragma unroll
    for (int j = 0; j < J; ++j) wm[j] = max(wm[j], (uint32_t)dpp_i32<0x4E>((int)wm[j]));
#pragma unroll
    for (int j = 0; j < J; ++j) wm[j] = max(wm[j], (uint32_t)dpp_i32<0x141>((int)wm[j]));
#pragma unroll
    for (int j = 0; j < J; ++j) wm[j] = max(wm[j], (uint32_t)dpp_i32<0x140>((int)wm[j]));
    uint32_t wmax[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)wm[j], 0);
        const uint32_t r1 = (uint32_t)__builtin_amdgcn_readlane((int)wm[j], 16);
        const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)wm[j], 32);
        const uint32_t r3 = (uint32_t)__builtin_amdgcn_readlane((int)wm[j], 48);
        wmax[j] = max(max(r0, r1), max(r2, r3));
    }
    // the signed maximum element of each chunk: the first element with |x| == w, i.e. the
    // lowest lane holding one, then its first (selects from the last element back, no branch)
    float mx[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const float w = __builtin_bit_cast(float, wmax[j]);
        float mine = x[j][3];
        mine = fabsf(x[j][2]) == w ? x[j][2] : mine;
        mine = fabsf(x[j][1]) == w ? x[j][1] : mine;
        mine = fabsf(x[j][0]) == w ? x[j][0] : mine;
        const uint64_t hit = __ballot(am[j] == w);
        const int src = hit ? __builtin_ctzll(hit) : 0;
        mx[j] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mine), src));
    }
    // iscale = -128 / max and d = 1 / iscale of the J chunks in one pair of divisions: chunk
    // j's max in lane j (the other lanes divide a copy, never read)
    float mxv = mx[0];
#pragma unroll
    for (int j = 1; j < J; ++j) mxv = lane == j ? mx[j] : mxv;
    const float isv = -128.0f / mxv;
    const float dv = 1.0f / isv;
    int q[J][4];
    float d[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        q[j][0] = q[j][1] = q[j][2] = q[j][3] = 0;
        d[j] = 0.0f;
        if (wmax[j] != 0u) {  // uniform
            const float iscale = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, isv), j));
#pragma unroll
            for (int r = 0; r < 4; ++r) q[j][r] = (int)fminf(round_away(iscale * x[j][r]), 127.0f);
            d[j] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, dv), j));
        }
    }
#pragma unroll
    for (int j = 0; j < J; ++j) {
        if (!valid[j]) continue;
        const uint32_t packed = (uint32_t)(q[j][0] & 0xFF) | ((uint32_t)(q[j][1] & 0xFF) << 8) |
                                ((uint32_t)(q[j][2] & 0xFF) << 16) | ((uint32_t)(q[j][3] & 0xFF) << 24);
        // bsums: 16 elements = 4 lanes (a quad); bs2: 32 elements = 8 lanes
        int s4 = __builtin_amdgcn_sdot4((int)packed, 0x01010101, 0, false);
        s4 += dpp_i32<0xB1>(s4);
        s4 += dpp_i32<0x4E>(s4);
        if (CANON) {
            BlockQ8K* b = (BlockQ8K*)out[j];
            ((uint32_t*)b->qs)[lane] = packed;
            if ((lane & 3) == 0) b->bsums[lane >> 2] = (int16_t)s4;
            if (lane == 0) b->d = d[j];
        } else {
            const int s8 = s4 + dpp_i32<0x141>(s4);
            ActQ8K* b = (ActQ8K*)out[j];
            // element e = 4*lane + r: sub-block jj = lane/8, class l = 4*(lane%2) + r, t = (lane%8)/2
            const int jj = lane >> 3, t = (lane & 7) >> 1, l0 = 4 * (lane & 1);
#pragma unroll
            for (int r = 0; r < 4; ++r) b->qs[4 * (8 * (l0 + r) + jj) + t] = (int8_t)q[j][r];
            if ((lane & 7) == 0) b->bs2[jj] = s8;
            if (lane == 0) b->d = d[j];
            if (rec && rec[j]) {
                // element 4*lane + r: class l0 + r, lane group jj / 2, slot 4 (jj % 2) + {0,2,1,3}[t]
                MmaRec* R = rec[j];
                const int g = jj >> 1, slot = 4 * (jj & 1) + ((t & 1) << 1) + (t >> 1);
#pragma unroll
                for (int r = 0; r < 4; ++r) R->q[l0 + r][rec_row][g][slot] = (_Float16)(float)q[j][r];
                if ((lane & 7) == 0) R->bs[jj >> 2][rec_row][jj & 3] = (float)s8;
                if (lane == 0) R->d[rec_row] = d[j];
            }
        }
    }
}

// One chunk: see wave_quantize_q8k_n.
template <bool CANON>
SXQ_DEV void wave_quantize_q8k(float4 v, int lane, void* out, MmaRec* rec = nullptr, int rec_row = 0) {
    const float4 vv[1] = {v};
    void* const oo[1] = {out};
    const bool ok[1] = {true};
    MmaRec* const rr[1] = {rec};
    wave_quantize_q8k_n<1, CANON>(vv, lane, oo, ok, rr, rec_row);
}

// Quantize 256 consecutive activations (8 Q8_0 blocks; lanes 8b..8b+7 own block b) to
// Q8_0: k_quants.rs BlockQ8_0::from_float.  `valid` = this lane's block lies inside k.
template <bool CANON>
SXQ_DEV void wave_quantize_q8_0(float4 v, int lane, bool valid, void* out) {
    const float x[4] = {v.x, v.y, v.z, v.w};
    float am = 0.0f;
#pragma unroll
    for (int r = 0; r < 4; ++r) am = fmaxf(am, fabsf(x[r]));
    am = fmaxf(am, dpp_f32<0xB1>(am));   // xor 1
    am = fmaxf(am, dpp_f32<0x4E>(am));   // xor 2
    am = fmaxf(am, dpp_f32<0x141>(am));  // the other quad of the 8: the 8-lane max
    const float d = am / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    int q[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) q[r] = sat_i8(roundf(x[r] * id));
    const uint16_t dh = f32_to_f16_bits(d);
    int s = q[0] + q[1] + q[2] + q[3];
    s += dpp_i32<0xB1>(s);
    s += dpp_i32<0x4E>(s);
    s += dpp_i32<0x141>(s);
    if (!valid) return;
    const int blk = lane >> 3, w = lane & 7;
    const uint32_t packed = (uint32_t)(q[0] & 0xFF) | ((uint32_t)(q[1] & 0xFF) << 8) |
                            ((uint32_t)(q[2] & 0xFF) << 16) | ((uint32_t)(q[3] & 0xFF) << 24);
    if (CANON) {
        // 34-byte blocks are only 2-byte aligned: write halves.
        BlockQ8_0* b = (BlockQ8_0*)out + blk;
        uint16_t* qs16 = (uint16_t*)b->qs;
        qs16[2 * w] = (uint16_t)(packed & 0xFFFF);
        qs16[2 * w + 1] = (uint16_t)(packed >> 16);
        if (w == 0) b->d = dh;
    } else {
        ActQ8_0* b = (ActQ8_0*)out + blk;
        ((uint32_t*)b->qs)[w] = packed;
        if (w == 0) {
            b->d = f16_bits_to_f32(dh);
            b->asum = s;
        }
    }
}

}  // namespace sxq
