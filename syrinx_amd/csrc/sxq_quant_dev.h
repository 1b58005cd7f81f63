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

// Quantize 256 consecutive activations (lane i holds elements 4i..4i+3 in v) to one
// Q8_K block: k_quants.rs BlockQ8K::from_float.  Writes either the device layout
// (ActQ8K, class-major qs) or the canonical BlockQ8K.
template <bool CANON>
SXQ_DEV void wave_quantize_q8k(float4 v, int lane, void* out) {
    const float x[4] = {v.x, v.y, v.z, v.w};
    // first element of largest magnitude (Candle keeps the first on ties: `amax < |x|`)
    float am = fabsf(x[0]);
    int ix = 0;
#pragma unroll
    for (int r = 1; r < 4; ++r)
        if (am < fabsf(x[r])) { am = fabsf(x[r]); ix = r; }
    const float wmax = wave_max_f32(am);
    const int first = wave_min_i32(am == wmax ? 4 * lane + ix : 256);
    const int src = first >> 2, comp = first & 3;
    const float c0 = __shfl(x[0], src, 64), c1 = __shfl(x[1], src, 64);
    const float c2 = __shfl(x[2], src, 64), c3 = __shfl(x[3], src, 64);
    const float mx = comp == 0 ? c0 : comp == 1 ? c1 : comp == 2 ? c2 : c3;
    int q[4] = {0, 0, 0, 0};
    float d = 0.0f;
    if (wmax != 0.0f) {
        const float iscale = -128.0f / mx;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float t = roundf(iscale * x[r]);
            t = (t != t || t > 127.0f) ? 127.0f : t;  // f32::min(t, 127.0) ignores NaN
            q[r] = sat_i8(t);
        }
        d = 1.0f / iscale;
    }
    // bsums: 16 elements = 4 lanes (a quad); bs2: 32 elements = 8 lanes.
    int s4 = q[0] + q[1] + q[2] + q[3];
    s4 += __shfl_xor(s4, 1, 64);
    s4 += __shfl_xor(s4, 2, 64);
    const int s8 = s4 + __shfl_xor(s4, 4, 64);
    if (CANON) {
        BlockQ8K* b = (BlockQ8K*)out;
        uint32_t packed = (uint32_t)(q[0] & 0xFF) | ((uint32_t)(q[1] & 0xFF) << 8) |
                          ((uint32_t)(q[2] & 0xFF) << 16) | ((uint32_t)(q[3] & 0xFF) << 24);
        ((uint32_t*)b->qs)[lane] = packed;
        if ((lane & 3) == 0) b->bsums[lane >> 2] = (int16_t)s4;
        if (lane == 0) b->d = d;
    } else {
        ActQ8K* b = (ActQ8K*)out;
        // element e = 4*lane + r: j = lane/8, l = 4*(lane%2) + r, t = (lane%8)/2
        const int j = lane >> 3, t = (lane & 7) >> 1, l0 = 4 * (lane & 1);
#pragma unroll
        for (int r = 0; r < 4; ++r) b->qs[4 * (8 * (l0 + r) + j) + t] = (int8_t)q[r];
        if ((lane & 7) == 0) b->bs2[j] = s8;
        if (lane == 0) b->d = d;
    }
}

// Quantize 256 consecutive activations (8 Q8_0 blocks; lanes 8b..8b+7 own block b) to
// Q8_0: k_quants.rs BlockQ8_0::from_float.  `valid` = this lane's block lies inside k.
template <bool CANON>
SXQ_DEV void wave_quantize_q8_0(float4 v, int lane, bool valid, void* out) {
    const float x[4] = {v.x, v.y, v.z, v.w};
    float am = 0.0f;
#pragma unroll
    for (int r = 0; r < 4; ++r) am = fmaxf(am, fabsf(x[r]));
    am = fmaxf(am, __shfl_xor(am, 1, 64));
    am = fmaxf(am, __shfl_xor(am, 2, 64));
    am = fmaxf(am, __shfl_xor(am, 4, 64));
    const float d = am / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    int q[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) q[r] = sat_i8(roundf(x[r] * id));
    const uint16_t dh = f32_to_f16_bits(d);
    int s = q[0] + q[1] + q[2] + q[3];
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    s += __shfl_xor(s, 4, 64);
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
