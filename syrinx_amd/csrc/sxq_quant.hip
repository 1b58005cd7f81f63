// sxq_quant.hip -- block quantizers, dequantizers, weight repacking and the synthetic
// weight generator for gfx950.
//
// Bit-exactness: every float operation below is the one candle-core 0.8's CPU code
// performs (k_quants.rs from_float/to_float; utils.rs make_qkx1_quants), in the same
// order, compiled with -ffp-contract=off and IEEE division/sqrt, so results match the
// CPU byte for byte.  Call sites in the reference: QTensor::quantize at
// crates/syrinx-lm/src/cv2/load.rs:102, QTensor::dequantize at
// crates/syrinx-vocoder/src/cv2/mod.rs:172.
#include "sxq_kernels.h"
#include "sxq_quant_dev.h"

namespace sxq {

// Activation quantization kernel: rows x [m, k] (row stride ldx floats) -> blocks.
// One wave per 256-element chunk.  out_canon: canonical Candle blocks [m][k/bs];
// otherwise the device layout ActQ8K/ActQ8_0 [m][k/bs].
template <int VDT, bool CANON>
__global__ __launch_bounds__(256) void k_quantize_act(const float* __restrict__ x, int64_t ldx, int m,
                                                      int k, void* __restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int chunk = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int chunks_per_row = (k + 255) / 256;
    const int row = blockIdx.y;
    if (row >= m || chunk >= chunks_per_row) return;
    const int e0 = chunk * 256 + 4 * lane;
    const float* xr = x + (int64_t)row * ldx;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (e0 < k) v = *(const float4*)(xr + e0);  // k is a multiple of 32, so 4 | k
    if (VDT == kQ8K) {
        const int nb = k / 256;
        char* base = (char*)out + ((int64_t)row * nb + chunk) * (CANON ? sizeof(BlockQ8K) : sizeof(ActQ8K));
        wave_quantize_q8k<CANON>(v, lane, base);
    } else {
        const int nb = k / 32;
        const int blk0 = chunk * 8;
        char* base = (char*)out + ((int64_t)row * nb + blk0) * (CANON ? sizeof(BlockQ8_0) : sizeof(ActQ8_0));
        wave_quantize_q8_0<CANON>(v, lane, blk0 + (lane >> 3) < nb, base);
    }
}

hipError_t launch_quantize_act(int vdt, bool canon, const float* x, int64_t ldx, int m, int k, void* out,
                               hipStream_t s) {
    const int chunks = (k + 255) / 256;
    dim3 grid((chunks + 3) / 4, m);
    if (vdt == kQ8K) {
        if (canon) hipLaunchKernelGGL((k_quantize_act<kQ8K, true>), grid, dim3(256), 0, s, x, ldx, m, k, out);
        else hipLaunchKernelGGL((k_quantize_act<kQ8K, false>), grid, dim3(256), 0, s, x, ldx, m, k, out);
    } else {
        if (canon) hipLaunchKernelGGL((k_quantize_act<kQ8_0, true>), grid, dim3(256), 0, s, x, ldx, m, k, out);
        else hipLaunchKernelGGL((k_quantize_act<kQ8_0, false>), grid, dim3(256), 0, s, x, ldx, m, k, out);
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------
// Weight from_float (QTensor::quantize on the device), canonical output.
__global__ void k_from_float_q8_0(const float* __restrict__ x, int64_t nblocks, BlockQ8_0* __restrict__ out) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const float* xb = x + b * 32;
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(xb[i]));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint8_t tmp[34];
    const uint16_t dh = f32_to_f16_bits(d);
    tmp[0] = dh & 0xFF;
    tmp[1] = dh >> 8;
    for (int i = 0; i < 32; ++i) tmp[2 + i] = (uint8_t)(int8_t)sat_i8(roundf(xb[i] * id));
    uint8_t* o = (uint8_t*)(out + b);
    for (int i = 0; i < 34; ++i) o[i] = tmp[i];
}

__global__ void k_from_float_q4_0(const float* __restrict__ x, int64_t nblocks, BlockQ4_0* __restrict__ out) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const float* xb = x + b * 32;
    float amax = 0.0f, mx = 0.0f;
    for (int i = 0; i < 32; ++i) {
        const float a = fabsf(xb[i]);
        if (amax < a) { amax = a; mx = xb[i]; }
    }
    const float d = mx / -8.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint8_t tmp[18];
    const uint16_t dh = f32_to_f16_bits(d);
    tmp[0] = dh & 0xFF;
    tmp[1] = dh >> 8;
    for (int j = 0; j < 16; ++j) {
        // Rust `(x + 8.5) as u8`: truncate toward zero, saturating at 0 and 255.
        float v0 = xb[j] * id + 8.5f, v1 = xb[16 + j] * id + 8.5f;
        int a0 = v0 != v0 ? 0 : (v0 <= 0.0f ? 0 : (v0 >= 255.0f ? 255 : (int)v0));
        int a1 = v1 != v1 ? 0 : (v1 <= 0.0f ? 0 : (v1 >= 255.0f ? 255 : (int)v1));
        a0 = a0 > 15 ? 15 : a0;
        a1 = a1 > 15 ? 15 : a1;
        tmp[2 + j] = (uint8_t)(a0 | (a1 << 4));
    }
    uint8_t* o = (uint8_t*)(out + b);
    for (int i = 0; i < 18; ++i) o[i] = tmp[i];
}

// make_qkx1_quants(15, 5, x[32]) for one Q4_K sub-block (utils.rs): one thread runs the
// sequential algorithm so every float sum has Candle's order.
SXQ_DEV int nearest_int(float v) {
    const float r = roundf(v);
    return r != r ? 0 : (r >= 2147483647.0f ? 2147483647 : (r <= -2147483648.0f ? (int)0x80000000u : (int)r));
}
SXQ_DEV int total_key(float f) {
    int a = __builtin_bit_cast(int, f);
    return a ^ (int)(((unsigned)(a >> 31)) >> 1);
}
SXQ_DEV void make_qkx1_quants(const float* x, float* scale_out, float* min_out) {
    const int n = 32, nmax = 15;
    uint8_t L[32];
    for (int i = 0; i < n; ++i) L[i] = 0;
    float mn = x[0], mx = x[0];
    for (int i = 0; i < n; ++i) {
        const int k = total_key(x[i]);
        if (k < total_key(mn)) mn = x[i];
        if (k >= total_key(mx)) mx = x[i];
    }
    if (mx == mn) {
        *scale_out = 0.0f;
        *min_out = 0.0f;
        return;
    }
    float min = fminf(mn, 0.0f);
    float iscale = (float)nmax / (mx - min);
    float scale = 1.0f / iscale;
    for (int it = 0; it < 5; ++it) {
        float sumlx = 0.0f;
        int suml2 = 0;
        bool changed = false;
        for (int i = 0; i < n; ++i) {
            int li = nearest_int(iscale * (x[i] - min));
            li = li < 0 ? 0 : (li > nmax ? nmax : li);
            if ((uint8_t)li != L[i]) {
                L[i] = (uint8_t)li;
                changed = true;
            }
            sumlx += (x[i] - min) * (float)li;
            suml2 += li * li;
        }
        scale = sumlx / (float)suml2;
        float sum = -0.0f;
        for (int i = 0; i < n; ++i) sum += x[i] - scale * (float)L[i];
        min = sum / (float)n;
        if (min > 0.0f) min = 0.0f;
        iscale = 1.0f / scale;
        if (!changed) break;
    }
    *scale_out = scale;
    *min_out = -min;
}

SXQ_DEV void get_scale_min_k4(int j, const uint8_t* q, int& d, int& m) {
    if (j < 4) {
        d = q[j] & 63;
        m = q[j + 4] & 63;
    } else {
        d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

// One workgroup of 256 threads per Q4_K super-block: threads 0..7 run make_qkx1_quants
// on the 8 sub-blocks, thread 0 packs scales/d/dmin, then every thread quantizes one
// element (each element's level is independent).
__global__ __launch_bounds__(256) void k_from_float_q4k(const float* __restrict__ x, BlockQ4K* __restrict__ out) {
    __shared__ float s_scale[8], s_min[8];
    __shared__ uint8_t s_hdr[16];
    __shared__ uint8_t s_L[256];
    const int64_t b = blockIdx.x;
    const float* xb = x + b * 256;
    const int t = threadIdx.x;
    if (t < 8) {
        float xs[32];
        for (int i = 0; i < 32; ++i) xs[i] = xb[32 * t + i];
        make_qkx1_quants(xs, &s_scale[t], &s_min[t]);
    }
    __syncthreads();
    if (t == 0) {
        float max_scale = 0.0f, max_min = 0.0f;
        for (int j = 0; j < 8; ++j) {
            max_scale = fmaxf(s_scale[j], max_scale);
            max_min = fmaxf(s_min[j], max_min);
        }
        const float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
        const float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
        uint8_t sc[12];
        for (int j = 0; j < 12; ++j) sc[j] = 0;
        for (int j = 0; j < 8; ++j) {
            const int lsi = nearest_int(inv_scale * s_scale[j]);
            const int lmi = nearest_int(inv_min * s_min[j]);
            const uint8_t ls = (uint8_t)(lsi < 63 ? lsi : 63);
            const uint8_t lm = (uint8_t)(lmi < 63 ? lmi : 63);
            if (j < 4) {
                sc[j] = ls;
                sc[j + 4] = lm;
            } else {
                sc[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
                sc[j - 4] |= (uint8_t)((ls >> 4) << 6);
                sc[j] |= (uint8_t)((lm >> 4) << 6);
            }
        }
        const uint16_t dh = f32_to_f16_bits(max_scale / 63.0f);
        const uint16_t mh = f32_to_f16_bits(max_min / 63.0f);
        s_hdr[0] = dh & 0xFF;
        s_hdr[1] = dh >> 8;
        s_hdr[2] = mh & 0xFF;
        s_hdr[3] = mh >> 8;
        for (int j = 0; j < 12; ++j) s_hdr[4 + j] = sc[j];
    }
    __syncthreads();
    {
        const int j = t >> 5;
        int sc, m;
        get_scale_min_k4(j, s_hdr + 4, sc, m);
        const float d = f16_bits_to_f32((uint16_t)(s_hdr[0] | (s_hdr[1] << 8))) * (float)sc;
        int lv = 0;
        if (d != 0.0f) {
            const float dm = f16_bits_to_f32((uint16_t)(s_hdr[2] | (s_hdr[3] << 8))) * (float)m;
            lv = nearest_int((xb[t] + dm) / d);
            lv = lv < 0 ? 0 : (lv > 15 ? 15 : lv);
        }
        s_L[t] = (uint8_t)lv;
    }
    __syncthreads();
    uint8_t* o = (uint8_t*)(out + b);
    if (t < 16) o[t] = s_hdr[t];
    if (t < 128) {
        const int c = t >> 5, l = t & 31;
        o[16 + t] = (uint8_t)(s_L[64 * c + l] | (s_L[64 * c + l + 32] << 4));
    }
}

hipError_t launch_from_float(int dt, const float* x, int64_t nblocks, void* out, hipStream_t s) {
    if (nblocks <= 0) return hipSuccess;
    if (dt == kQ8_0) hipLaunchKernelGGL(k_from_float_q8_0, dim3((nblocks + 255) / 256), dim3(256), 0, s, x, nblocks, (BlockQ8_0*)out);
    else if (dt == kQ4_0) hipLaunchKernelGGL(k_from_float_q4_0, dim3((nblocks + 255) / 256), dim3(256), 0, s, x, nblocks, (BlockQ4_0*)out);
    else if (dt == kQ4K) hipLaunchKernelGGL(k_from_float_q4k, dim3(nblocks), dim3(256), 0, s, x, (BlockQ4K*)out);
    else if (dt == kQ8K) {
        // Q8_K is an activation type; rows of 256 are quantized one wave each.
        return launch_quantize_act(kQ8K, true, x, 256, (int)nblocks, 256, out, s);
    } else return hipErrorInvalidValue;
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------
// to_float from canonical blocks.  One thread per element.
__global__ void k_to_float(int dt, const uint8_t* __restrict__ blocks, int64_t nelem, float* __restrict__ y) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= nelem) return;
    if (dt == kQ8_0) {
        const uint8_t* b = blocks + (e / 32) * 34;
        const float d = f16_bits_to_f32((uint16_t)(b[0] | (b[1] << 8)));
        y[e] = (float)(int8_t)b[2 + (e % 32)] * d;
    } else if (dt == kQ4_0) {
        const uint8_t* b = blocks + (e / 32) * 18;
        const float d = f16_bits_to_f32((uint16_t)(b[0] | (b[1] << 8)));
        const int i = (int)(e % 32);
        const int q = i < 16 ? (b[2 + i] & 0xF) : (b[2 + i - 16] >> 4);
        y[e] = (float)(q - 8) * d;
    } else if (dt == kQ8K) {
        const uint8_t* b = blocks + (e / 256) * 292;
        const float d = __builtin_bit_cast(float, (uint32_t)(b[0] | (b[1] << 8) | (b[2] << 16) | ((uint32_t)b[3] << 24)));
        y[e] = d * (float)(int8_t)b[4 + (e % 256)];
    } else if (dt == kQ4K) {
        const uint8_t* b = blocks + (e / 256) * 144;
        const int i = (int)(e % 256);
        const int c = i / 64, p = i % 64, hi = p >= 32, l = p & 31;
        const float d = f16_bits_to_f32((uint16_t)(b[0] | (b[1] << 8)));
        const float dmin = f16_bits_to_f32((uint16_t)(b[2] | (b[3] << 8)));
        int sc, m;
        get_scale_min_k4(2 * c + hi, b + 4, sc, m);
        const float d1 = d * (float)sc, m1 = dmin * (float)m;
        const uint8_t qb = b[16 + 32 * c + l];
        const int q = hi ? (qb >> 4) : (qb & 0xF);
        y[e] = d1 * (float)q - m1;
    }
}

hipError_t launch_to_float(int dt, const void* blocks, int64_t nelem, float* y, hipStream_t s) {
    if (nelem <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_to_float, dim3((nelem + 255) / 256), dim3(256), 0, s, dt, (const uint8_t*)blocks, nelem, y);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------
// Repack canonical weight blocks into the device layout (and back).  One thread per block.
__global__ void k_repack(int dt, const uint8_t* __restrict__ canon, int64_t nblocks, uint8_t* __restrict__ hdr,
                         uint8_t* __restrict__ qs, bool to_device) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    if (dt == kQ4K) {
        uint8_t* cb = (uint8_t*)canon + b * 144;
        uint8_t* h = hdr + b * 16;
        uint8_t* q = qs + b * 128;
        if (to_device) {
            for (int i = 0; i < 16; ++i) h[i] = cb[i];
            // device byte (4*(4l + c) + t) <- canonical qs byte 32c + l + 8t
            for (int l = 0; l < 8; ++l)
                for (int c = 0; c < 4; ++c)
                    for (int t = 0; t < 4; ++t) q[4 * (4 * l + c) + t] = cb[16 + 32 * c + l + 8 * t];
        } else {
            for (int i = 0; i < 16; ++i) cb[i] = h[i];
            for (int l = 0; l < 8; ++l)
                for (int c = 0; c < 4; ++c)
                    for (int t = 0; t < 4; ++t) cb[16 + 32 * c + l + 8 * t] = q[4 * (4 * l + c) + t];
        }
    } else {
        const int qb = dt == kQ8_0 ? 32 : 16, tb = qb + 2;
        uint8_t* cb = (uint8_t*)canon + b * tb;
        if (to_device) {
            hdr[2 * b] = cb[0];
            hdr[2 * b + 1] = cb[1];
            for (int i = 0; i < qb; ++i) qs[b * qb + i] = cb[2 + i];
        } else {
            cb[0] = hdr[2 * b];
            cb[1] = hdr[2 * b + 1];
            for (int i = 0; i < qb; ++i) cb[2 + i] = qs[b * qb + i];
        }
    }
}

hipError_t launch_repack(int dt, const void* canon, int64_t nblocks, void* hdr, void* qs, bool to_device, hipStream_t s) {
    if (nblocks <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_repack, dim3((nblocks + 255) / 256), dim3(256), 0, s, dt, (const uint8_t*)canon, nblocks,
                       (uint8_t*)hdr, (uint8_t*)qs, to_device);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------
// Synthetic weights: element i of stream `seed` is N(mean, std) from a counter-based
// SplitMix64 pair and the Box-Muller transform (f64), rounded to f32.
SXQ_DEV uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
__global__ void k_fill_normal(float* __restrict__ y, int64_t n, uint64_t seed, float mean, float stdv) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint64_t base = seed * 0xD1B54A32D192ED03ull;
    const uint64_t a = splitmix64(base + 2 * (uint64_t)i), b = splitmix64(base + 2 * (uint64_t)i + 1);
    const double u1 = ((double)(a >> 11) + 1.0) * 0x1.0p-53;
    const double u2 = (double)(b >> 11) * 0x1.0p-53;
    const double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
    y[i] = (float)((double)mean + (double)stdv * z);
}

__global__ void k_bf16_to_f32(const uint16_t* __restrict__ x, int64_t n, float* __restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = __uint_as_float((uint32_t)x[i] << 16);
}

hipError_t launch_bf16_to_f32(const uint16_t* x, int64_t n, float* y, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_bf16_to_f32, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, n, y);
    return hipGetLastError();
}

hipError_t launch_fill_normal(float* y, int64_t n, uint64_t seed, float mean, float stdv, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_fill_normal, dim3((n + 255) / 256), dim3(256), 0, s, y, n, seed, mean, stdv);
    return hipGetLastError();
}

}  // namespace sxq
