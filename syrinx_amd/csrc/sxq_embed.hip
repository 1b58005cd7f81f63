// sxq_embed.hip -- per-row symmetric int8 / int4 embedding tables and their
// dequant-on-gather:
//   quantize_embed_int8 / _int4   crates/syrinx-lm/src/cv2/quant.rs:50-89
//   embed_rows (Int8 / Int4)      crates/syrinx-lm/src/cv2/generate.rs:22-67
//
// A table row x[0..h) gets scale = max|x| / qmax + 1e-12 and codes round(x / scale)
// clamped to [-qmax, qmax] (qmax 127 or 7), stored as the byte q + 128 (int8) or as
// nibbles q + 8, element 2j in the low nibble of byte j and 2j + 1 in the high one
// (int4).  The float steps are Candle's on f32 tensors: `t / 127.0` and `t + 1e-12` are
// its affine map t * m + a with m, a rounded to f32 (no fused multiply-add), the division
// x / scale is an f32 division and round() rounds halves away from zero.  A gathered row
// is (float)q * scale, one f32 product per element -- the same bits as the reference.
//
// One workgroup per row: the row is read once for max|x| (a max is order-free) and once
// more for the codes; tables are at most a few hundred MB, so this is an HBM-bound pass.
#include <hip/hip_runtime.h>

#include "../../include/sxq.h"
#include "sxq_abi.h"

using namespace sxq;
using namespace sxq::abi;

namespace {

constexpr int kEQ = 256;

SXQ_DEV float embed_scale(float amax, float inv_qmax, float eps) {
    return __fadd_rn(__fmul_rn(amax, inv_qmax), eps);
}

template <int QMAX>
SXQ_DEV int embed_code(float x, float s) {
    float q = roundf(__fdiv_rn(x, s));
    q = fminf(fmaxf(q, -(float)QMAX), (float)QMAX);
    return (int)q;
}

template <int BITS>
__global__ __launch_bounds__(kEQ) void k_embed_quantize(const float* __restrict__ table, int h, float inv_qmax,
                                                        float eps, uint8_t* __restrict__ q, float* __restrict__ scale) {
    __shared__ float red[kEQ / 64];
    const int64_t r = blockIdx.x;
    const int tid = threadIdx.x;
    const float* x = table + r * h;
    float m = 0.0f;
    for (int j = tid; j < h; j += kEQ) m = fmaxf(m, fabsf(x[j]));
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    m = red[0];
    for (int w = 1; w < kEQ / 64; ++w) m = fmaxf(m, red[w]);
    const float s = embed_scale(m, inv_qmax, eps);
    if (tid == 0) scale[r] = s;
    if (BITS == 8) {
        uint8_t* qr = q + r * h;
        for (int j = tid; j < h; j += kEQ) qr[j] = (uint8_t)(embed_code<127>(x[j], s) + 128);
    } else {
        const int hp = h / 2;
        uint8_t* qr = q + r * hp;
        for (int j = tid; j < hp; j += kEQ) {
            const int lo = (embed_code<7>(x[2 * j], s) + 8) & 15;
            const int hi = (embed_code<7>(x[2 * j + 1], s) + 8) & 15;
            qr[j] = (uint8_t)(lo | (hi << 4));
        }
    }
}

// grid (n, ceil(h / 256)): out[i][e] = (float)(code - offset) * scale[id]; an id outside
// the table gives a zero row.
template <int BITS>
__global__ __launch_bounds__(256) void k_embed_gather(const uint8_t* __restrict__ q, const float* __restrict__ scale,
                                                      int64_t rows, int h, const int32_t* __restrict__ ids,
                                                      int ids_stride, float* __restrict__ out) {
    const int i = blockIdx.x;
    const int e = blockIdx.y * 256 + threadIdx.x;
    if (e >= h) return;
    const int64_t id = ids[(int64_t)i * ids_stride];
    float v = 0.0f;
    if (id >= 0 && id < rows) {
        int c;
        if (BITS == 8) {
            c = (int)q[id * h + e] - 128;
        } else {
            const uint8_t b = q[id * (h / 2) + (e >> 1)];
            c = (int)((e & 1) ? (b >> 4) : (b & 15)) - 8;
        }
        v = (float)c * scale[id];
    }
    out[(int64_t)i * h + e] = v;
}

}  // namespace

namespace sxq {
namespace abi {

int embed_effective_scheme(int scheme, int64_t h) {
    return (scheme == SXQ_EMBED_INT4 && (h % 2) != 0) ? SXQ_EMBED_INT8 : scheme;
}

size_t embed_code_bytes(int scheme, int64_t rows, int64_t h) {
    return (size_t)rows * (size_t)(scheme == SXQ_EMBED_INT4 ? h / 2 : h);
}

hipError_t launch_embed_gather(int scheme, const uint8_t* q, const float* scale, int64_t rows, int h, const int32_t* ids,
                               int ids_stride, int n, float* out, hipStream_t s) {
    const dim3 grid(n, (h + 255) / 256);
    if (scheme == SXQ_EMBED_INT4)
        hipLaunchKernelGGL(k_embed_gather<4>, grid, dim3(256), 0, s, q, scale, rows, h, ids, ids_stride, out);
    else
        hipLaunchKernelGGL(k_embed_gather<8>, grid, dim3(256), 0, s, q, scale, rows, h, ids, ids_stride, out);
    return hipGetLastError();
}

}  // namespace abi
}  // namespace sxq

extern "C" {

sxq_status sxq_embed_scheme(int requested, int64_t h, int* effective) {
    if (!effective) return fail(SXQ_ERR_INVALID, "embed_scheme: null output");
    if (requested != SXQ_EMBED_INT8 && requested != SXQ_EMBED_INT4)
        return fail(SXQ_ERR_INVALID, "embed_scheme: unknown scheme %d", requested);
    if (h < 1) return fail(SXQ_ERR_INVALID, "embed_scheme: row width %lld", (long long)h);
    *effective = embed_effective_scheme(requested, h);
    return SXQ_OK;
}

sxq_status sxq_embed_quantize(int device, int scheme, const float* table, int64_t rows, int64_t h, uint8_t* q,
                              float* scale, void* stream) {
    if (scheme != SXQ_EMBED_INT8 && scheme != SXQ_EMBED_INT4)
        return fail(SXQ_ERR_INVALID, "embed_quantize: unknown scheme %d", scheme);
    if (scheme == SXQ_EMBED_INT4 && h % 2 != 0)
        return fail(SXQ_ERR_INVALID, "embed_quantize: int4 packs pairs, row width %lld is odd (use int8)", (long long)h);
    if (rows < 1 || h < 1 || h > (int64_t)1 << 30 || rows > 0x7FFFFFFF)
        return fail(SXQ_ERR_INVALID, "embed_quantize: bad table shape [%lld, %lld]", (long long)rows, (long long)h);
    if (!table || !q || !scale) return fail(SXQ_ERR_INVALID, "embed_quantize: null pointer");
    DeviceGuard g(device);
    HIP_TRY(g.err, "hipSetDevice");
    const float eps = 1e-12f;
    if (scheme == SXQ_EMBED_INT8)
        hipLaunchKernelGGL(k_embed_quantize<8>, dim3((unsigned)rows), dim3(kEQ), 0, (hipStream_t)stream, table, (int)h,
                           (float)(1.0 / 127.0), eps, q, scale);
    else
        hipLaunchKernelGGL(k_embed_quantize<4>, dim3((unsigned)rows), dim3(kEQ), 0, (hipStream_t)stream, table, (int)h,
                           (float)(1.0 / 7.0), eps, q, scale);
    HIP_TRY(hipGetLastError(), "embed_quantize");
    return SXQ_OK;
}

sxq_status sxq_embed_gather(int device, int scheme, const uint8_t* q, const float* scale, int64_t rows, int64_t h,
                            const int32_t* ids, int n, float* out, void* stream) {
    if (scheme != SXQ_EMBED_INT8 && scheme != SXQ_EMBED_INT4)
        return fail(SXQ_ERR_INVALID, "embed_gather: unknown scheme %d", scheme);
    if (scheme == SXQ_EMBED_INT4 && h % 2 != 0) return fail(SXQ_ERR_INVALID, "embed_gather: int4 with odd row width");
    if (rows < 1 || h < 1 || h > (int64_t)1 << 30 || n < 0 || n > 0x7FFFFFFF)
        return fail(SXQ_ERR_INVALID, "embed_gather: bad shape");
    if (n == 0) return SXQ_OK;
    if (!q || !scale || !ids || !out) return fail(SXQ_ERR_INVALID, "embed_gather: null pointer");
    DeviceGuard g(device);
    HIP_TRY(g.err, "hipSetDevice");
    HIP_TRY(launch_embed_gather(scheme, q, scale, rows, (int)h, ids, 1, n, out, (hipStream_t)stream), "embed_gather");
    return SXQ_OK;
}

}  // extern "C"
