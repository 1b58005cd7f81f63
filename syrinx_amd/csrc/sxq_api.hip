// sxq_api.hip -- the C-ABI (include/sxq.h): argument checks with candle-core's error
// behaviour, device selection, workspace management and dispatch to the kernels.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "../../include/sxq.h"
#include "sxq_abi.h"
#include "sxq_kernels.h"

using namespace sxq;

namespace sxq {
namespace abi {

thread_local std::string g_last_error;

sxq_status fail(sxq_status code, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

sxq_status hip_fail(hipError_t e, const char* what) {
    return fail(e == hipErrorOutOfMemory ? SXQ_ERR_OOM : SXQ_ERR_DEVICE, "%s: %s", what, hipGetErrorString(e));
}

}  // namespace abi
}  // namespace sxq

using namespace sxq::abi;

namespace {

// QMatMul::forward's workspace for sxq_qmm_forward: one buffer per device, kept between
// calls.  A call holds it from acquire to release: it makes its stream wait for the
// previous user's event (so calls on different streams, or from different threads, take
// turns on the buffer), grows it stream-ordered when too small, and records the event
// after its last use.  Allocating per call instead (hipMallocAsync / hipFreeAsync) made
// every call wait for the previous one's kernels on the host.  Growth at least doubles
// the size, so a process sees few regrowths.  A stream that is being captured into a
// graph never touches this buffer: a captured forward gets its workspace from the caller
// (sxq_qmm_forward_ws), which the graph then owns, so no replay can alias an eager call
// and no regrowth can free memory a graph still uses.
struct Workspace {
    std::mutex mu;
    void* buf = nullptr;
    size_t size = 0;
    hipEvent_t done = nullptr;
};
Workspace g_ws[64];

struct WorkspaceLease {
    Workspace* w = nullptr;
    hipStream_t s = nullptr;
    uint8_t* ptr = nullptr;
    hipError_t err = hipSuccess;
    WorkspaceLease(int dev, size_t need, hipStream_t st) : s(st) {
        if (dev < 0 || dev >= 64) { err = hipErrorInvalidDevice; return; }
        w = &g_ws[dev];
        w->mu.lock();
        if (!w->done) err = hipEventCreateWithFlags(&w->done, hipEventDisableTiming);
        if (err == hipSuccess) err = hipStreamWaitEvent(s, w->done, 0);
        if (err == hipSuccess && w->size < need) {
            size_t grow = need > 2 * w->size ? need : 2 * w->size;
            grow = (grow + (1u << 20) - 1) & ~(size_t)((1u << 20) - 1);
            if (w->buf) err = hipFreeAsync(w->buf, s);
            w->buf = nullptr;
            w->size = 0;
            if (err == hipSuccess) err = hipMallocAsync(&w->buf, grow, s);
            if (err == hipSuccess) w->size = grow;
        }
        ptr = (uint8_t*)w->buf;
    }
    ~WorkspaceLease() {
        if (!w) return;
        if (w->done) (void)hipEventRecord(w->done, s);
        w->mu.unlock();
    }
    WorkspaceLease(const WorkspaceLease&) = delete;
    WorkspaceLease& operator=(const WorkspaceLease&) = delete;
};

bool quant_weight_dtype(int dt) { return dt == kQ4_0 || dt == kQ8_0 || dt == kQ4K; }
bool block_dtype(int dt) { return dt == kQ4_0 || dt == kQ8_0 || dt == kQ4K || dt == kQ8K; }

const char* dtype_name(int dt) {
    switch (dt) {
    case kF32: return "F32";
    case kF16: return "F16";
    case kQ4_0: return "Q4_0";
    case kQ8_0: return "Q8_0";
    case kQ4K: return "Q4K";
    case kQ8K: return "Q8K";
    default: return "?";
    }
}

std::string shape_str(const int64_t* s, int nd) {
    std::string o = "[";
    for (int i = 0; i < nd; ++i) {
        if (i) o += ", ";
        o += std::to_string((long long)s[i]);
    }
    return o + "]";
}

}  // namespace

extern "C" {

const char* sxq_last_error(void) { return g_last_error.c_str(); }
const char* sxq_version(void) { return "sxq 0.1 (gfx950)"; }
size_t sxq_block_size(int dtype) { return (size_t)block_size(dtype); }
size_t sxq_type_size(int dtype) { return (size_t)type_size(dtype); }

sxq_status sxq_device_count(int* count) {
    if (!count) return fail(SXQ_ERR_INVALID, "sxq_device_count: null pointer");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) {
        *count = 0;
        return hip_fail(e, "hipGetDeviceCount");
    }
    *count = n;
    return SXQ_OK;
}

sxq_status sxq_quantize_rows(int device, int dtype, const float* x, int64_t rows, int64_t k, void* out, void* stream) {
    if (!block_dtype(dtype)) return fail(SXQ_ERR_DTYPE, "quantize: unsupported dtype %s (%d)", dtype_name(dtype), dtype);
    if (rows < 0 || k <= 0) return fail(SXQ_ERR_INVALID, "quantize: bad shape [%lld, %lld]", (long long)rows, (long long)k);
    const int bs = block_size(dtype);
    if (k % bs != 0)
        return fail(SXQ_ERR_BLOCK_ALIGN,
                    "quantized tensor must have their last dim divisible by block size [%lld, %lld] %d",
                    (long long)rows, (long long)k, bs);
    if (rows == 0) return SXQ_OK;
    if (!x || !out) return fail(SXQ_ERR_INVALID, "quantize: null pointer");
    DeviceGuard g(device);
    HIP_TRY(g.err, "hipSetDevice");
    hipStream_t s = (hipStream_t)stream;
    if (dtype == kQ8K) {
        if (rows > 65535) return fail(SXQ_ERR_INVALID, "quantize: too many rows for Q8_K (%lld)", (long long)rows);
        HIP_TRY(launch_quantize_act(kQ8K, true, x, k, (int)rows, (int)k, out, s), "quantize Q8K");
    } else {
        HIP_TRY(launch_from_float(dtype, x, rows * (k / bs), out, s), "quantize");
    }
    return SXQ_OK;
}

sxq_status sxq_dequantize_rows(int device, int dtype, const void* blocks, int64_t rows, int64_t k, float* out,
                               void* stream) {
    if (!block_dtype(dtype)) return fail(SXQ_ERR_DTYPE, "dequantize: unsupported dtype %s (%d)", dtype_name(dtype), dtype);
    if (rows < 0 || k <= 0) return fail(SXQ_ERR_INVALID, "dequantize: bad shape");
    if (k % block_size(dtype) != 0)
        return fail(SXQ_ERR_BLOCK_ALIGN, "dequantize: %lld is not divisible by %d", (long long)k, block_size(dtype));
    if (rows == 0) return SXQ_OK;
    if (!blocks || !out) return fail(SXQ_ERR_INVALID, "dequantize: null pointer");
    DeviceGuard g(device);
    HIP_TRY(g.err, "hipSetDevice");
    HIP_TRY(launch_to_float(dtype, blocks, rows * k, out, (hipStream_t)stream), "dequantize");
    return SXQ_OK;
}

sxq_status sxq_act_quantize(int device, int vec_dtype, const float* x, int64_t m, int64_t k, void* out, void* stream) {
    if (vec_dtype != kQ8_0 && vec_dtype != kQ8K)
        return fail(SXQ_ERR_DTYPE, "act_quantize: vec-dot dtype must be Q8_0 or Q8K, got %d", vec_dtype);
    if (m < 0 || k <= 0 || m > 65535) return fail(SXQ_ERR_INVALID, "act_quantize: bad shape");
    if (k % block_size(vec_dtype) != 0)
        return fail(SXQ_ERR_BLOCK_ALIGN, "act_quantize: %lld is not divisible by %d", (long long)k, block_size(vec_dtype));
    if (m == 0) return SXQ_OK;
    if (!x || !out) return fail(SXQ_ERR_INVALID, "act_quantize: null pointer");
    DeviceGuard g(device);
    HIP_TRY(g.err, "hipSetDevice");
    HIP_TRY(launch_quantize_act(vec_dtype, true, x, k, (int)m, (int)k, out, (hipStream_t)stream), "act_quantize");
    return SXQ_OK;
}

sxq_status sxq_qmm_create(int device, int dtype, int64_t n, int64_t k, const void* blocks, size_t nbytes,
                          int src_is_device, sxq_qmm** out) {
    if (!out) return fail(SXQ_ERR_INVALID, "qmm_create: null output handle");
    *out = nullptr;
    if (!quant_weight_dtype(dtype))
        return fail(SXQ_ERR_DTYPE, "qmm_create: weight dtype %s (%d) not supported (Q4_0, Q8_0, Q4K)",
                    dtype_name(dtype), dtype);
    if (n <= 0 || k <= 0) return fail(SXQ_ERR_INVALID, "qmm_create: bad shape [%lld, %lld]", (long long)n, (long long)k);
    const int bs = block_size(dtype);
    if (k % bs != 0)
        return fail(SXQ_ERR_BLOCK_ALIGN,
                    "quantized tensor must have their last dim divisible by block size [%lld, %lld] %d",
                    (long long)n, (long long)k, bs);
    if (k / bs > (1 << 30) / 2 || n > (int64_t)1 << 31) return fail(SXQ_ERR_INVALID, "qmm_create: shape too large");
    const int64_t nb = k / bs, nblocks = n * nb;
    const size_t canon = (size_t)nblocks * (size_t)type_size(dtype);
    if (nbytes != canon)
        return fail(SXQ_ERR_SHAPE, "qmm_create: %zu bytes given, [%lld, %lld] %s needs %zu", nbytes, (long long)n,
                    (long long)k, dtype_name(dtype), canon);
    if (!blocks) return fail(SXQ_ERR_INVALID, "qmm_create: null blocks");
    DeviceGuard g(device);
    HIP_TRY(g.err, "hipSetDevice");

    sxq_qmm* q = new sxq_qmm();
    q->device = device;
    q->storage = canon;
    const size_t hdr_bytes = (size_t)nblocks * weight_hdr_bytes(dtype);
    const size_t hdr_pad = (hdr_bytes + 255) & ~(size_t)255;
    const size_t qs_bytes = (size_t)nblocks * weight_qs_bytes(dtype);
    hipError_t e = hipMalloc(&q->mem, hdr_pad + qs_bytes);
    if (e != hipSuccess) {
        delete q;
        return hip_fail(e, "qmm_create: hipMalloc");
    }
    void* staging = nullptr;
    const void* src = blocks;
    if (!src_is_device) {
        e = hipMalloc(&staging, canon);
        if (e == hipSuccess) e = hipMemcpy(staging, blocks, canon, hipMemcpyHostToDevice);
        src = staging;
    }
    if (e == hipSuccess)
        e = launch_repack(dtype, src, nblocks, q->mem, (uint8_t*)q->mem + hdr_pad, true, nullptr);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (staging) (void)hipFree(staging);
    if (e != hipSuccess) {
        (void)hipFree(q->mem);
        delete q;
        return hip_fail(e, "qmm_create: upload/repack");
    }
    q->w.dtype = dtype;
    q->w.n = n;
    q->w.k = k;
    q->w.nb = nb;
    q->w.hdr = (const uint8_t*)q->mem;
    q->w.qs = (const uint8_t*)q->mem + hdr_pad;
    *out = q;
    return SXQ_OK;
}

sxq_status sxq_qmm_info(const sxq_qmm* q, int* dtype, int64_t* n, int64_t* k, size_t* storage) {
    if (!q) return fail(SXQ_ERR_INVALID, "qmm_info: null handle");
    if (dtype) *dtype = q->w.dtype;
    if (n) *n = q->w.n;
    if (k) *k = q->w.k;
    if (storage) *storage = q->storage;
    return SXQ_OK;
}

sxq_status sxq_qmm_export(const sxq_qmm* q, void* out, void* stream) {
    if (!q || !out) return fail(SXQ_ERR_INVALID, "qmm_export: null pointer");
    DeviceGuard g(q->device);
    HIP_TRY(g.err, "hipSetDevice");
    HIP_TRY(launch_repack(q->w.dtype, out, q->w.n * q->w.nb, (void*)q->w.hdr, (void*)q->w.qs, false, (hipStream_t)stream),
            "qmm_export");
    return SXQ_OK;
}

sxq_status sxq_qmm_dequantize(const sxq_qmm* q, float* out, void* stream) {
    if (!q || !out) return fail(SXQ_ERR_INVALID, "qmm_dequantize: null pointer");
    DeviceGuard g(q->device);
    HIP_TRY(g.err, "hipSetDevice");
    hipStream_t s = (hipStream_t)stream;
    void* canon = nullptr;
    HIP_TRY(hipMallocAsync(&canon, q->storage, s), "qmm_dequantize: workspace");
    hipError_t e = launch_repack(q->w.dtype, canon, q->w.n * q->w.nb, (void*)q->w.hdr, (void*)q->w.qs, false, s);
    if (e == hipSuccess) e = launch_to_float(q->w.dtype, canon, q->w.n * q->w.k, out, s);
    hipError_t e2 = hipFreeAsync(canon, s);
    if (e != hipSuccess) return hip_fail(e, "qmm_dequantize");
    if (e2 != hipSuccess) return hip_fail(e2, "qmm_dequantize: free");
    return SXQ_OK;
}

sxq_status sxq_qmm_destroy(sxq_qmm* q) {
    if (!q) return SXQ_OK;
    DeviceGuard g(q->device);
    if (q->mem) (void)hipFree(q->mem);
    delete q;
    return SXQ_OK;
}

}  // extern "C"

namespace sxq {
namespace abi {

sxq_status plan_forward(const sxq_qmm* q, const int64_t* shape, int ndim, const int64_t* strides, unsigned flags,
                        unsigned allowed, FwdPlan* p) {
    if (!q) return fail(SXQ_ERR_INVALID, "qmm_forward: null handle");
    if (!shape || ndim <= 0) return fail(SXQ_ERR_INVALID, "qmm_forward: missing input shape");
    if (flags & ~allowed) return fail(SXQ_ERR_INVALID, "qmm_forward: unsupported flags 0x%x", flags & ~allowed);
    const std::string ss = shape_str(shape, ndim);
    if (ndim < 2) return fail(SXQ_ERR_SHAPE, "input tensor has only one dimension %s", ss.c_str());
    if (strides) {
        int64_t expect = 1;
        for (int i = ndim - 1; i >= 0; --i) {
            if (shape[i] != 1 && strides[i] != expect)
                return fail(SXQ_ERR_NOT_CONTIGUOUS, "input tensor is not contiguous %s strides %s", ss.c_str(),
                            shape_str(strides, ndim).c_str());
            expect *= shape[i];
        }
    }
    if (shape[ndim - 1] != q->w.k)
        return fail(SXQ_ERR_SHAPE, "input tensor %s incompatible with [%lld, %lld]", ss.c_str(), (long long)q->w.n,
                    (long long)q->w.k);
    int64_t m = 1;
    for (int i = 0; i < ndim - 1; ++i) {
        if (shape[i] < 0) return fail(SXQ_ERR_INVALID, "qmm_forward: negative dim in %s", ss.c_str());
        m *= shape[i];
    }
    if (m > 65535) return fail(SXQ_ERR_INVALID, "qmm_forward: %lld rows exceed the 65535-row limit", (long long)m);
    p->m = m;
    p->vdt = vec_dot_type(q->w.dtype);
    p->nbv = q->w.k / block_size(p->vdt);
    // Many rows: a GEMM, one pass over the weights.  Q8_0 / Q4_0 run the int8 matrix-core
    // GEMM, bit-identical to Candle's vec-dot.  Q4_K runs the f16 MFMA GEMM (operands
    // rounded to f16, error below 2^-10 * sum |w x| per output) unless SXQ_BIT_EXACT asks
    // for Candle's integer vec-dot (the GEMV, 16 rows at a time).
    const bool q80 = q->w.dtype == kQ8_0 || q->w.dtype == kQ4_0;
    p->gemm = q80 ? m >= kGemmQ80MinRows : (m >= kGemmMinRows && !(flags & SXQ_BIT_EXACT));
    p->ws = m == 0 ? 0
                   : up256(p->gemm && !q80 ? gemm_q4k_workspace(q->w.n, (int)m, q->w.k)
                                           : (size_t)m * (size_t)p->nbv * act_block_bytes(p->vdt));
    // bf16 input: widened to f32 at the workspace's end, then the f32 forward
    p->xconv = (flags & SXQ_BF16_INPUT) && m > 0 ? up256((size_t)m * (size_t)q->w.k * 4) : 0;
    p->ws += p->xconv;
    return SXQ_OK;
}

hipError_t run_forward(const sxq_qmm* q, const FwdPlan& p, const float* x, float* y, const float* bias, uint8_t* ws,
                       hipStream_t s) {
    const int64_t k = q->w.k, n = q->w.n, m = p.m;
    if (p.xconv) {  // x is bf16: its exact f32 values at the end of the workspace
        float* xf = (float*)(ws + p.ws - p.xconv);
        const hipError_t e = launch_bf16_to_f32((const uint16_t*)(const void*)x, m * k, xf, s);
        if (e != hipSuccess) return e;
        x = xf;
    }
    if (p.gemm && q->w.dtype == kQ4K) {
        hipError_t e = launch_gemm_q4k_prep(x, k, (int)m, n, (int)k, ws, s);
        if (e == hipSuccess) e = launch_gemm_q4k(q->w, ws, (int)m, y, n, bias, nullptr, 0, s);
        return e;
    }
    // one row of Q8_0 / Q4_0: the GEMV quantizes x in its own prologue (one launch, same bits)
    static const bool separate = getenv("SXQ_GEMV_QUANT_SEPARATE") != nullptr;  // A/B: two launches
    if (m == 1 && !p.gemm && !separate && gemv_quant_fits(q->w)) return launch_gemv_quant(q->w, x, y, bias, nullptr, s);
    hipError_t e = launch_quantize_act(p.vdt, false, x, k, (int)m, (int)k, ws, s);
    if (p.gemm) return e == hipSuccess ? launch_gemm_q80(q->w, ws, (int)m, y, n, bias, nullptr, 0, s) : e;
    for (int64_t r0 = 0; r0 < m && e == hipSuccess; r0 += 16) {
        const int mm = (int)(m - r0 < 16 ? m - r0 : 16);
        e = launch_gemv(q->w, ws + (size_t)r0 * p.nbv * act_block_bytes(p.vdt), mm, y + r0 * n, n, bias, nullptr, 0, s);
    }
    return e;
}

}  // namespace abi
}  // namespace sxq

extern "C" {

sxq_status sxq_qmm_forward(const sxq_qmm* q, const float* x, const int64_t* shape, int ndim, const int64_t* strides,
                           float* y, const float* bias, unsigned flags, void* stream) {
    FwdPlan p;
    sxq_status st = plan_forward(q, shape, ndim, strides, flags, SXQ_HOST_PTRS | SXQ_BIT_EXACT | SXQ_BF16_INPUT, &p);
    if (st != SXQ_OK) return st;
    if (p.m == 0) return SXQ_OK;
    if (!x || !y) return fail(SXQ_ERR_INVALID, "qmm_forward: null x or y");

    DeviceGuard g(q->device);
    HIP_TRY(g.err, "hipSetDevice");
    hipStream_t s = (hipStream_t)stream;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    HIP_TRY(hipStreamIsCapturing(s, &cs), "qmm_forward: capture status");
    if (cs != hipStreamCaptureStatusNone)
        return fail(SXQ_ERR_INVALID,
                    "qmm_forward: the stream is being captured into a graph; a captured forward needs its own "
                    "workspace (sxq_qmm_forward_ws) or the fixed scratch (sxq_qmm_forward_noalloc)");
    const bool host = (flags & SXQ_HOST_PTRS) != 0;
    const int64_t k = q->w.k, n = q->w.n, m = p.m;

    // One stream-ordered workspace: [plan | x | y | bias] (the last three only for host pointers).
    const size_t xb = host ? (size_t)(m * k) * ((flags & SXQ_BF16_INPUT) ? 2 : 4) : 0, yb = host ? (size_t)(m * n) * 4 : 0;
    const size_t bb = (host && bias) ? (size_t)n * 4 : 0;
    WorkspaceLease lease(q->device, p.ws + up256(xb) + up256(yb) + up256(bb), s);
    HIP_TRY(lease.err, "qmm_forward: workspace");
    uint8_t* ws = lease.ptr;
    const float* dx = x;
    float* dy = y;
    const float* dbias = bias;
    hipError_t e = hipSuccess;
    if (host) {
        float* hx = (float*)(ws + p.ws);
        dy = (float*)(ws + p.ws + up256(xb));
        e = hipMemcpyAsync(hx, x, xb, hipMemcpyHostToDevice, s);
        dx = hx;
        if (e == hipSuccess && bias) {
            float* hb = (float*)(ws + p.ws + up256(xb) + up256(yb));
            e = hipMemcpyAsync(hb, bias, bb, hipMemcpyHostToDevice, s);
            dbias = hb;
        }
    }
    if (e == hipSuccess) e = run_forward(q, p, dx, dy, dbias, ws, s);
    if (host && e == hipSuccess) e = hipMemcpyAsync(y, dy, yb, hipMemcpyDeviceToHost, s);
    if (host && e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_fail(e, "qmm_forward");
    return SXQ_OK;
}

sxq_status sxq_qmm_workspace_size(const sxq_qmm* q, int64_t m, unsigned flags, size_t* bytes) {
    if (!bytes) return fail(SXQ_ERR_INVALID, "qmm_workspace_size: null output");
    if (!q) return fail(SXQ_ERR_INVALID, "qmm_workspace_size: null handle");
    if (m < 0) return fail(SXQ_ERR_INVALID, "qmm_workspace_size: negative row count");
    const int64_t shape[2] = {m, q->w.k};
    FwdPlan p;
    sxq_status st = plan_forward(q, shape, 2, nullptr, flags, SXQ_BIT_EXACT | SXQ_BF16_INPUT, &p);
    if (st != SXQ_OK) return st;
    *bytes = p.ws;
    return SXQ_OK;
}

sxq_status sxq_qmm_forward_ws(const sxq_qmm* q, const float* x, const int64_t* shape, int ndim,
                              const int64_t* strides, float* y, const float* bias, unsigned flags, void* workspace,
                              size_t workspace_bytes, void* stream) {
    FwdPlan p;
    sxq_status st = plan_forward(q, shape, ndim, strides, flags, SXQ_BIT_EXACT | SXQ_BF16_INPUT, &p);
    if (st != SXQ_OK) return st;
    if (p.m == 0) return SXQ_OK;
    if (!x || !y) return fail(SXQ_ERR_INVALID, "qmm_forward_ws: null x or y");
    if (workspace_bytes < p.ws || !workspace)
        return fail(SXQ_ERR_INVALID, "qmm_forward_ws: the workspace holds %zu bytes, this call needs %zu",
                    workspace ? workspace_bytes : (size_t)0, p.ws);
    if ((uintptr_t)workspace & 255) return fail(SXQ_ERR_INVALID, "qmm_forward_ws: workspace not 256-byte aligned");
    DeviceGuard g(q->device);
    HIP_TRY(g.err, "hipSetDevice");
    HIP_TRY(run_forward(q, p, x, y, bias, (uint8_t*)workspace, (hipStream_t)stream), "qmm_forward_ws");
    return SXQ_OK;
}

sxq_status sxq_fill_normal(int device, float* out, int64_t n, uint64_t seed, float mean, float std_dev, void* stream) {
    if (n < 0 || (n > 0 && !out)) return fail(SXQ_ERR_INVALID, "fill_normal: bad arguments");
    DeviceGuard g(device);
    HIP_TRY(g.err, "hipSetDevice");
    HIP_TRY(launch_fill_normal(out, n, seed, mean, std_dev, (hipStream_t)stream), "fill_normal");
    return SXQ_OK;
}

}  // extern "C"
