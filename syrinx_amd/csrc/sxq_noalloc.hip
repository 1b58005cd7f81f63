// sxq_noalloc.hip -- sxq_qmm_forward_noalloc: QMatMul::forward for callers that cannot
// allocate device memory (code under HIP graph capture, serving loops that forbid
// hipMalloc).  Its workspace is a fixed array in the library's device image instead of
// a runtime allocation.
#include <hip/hip_runtime.h>

#include <mutex>

#include "sxq_abi.h"

using namespace sxq;
using namespace sxq::abi;

namespace {

// The fixed scratch: one copy per GPU, loaded with the library's code object and held
// until the process ends.  It holds the forward's quantized activation blocks (decode
// GEMV) or the prefill GEMM's f16 activations, row scales and split-K partials; every
// byte is written before it is read within a call, so nothing needs clearing between
// calls.  64 MiB covers the GEMV at any row count whose activation blocks fit and the
// prefill GEMM of the Qwen3-4B projections up to 1024 rows.
constexpr size_t kScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

// Device address of `scratch` per GPU.  In host code the name `scratch` is a host-side
// stand-in, not a device address, so it is never passed to a kernel or copy: the
// address comes from hipGetSymbolAddress, once per device with that device current.
std::mutex g_mu;
void* g_scratch_dev[64];

hipError_t scratch_on(int dev, uint8_t** out) {
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_scratch_dev[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        g_scratch_dev[dev] = p;
    }
    *out = (uint8_t*)g_scratch_dev[dev];
    return hipSuccess;
}

}  // namespace

extern "C" {

sxq_status sxq_qmm_forward_noalloc(const sxq_qmm* q, const float* x, const int64_t* shape, int ndim,
                                   const int64_t* strides, float* y, const float* bias, unsigned flags, void* stream) {
    FwdPlan p;
    sxq_status st = plan_forward(q, shape, ndim, strides, flags, SXQ_BIT_EXACT | SXQ_BF16_INPUT, &p);
    if (st != SXQ_OK) return st;
    if (p.m == 0) return SXQ_OK;
    if (!x || !y) return fail(SXQ_ERR_INVALID, "qmm_forward_noalloc: null x or y");
    if (p.ws > kScratchBytes)
        return fail(SXQ_ERR_INVALID,
                    "qmm_forward_noalloc: %lld rows of [%lld, %lld] need %zu bytes of scratch, the fixed scratch "
                    "holds %zu",
                    (long long)p.m, (long long)q->w.n, (long long)q->w.k, p.ws, kScratchBytes);
    if (q->device < 0 || q->device >= 64) return fail(SXQ_ERR_DEVICE, "qmm_forward_noalloc: device %d", q->device);
    DeviceGuard g(q->device);
    HIP_TRY(g.err, "hipSetDevice");
    uint8_t* ws = nullptr;
    HIP_TRY(scratch_on(q->device, &ws), "qmm_forward_noalloc: scratch address");
    HIP_TRY(run_forward(q, p, x, y, bias, ws, (hipStream_t)stream), "qmm_forward_noalloc");
    return SXQ_OK;
}

}  // extern "C"
