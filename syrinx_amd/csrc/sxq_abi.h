// sxq_abi.h -- error reporting and device scoping shared by the C-ABI translation units.
#pragma once
#include <hip/hip_runtime.h>

#include "../../include/sxq.h"
#include "sxq_kernels.h"

namespace sxq {
// bf16 -> f32 (exact: the bf16 bits are the f32's upper half), n elements (sxq_quant.hip).
hipError_t launch_bf16_to_f32(const uint16_t* x, int64_t n, float* y, hipStream_t s);
// One-row Q8_0 / Q4_0 GEMV that quantizes its f32 row in the prologue (sxq_gemv.hip):
// y = quant(x) . W^T (+ bias, + res), the bits of launch_quantize_act + launch_gemv.
bool gemv_quant_fits(const QWeight& w);
hipError_t launch_gemv_quant(const QWeight& w, const float* x, float* y, const float* bias, const float* res,
                             hipStream_t s);
namespace abi {

// Fish samplers shared with the fast-AR driver (sxq_sample.hip): the codebook draw into
// out (and a copy into out2, may be null), and FastAr::first_code into ids (and codes).
bool fish_sampling_fits(const sxq_fish_sampling& p);
hipError_t launch_sample_codebook(const float* logits, int64_t stride, int n, int vocab, const sxq_fish_sampling& p,
                                  uint64_t* rng, const int32_t* active, int32_t* out, int out_stride, int32_t* out2,
                                  int out2_stride, hipStream_t s);
hipError_t launch_first_codes(const int32_t* semantic, int sem_stride, int n, int begin, int residual,
                              const int32_t* active, int32_t* ids, int32_t* codes, int codes_stride, hipStream_t s);

// Per-row int8 / int4 embedding tables (sxq_embed.hip).
int embed_effective_scheme(int scheme, int64_t h);
size_t embed_code_bytes(int scheme, int64_t rows, int64_t h);
hipError_t launch_embed_gather(int scheme, const uint8_t* q, const float* scale, int64_t rows, int h, const int32_t* ids,
                               int ids_stride, int n, float* out, hipStream_t s);

// Record `fmt` as this thread's sxq_last_error() and return `code`.
sxq_status fail(sxq_status code, const char* fmt, ...);
// Map a HIP error to SXQ_ERR_OOM / SXQ_ERR_DEVICE with its text.
sxq_status hip_fail(hipError_t e, const char* what);

inline size_t up256(size_t v) { return (v + 255) & ~(size_t)255; }

// One QMatMul::forward, checked: m rows of x, which kernel family, workspace bytes.
struct FwdPlan {
    int64_t m = 0;
    bool gemm = false;  // the MFMA prefill GEMM (else quantized activations + GEMV)
    int vdt = 0;
    int64_t nbv = 0;    // activation blocks per row
    size_t ws = 0;      // device workspace: activation blocks, or the GEMM's staging
    size_t xconv = 0;   // SXQ_BF16_INPUT: the f32 copy of x at the workspace's end (inside ws)
};
// Candle's argument checks of QMatMul::forward (its error texts), then the plan; flags
// outside `allowed` are rejected.
sxq_status plan_forward(const sxq_qmm* q, const int64_t* shape, int ndim, const int64_t* strides, unsigned flags,
                        unsigned allowed, FwdPlan* p);
// The kernels of one planned forward on device pointers, with `ws` (p.ws bytes, 256-byte
// aligned) as workspace.  Nothing in `ws` needs to hold anything on entry.
hipError_t run_forward(const sxq_qmm* q, const FwdPlan& p, const float* x, float* y, const float* bias, uint8_t* ws,
                       hipStream_t s);

#define HIP_TRY(expr, what)                                      \
    do {                                                         \
        hipError_t e_ = (expr);                                  \
        if (e_ != hipSuccess) return ::sxq::abi::hip_fail(e_, what); \
    } while (0)

// Makes `dev` current for the scope and restores the caller's device afterwards.
struct DeviceGuard {
    int prev = -1;
    hipError_t err = hipSuccess;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) err = hipSetDevice(dev);
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
    DeviceGuard(const DeviceGuard&) = delete;
    DeviceGuard& operator=(const DeviceGuard&) = delete;
};

}  // namespace abi
}  // namespace sxq
