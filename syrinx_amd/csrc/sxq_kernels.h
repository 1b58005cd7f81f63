// sxq_kernels.h -- launchers shared between the library's translation units.
#pragma once
#include "sxq_common.h"

namespace sxq {

// Activation quantization (QMatMul's first step): x [m, k] -> Q8_K / Q8_0 blocks.
// canon = Candle's block bytes; otherwise the device layout (ActQ8K / ActQ8_0).
hipError_t launch_quantize_act(int vdt, bool canon, const float* x, int64_t ldx, int m, int k, void* out,
                               hipStream_t s);
// Weight quantization (QTensor::quantize): x [nblocks * bs] -> canonical blocks.
hipError_t launch_from_float(int dt, const float* x, int64_t nblocks, void* out, hipStream_t s);
// Dequantization (QTensor::dequantize) of canonical blocks.
hipError_t launch_to_float(int dt, const void* blocks, int64_t nelem, float* y, hipStream_t s);
// Canonical <-> device weight layout.
hipError_t launch_repack(int dt, const void* canon, int64_t nblocks, void* hdr, void* qs, bool to_device,
                         hipStream_t s);
hipError_t launch_fill_normal(float* y, int64_t n, uint64_t seed, float mean, float stdv, hipStream_t s);

// A quantized weight in the device layout.
struct QWeight {
    int dtype = 0;
    int64_t n = 0, k = 0, nb = 0;
    const uint8_t* hdr = nullptr;  // Q4_K: 16 B per block; Q8_0/Q4_0: f16 d per block
    const uint8_t* qs = nullptr;   // Q4_K: 128 B; Q8_0: 32 B; Q4_0: 16 B per block
};

// Decode GEMV, m in 1..16: y[m, n] (row stride ldy) = act[m] . W^T (+ bias) and, if
// `res` is given, y = res + that (res may alias y: each element is read then written
// by one lane).  act is the device activation layout [m][nb] (ActQ8K for Q4_K,
// ActQ8_0 otherwise).
hipError_t launch_gemv(const QWeight& w, const void* act, int m, float* y, int64_t ldy, const float* bias,
                       const float* res, int64_t ldr, hipStream_t s);
// The same product, for the m (5..16) rows launch_gemv runs on the Q4_K matrix-core GEMV,
// read from the MmaRec records [nb] the quantizers wrote beside `act` (the same values):
// gemv_rec_fits tells when it applies; otherwise (or with rec null) this is launch_gemv.
// ws (optional): where the tiles alone would leave compute units idle (the 2560-row wo
// and w2 at 16 rows: 160 tiles), each tile's K is split over up to kGemvRecMaxKs
// workgroups, each adding its own class chains into one partial per output, and the
// tile's last slice adds the partials in slice order: the same terms in another
// association (float rounding only, deterministic), not Candle's bits.  Without ws, or with SXQ_BIT_EXACT set, every tile runs in one workgroup and
// the result is bit-identical to Candle's vec-dot.  The workspace belongs to one stream
// of launches at a time.
// Arrival counters that many workgroups of one launch update (the fused attention's per
// head group, the O projection's per layer, a split GEMV's per tile) sit kCounterStride
// words (256 B) apart: atomics on one line are performed one after another (~14 ns
// each), so counters sharing a line would queue every group's arrivals behind each
// other's.
constexpr int kCounterStride = 64;
constexpr int kGemvRecMaxKs = 4;
constexpr int kGemvRecMaxSplitTiles = 256;  // the most tiles a split launch has
struct GemvRecWs {
    float* part = nullptr;       // [kGemvRecMaxSplitTiles * kGemvRecMaxKs][256] slice partials
    unsigned* count = nullptr;   // [kGemvRecMaxSplitTiles * kCounterStride], zero between launches
    static size_t part_bytes() { return sizeof(float) * (size_t)kGemvRecMaxSplitTiles * kGemvRecMaxKs * 256; }
    static size_t count_bytes() { return sizeof(unsigned) * (size_t)kGemvRecMaxSplitTiles * kCounterStride; }
};
bool gemv_rec_fits(const QWeight& w, int m);
hipError_t launch_gemv_rec(const QWeight& w, const void* act, const MmaRec* rec, int m, float* y, int64_t ldy,
                           const float* bias, const float* res, int64_t ldr, hipStream_t s,
                           const GemvRecWs* ws = nullptr);

// RMSNorm of f32 rows x [m, k] (crates/syrinx-fish/src/s2/nn.rs:100-106), the result
// quantized and multiplied: y = quant(rmsnorm(x) * w_norm) . W^T (+ bias, + res).
// For one row of at most kNormMaxDim elements the norm runs in the GEMV's own
// prologue; otherwise a separate RMSNorm kernel fills `act_scratch` [m][nb] first.
// Both give the same bits.  `normed` (optional) receives the f32 normalised rows.
constexpr int kNormMaxDim = 4096;
struct NormIn {
    const float* x = nullptr;     // rows to normalise, row stride k
    const float* w = nullptr;     // norm weight [k]
    float eps = 0.0f;
    float* normed = nullptr;      // optional f32 copy of the normalised rows [m, k]
};
// rec (optional): MmaRec records [k / 256] for the 5..16-row Q4_K matrix-core GEMV, which
// the RMSNorm kernel then also fills and the GEMV reads instead of act_scratch.
hipError_t launch_gemv_rmsnorm(const QWeight& w, const NormIn& ni, int m, uint8_t* act_scratch, float* y,
                               int64_t ldy, const float* bias, const float* res, int64_t ldr, hipStream_t s,
                               MmaRec* rec = nullptr);

// The feed-forward of one decode row (m = 1) around SwiGLU, Q4_K weights: the fused
// RMSNorm GEMV of the gate|up weight [2I][k] (gate rows first) writes gu [2I] and
// act_f32 = silu(gate) * up [I]; the down GEMV [n][I] quantizes act_f32 in its prologue
// and writes y = res + down . act (res may be null).  Two launches; the same bits as the
// GEMV + SiLU*mul + quantize + GEMV sequence.
bool swiglu_pair_fits(const QWeight& gate_up, const QWeight& down);
hipError_t launch_swiglu_pair(const QWeight& gate_up, const QWeight& down, const NormIn& ni, float* gu, float* act_f32,
                              float* y, const float* res, hipStream_t s);

// Prefill GEMM for Q4_K weights (sxq_gemm.hip): y = x . dequant(W)^T on MFMA with f16
// operands (+ bias, + res).  The workspace (gemm_q4k_workspace bytes) holds x rounded to
// f16 in the GEMM's K order and, when K is split across workgroups, the partial tiles
// and their counters; launch_gemm_q4k_prep fills it from x, then launch_gemm_q4k runs.
constexpr int kGemmMinRows = 64;  // QMatMul::forward uses the Q4_K GEMM from this many rows on
constexpr int kGemmQ80MinRows = 128;  // ... and the Q8_0 / Q4_0 GEMM (below: the GEMV, 16 rows at a time)
size_t gemm_q4k_workspace(int64_t n, int m, int64_t k);
hipError_t launch_gemm_q4k_prep(const float* x, int64_t ldx, int m, int64_t n, int k, void* ws, hipStream_t s);
hipError_t launch_gemm_q4k(const QWeight& w, const void* ws, int m, float* y, int64_t ldy, const float* bias,
                           const float* res, int64_t ldr, hipStream_t s);

// Prefill GEMM for Q8_0 / Q4_0 weights (sxq_gemm_q80.hip): the same outputs as the GEMV
// (Candle's vec-dot, bit for bit) from one pass over the weights on the int8 matrix
// cores.  act: the Q8_0 activation blocks [m][nb] of launch_quantize_act (device layout).
hipError_t launch_gemm_q80(const QWeight& w, const void* act, int m, float* y, int64_t ldy, const float* bias,
                           const float* res, int64_t ldr, hipStream_t s);

}  // namespace sxq

// The QMatMul handle behind the C-ABI's opaque sxq_qmm.
struct sxq_qmm {
    int device = 0;
    sxq::QWeight w;
    void* mem = nullptr;  // one allocation: hdr region, then qs region
    size_t storage = 0;   // canonical byte count (storage_size_in_bytes)
};
