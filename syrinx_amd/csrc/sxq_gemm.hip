// sxq_gemm.hip -- prefill (many-row) QMatMul over Q4_K weights on CDNA4 MFMA.
//
// For m rows well beyond the decode GEMV (QMatMul::forward with M = prompt length; the
// reference calls it at crates/syrinx-lm/src/cv2/mod.rs:197 and, for the Fish slow AR
// prefill, through Weights::linear at crates/syrinx-fish/src/s2/nn.rs:61-74) the
// contraction is a real GEMM.  Weight tiles are dequantized into LDS as f16 values of
// Candle's to_float, (d*sc)*q - dmin*m: d*sc and dmin*m are exact in f32, and one
// mixed-precision fma rounds (d*sc)*q - dmin*m straight to f16 (Candle's f32 value,
// rounded again to f16, can differ from that by one f16 ulp in a double-rounding tie);
// the activations are rounded to f16; v_mfma_f32_32x32x16_f16 accumulates in f32.  (f16
// rather than bf16: the same MFMA rate on gfx950, with 3 more mantissa bits.)  The
// result therefore differs from Candle's integer Q8_K vec-dot by the f16 rounding of
// both operands, bounded by 2^-10 * sum_k |w_k x_k| per output (plus the f16 subnormal
// floor, 2^-25 per operand value).  A row of x with values beyond f16's range is scaled
// by a power of two 2^-e before the rounding and its results by 2^e after the
// accumulation (exact), so it stays finite; its subnormal floor becomes 2^(e-25).
//
// K order.  Inside each 256-element block the GEMM runs over K in an order chosen so that
// every lane of the kernel dequantizes whole dwords of the Q4_K device layout
// (sxq_common.h: byte B = 16*l + 4*c + t of the class-major qs holds elements
// 64c + l + 8t in its low nibble and 64c + 32 + l + 8t in its high nibble).  GEMM position
// P = 16i + 8h + j, with MFMA step i = 4g + s, half h and j = 0..7, is nibble j&1 of byte
// j>>1 of dword (l = 2g + h, c = s), i.e. element 64s + 32(j&1) + 2g + h + 8(j>>1).  So the
// 16 bytes of segment l = 2g + h feed steps 4g .. 4g+3 of the lanes of half h, and step s
// only needs sub-blocks 2s and 2s+1.  The activations are converted to f16 with the same
// permutation (k_x_to_f16_perm); a dot product does not depend on the order of its terms
// beyond rounding.
#include <stdlib.h>

#include <atomic>
#include <type_traits>

#include "sxq_kernels.h"
#include "sxq_sync_dev.h"

namespace sxq {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) uint8_t lds_u8;

// GEMM position p (0..255) inside a block -> element index of the canonical order.
SXQ_HD int q4k_perm_elem(int p) {
    const int i = p >> 4, h = (p >> 3) & 1, j = p & 7;
    const int g = i >> 2, s = i & 3;
    return 64 * s + 32 * (j & 1) + 2 * g + h + 8 * (j >> 1);
}

constexpr int kGemmBM = 256, kGemmBN = 128;
constexpr int kGemmAStage = kGemmBM * 64 * 2;  // activations of one K group: 256 rows x 64 halfs
constexpr int kGemmHalfBytes = 2 * kGemmAStage;  // one K half's region: 2 activation stages

int gemm_xh_rows(int m) { return (m + kGemmBM - 1) / kGemmBM * kGemmBM; }
size_t gemm_q4k_lds() { return 2 * (size_t)kGemmHalfBytes; }

// Rows whose largest magnitude reaches kF16Safe are scaled by a power of two 2^-e before
// the f16 rounding, so that no value overflows f16 (max 65504); the GEMM multiplies the
// row's f32 result by 2^e, which is exact.  Rows below it keep e = 0: the scale is 1 and
// the bits are those of the unscaled product.
constexpr float kF16Safe = 32768.0f;

// x f32 [m][k] (row stride ldx) -> xh f16 [gemm_xh_rows(m)][k] in the GEMM K order,
// xh[r][256b + p] = f16(x[r][256b + q4k_perm_elem(p)] * 2^-e_r), rows past m zero, and
// rs[r] = 2^e_r.  One workgroup per row: first the row's max |x| (e_r = 0 below
// kF16Safe), then wave w converts blocks w, w + 4, ...: it reads a block as 64 float4s
// (one contiguous 1 KB read, an L2 hit after the first pass), passes it through LDS, and
// lane l < 32 writes positions 8l .. 8l+7 (one MFMA operand chunk; one contiguous
// 512-byte write per wave); position 8l + j is element q4k_perm_elem(8l) + 32 (j & 1) +
// 8 (j >> 1).
__global__ __launch_bounds__(256) void k_x_to_f16_perm(const float* __restrict__ x, int64_t ldx, int m, int k,
                                                       _Float16* __restrict__ xh, float* __restrict__ rs) {
    __shared__ float4 blk[4][64];
    __shared__ float wmax[4];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nb = k >> 8;
    const int64_t r = blockIdx.x;
    const bool live = r < m;
    const float4* xr = (const float4*)(x + r * ldx);
    float amax = 0.0f;
    if (live)
        for (int i = threadIdx.x; i < (k >> 2); i += 256) {
            const float4 v = xr[i];
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
    if (lane == 0) wmax[wave] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    int e = 0;
    if (amax >= kF16Safe && amax <= 3.0e38f) {  // inf / NaN rows stay unscaled (they propagate either way)
        int ex = 0;
        (void)frexpf(amax, &ex);                // amax < 2^ex
        e = ex - 15;                             // amax * 2^-e < 2^15
    }
    const float sc = ldexpf(1.0f, -e);
    if (threadIdx.x == 0) rs[r] = ldexpf(1.0f, e);
    for (int b0 = 0; b0 < nb; b0 += 4) {  // uniform trip count: every wave reaches each barrier
        const int b = b0 + wave;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (live && b < nb) v = xr[64 * b + lane];
        blk[wave][lane] = v;
        __syncthreads();
        if (b < nb && lane < 32) {
            const float* el = (const float*)blk[wave] + q4k_perm_elem(8 * lane);
            half8 h;
#pragma unroll
            for (int j = 0; j < 8; ++j) h[j] = (_Float16)(el[32 * (j & 1) + 8 * (j >> 1)] * sc);
            *(half8*)(xh + r * k + 256 * b + 8 * lane) = h;
        }
        __syncthreads();
    }
}

// The same conversion in one pass over x, for rows of k <= 1024 * V4 elements: the row is
// loaded once (every thread's V4 float4 loads issued together), its max |x| reduced while
// it goes to LDS, and the f16 positions gathered from LDS -- thread t writes the 16-byte
// chunks t, t + 256, ... of the row (chunk c: block c / 32, positions 8 (c mod 32) .. + 7),
// so the row's writes are contiguous.  The bits are k_x_to_f16_perm's.
template <int V4>
__global__ __launch_bounds__(256) void k_x_to_f16_perm1(const float* __restrict__ x, int64_t ldx, int m, int k,
                                                        _Float16* __restrict__ xh, float* __restrict__ rs) {
    extern __shared__ float4 rowbuf[];  // the row, k floats
    __shared__ float wmax[4];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int n4 = k >> 2;
    const int64_t r = blockIdx.x;
    const bool live = r < m;
    const float4* xr = (const float4*)(x + r * ldx);
    float4 v[V4];
#pragma unroll
    for (int j = 0; j < V4; ++j) {
        const int i = tid + 256 * j;
        v[j] = live && i < n4 ? xr[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < V4; ++j) {
        const int i = tid + 256 * j;
        amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)), fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
        if (i < n4) rowbuf[i] = v[j];
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
    if (lane == 0) wmax[wave] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    int e = 0;
    if (amax >= kF16Safe && amax <= 3.0e38f) {  // as k_x_to_f16_perm
        int ex = 0;
        (void)frexpf(amax, &ex);
        e = ex - 15;
    }
    const float sc = ldexpf(1.0f, -e);
    if (tid == 0) rs[r] = ldexpf(1.0f, e);
    const int nchunks = k >> 3;  // 32 chunks of 8 positions per block
    for (int c = tid; c < nchunks; c += 256) {
        const int b = c >> 5, l = c & 31;
        const float* el = (const float*)rowbuf + 256 * b + q4k_perm_elem(8 * l);
        half8 h;
#pragma unroll
        for (int j = 0; j < 8; ++j) h[j] = (_Float16)(el[32 * (j & 1) + 8 * (j >> 1)] * sc);
        *(half8*)(xh + r * k + 8 * c) = h;
    }
}

// The 8 (scale, min) pairs of a Q4_K block header (get_scale_min_k4), times d and dmin:
// sv[j] = d * sc_j, nm[j] = -(dmin * m_j), both exact in f32 (11-bit times 6-bit
// significands).  The 12 scale bytes are header bytes 4..15 (dwords y, z, w = q[0..3],
// q[4..7], q[8..11]); the four 6-bit values of each kind are assembled a dword at a time
// (sc_j = q[j] & 63, m_j = q[j+4] & 63 for j < 4; sc_{j+4} = (q[j+8] & 15) | (q[j] >> 6) << 4,
// m_{j+4} = (q[j+8] >> 4) | (q[j+4] >> 6) << 4) and each byte converts with one
// v_cvt_f32_ubyte<t>.
SXQ_DEV void q4k_scales(const uint4& h, float sv[8], float nm[8]) {
    const uint32_t s03 = h.y & 0x3F3F3F3Fu, m03 = h.z & 0x3F3F3F3Fu;
    const uint32_t s47 = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
    const uint32_t m47 = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
    const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(h.x & 0xFFFF));
    const float dmin = (float)__builtin_bit_cast(_Float16, (uint16_t)(h.x >> 16));
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        sv[t] = d * (float)((s03 >> (8 * t)) & 0xFF);
        sv[t + 4] = d * (float)((s47 >> (8 * t)) & 0xFF);
        nm[t] = -(dmin * (float)((m03 >> (8 * t)) & 0xFF));
        nm[t + 4] = -(dmin * (float)((m47 >> (8 * t)) & 0xFF));
    }
}

// MFMA B operand of one step from one qs dword: element j = 2t + a is nibble a of byte t,
// of sub-block 2s + a, dequantized as scale * q - min with one rounding to f16
// (v_fma_mix: f32 operands, f16 result).  The nibble masks are opaque to the compiler so
// that every byte converts with a single v_cvt_f32_ubyte<t>.
SXQ_DEV half8 q4k_bfrag(uint32_t dw, float s0, float n0, float s1, float n1) {
    uint32_t lo, hi;
    asm("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(lo) : "v"(dw));
    asm("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(hi) : "v"(dw >> 4));
    u32x4 r;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const float ql = (float)((lo >> (8 * t)) & 0xFF), qh = (float)((hi >> (8 * t)) & 0xFF);
        uint32_t pk;
        asm("v_fma_mixlo_f16 %0, %1, %2, %3" : "=v"(pk) : "v"(s0), "v"(ql), "v"(n0));
        asm("v_fma_mixhi_f16 %0, %1, %2, %3" : "+v"(pk) : "v"(s1), "v"(qh), "v"(n1));
        r[t] = pk;
    }
    return __builtin_bit_cast(half8, r);
}

// s_waitcnt vmcnt(n), other counters untouched (gfx9 encoding: vmcnt bits 3:0 and 15:14).
#define SXQ_WAIT_VM(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))

// LDS reads of the GEMM loop, as inline asm: the compiler does not see them, so it does
// not order them after every outstanding global->LDS load (which it would, not knowing
// which LDS bytes those write).  The loop orders them itself: explicit vmcnt waits plus a
// barrier before a stage is read, and lgkm_wait before a read's value is used -- that
// asm takes the values as operands, so nothing that uses them can move above it.
template <int OFF>
SXQ_DEV u32x4 ds_read16(uint32_t addr) {
    u32x4 r;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
    return r;
}
template <int N>
SXQ_DEV void lgkm_wait(u32x4& a, u32x4& b) {
    asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(a), "+v"(b) : "i"(N));
}
template <int N>
SXQ_DEV void lgkm_wait(u32x4& a, u32x4& b, u32x4& c, u32x4& d) {
    asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d) : "i"(N));
}
SXQ_DEV uint32_t lds_addr(const lds_u8* p) { return (uint32_t)(uintptr_t)p; }

// Buffer resource over `bytes` bytes at `base` (raw offsets in bytes, no swizzle).
SXQ_DEV __amdgpu_buffer_rsrc_t tile_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// barrier_nofence (sxq_sync_dev.h) between stages: __syncthreads()'s fence would make
// the compiler wait for every outstanding global->LDS load, including the ones issued
// for later groups.  The caller waits for the loads it needs (SXQ_WAIT_VM); the memory
// clobber keeps the compiler from moving LDS accesses across the barrier.

// y[m][n] = x[m] . W[n] (+ bias[n], then res[m][n] + that), W Q4_K [n][k] in the device
// layout, xh from k_x_to_f16_perm (rows padded to 256).  One workgroup of 512 threads per
// tile (256 token rows x 128 weight rows) or per split of a tile (see GemmPlan).
//
// The 8 waves form two K halves of 4: half h takes the tile's K groups h, h+2, h+4, ...
// (a group is 64 of K, a quarter block); two waves share each SIMD, so one's LDS latency
// and VALU work hide under the other's MFMAs, and 8 waves draw twice the LDS read rate
// of 4.  Wave w of a half owns weight rows 32w .. 32w+31 of the tile and all 256 token
// rows: 8 MFMA tiles of 32 x 32 (128 accumulators per lane), so every dequantized B
// operand feeds 8 MFMAs.  At the end the halves add their accumulators through LDS, half
// 0's first, and each half finishes four of the eight 32-row tiles.
//
// Every operand is loaded one group ahead, by buffer loads whose per-group offsets sit in
// scalar registers (no per-lane address arithmetic in the loop), and the loop's only
// memory waits are explicit vmcnt counts:
//  - activations go straight to LDS (buffer_load ... lds), 2 stages per half; within a
//    stage row r's 16-byte chunk c sits at chunk slot 8r + (c ^ ((r >> 1) & 7)): the MFMA
//    operand reads of any 16 consecutive rows hit 16 different 16-byte bank groups (64
//    banks of 4 bytes);
//  - weights go to registers: lane (n, h) loads segment 2g + h of its row and dequantizes
//    each dword straight into MFMA B registers;
//  - block headers go to registers one block ahead and are decoded into 16 floats at the
//    block's first group, while that group's first activation reads are in flight.
// One barrier per group (both halves in lockstep).
//
// A tile split S ways: split z covers blocks [nb*z/S, nb*(z+1)/S); every split stores its
// partial tile, and k_gemm_splitk_sum, launched after this kernel, adds the partials in
// split order across the whole GPU.
__global__ __launch_bounds__(512) void k_gemm_q4k(const _Float16* __restrict__ xh, int M, int K,
                                                  const uint4* __restrict__ hdr, const uint4* __restrict__ qs, int N,
                                                  float* __restrict__ y, int64_t ldy, const float* __restrict__ bias,
                                                  const float* res, int64_t ldr, const float* __restrict__ rs,
                                                  float* part, int tiles_m, int full, int splits) {
    extern __shared__ uint4 lds[];
    const int nb = K >> 8;
    // Workgroups 0 .. full-1 take whole tiles; the rest split the remaining tiles' K range
    // `splits` ways.  Tile t covers weight rows 128 * (t / tiles_m), token rows 256 * (t % tiles_m).
    const int id = blockIdx.x;
    const int S = id < full ? 1 : splits;
    const int tile = id < full ? id : full + (id - full) / splits;
    const int sp = id < full ? 0 : (id - full) % splits;
    const int n0 = (tile / tiles_m) * kGemmBN, m0 = (tile % tiles_m) * kGemmBM;
    const int b0 = (int)((int64_t)nb * sp / S), b1 = (int)((int64_t)nb * (sp + 1) / S);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kh = wave >> 2, wv = wave & 3;  // K half, weight-row slice
    const int ln = lane & 31, lh = lane >> 5;
    lds_u8* hbase = (lds_u8*)lds + kh * kGemmHalfBytes;

    // Buffer resources over this tile's operands (activation rows m0 .., weight rows n0 ..),
    // so that every load of the loop takes its per-group offset from a scalar register.
    const int nrows = min(kGemmBN, N - n0);
    const __amdgpu_buffer_rsrc_t arsrc = tile_rsrc(xh + (int64_t)m0 * K, (uint32_t)kGemmBM * (uint32_t)K * 2u);
    const __amdgpu_buffer_rsrc_t wrsrc = tile_rsrc(qs + (int64_t)n0 * nb * 8, (uint32_t)nrows * (uint32_t)nb * 128u);
    const __amdgpu_buffer_rsrc_t hrsrc = tile_rsrc(hdr + (int64_t)n0 * nb, (uint32_t)nrows * (uint32_t)nb * 16u);
    // Activation loads: chunk slot (8 wv + u) * 64 + lane of a stage is row
    // r = 64 wv + 8u + lane/8, chunk (lane % 8) ^ ((r >> 1) % 8) of the group.  Row r + 8u has
    // (r >> 1) & 7 with bit 2 flipped when u is odd, so two lane offsets serve all 8 loads.
    const int ar = 64 * wv + (lane >> 3);
    const int ac0 = (lane & 7) ^ ((ar >> 1) & 7);
    const uint32_t aoff_even = (uint32_t)ar * (uint32_t)K * 2u + 16u * ac0;
    const uint32_t aoff_odd = (uint32_t)ar * (uint32_t)K * 2u + 16u * (ac0 ^ 4);
    const uint32_t arow8 = 16u * (uint32_t)K;  // 8 rows, in bytes
    // Weight row of this lane relative to n0 (rows past N clamped: loaded, never stored).
    const int wrel = min(32 * wv + ln, nrows - 1);
    const uint32_t woff = ((uint32_t)wrel * nb * 8u + lh) * 16u, hoff = (uint32_t)wrel * nb * 16u;
    // LDS byte addresses of this lane's reads (stage and row-tile offsets are immediates):
    // activation chunk of step s for row tile 0 (rows ln and 32 mt + ln share (r >> 1) & 7).
    uint32_t aaddr[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) aaddr[s] = lds_addr(hbase) + 16 * (8 * ln + ((2 * s + lh) ^ ((ln >> 1) & 7)));

    // The 8 activation loads of group grp (from the start of K) into stage st of this half.
    auto load_group = [&](int grp, int st) {
        lds_u8* dst = hbase + st * kGemmAStage + wv * 8192;
        const uint32_t g = (uint32_t)grp * 128u;
#pragma unroll
        for (int u = 0; u < 8; ++u)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(arsrc, (__attribute__((address_space(3))) void*)(dst + 1024 * u), 16,
                                                     u & 1 ? aoff_odd : aoff_even, g + u * arow8, 0, 0);
    };
    // This lane's 16 weight bytes of group grp: segment 2 (grp % 4) + lh of block grp / 4.
    auto load_w = [&](int grp) -> u32x4 {
        return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                             wrsrc, woff, (uint32_t)(grp >> 2) * 128u + (uint32_t)(grp & 3) * 32u, 0));
    };
    auto load_h = [&](int blk) -> u32x4 {
        return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(hrsrc, hoff, (uint32_t)blk * 16u, 0));
    };
    float sv[8], nm[8];
    floatx16 acc[8];
#pragma unroll
    for (int a = 0; a < 8; ++a)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[a][i] = 0.0f;

    // One group on stage ST with weight dwords w: per step, 8 activation reads, the B
    // operand dequantized meanwhile, then 8 MFMAs (the other wave of the SIMD covers the
    // read latency).  At a block's first group the block's scales are decoded from its
    // header while the first step's reads are in flight.
    auto compute = [&](auto stc, const u32x4& w, const u32x4* h) {
        constexpr int ST = decltype(stc)::value;
        constexpr int AO = ST * kGemmAStage;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            u32x4 a[8];
            a[0] = ds_read16<AO>(aaddr[s]);
            a[1] = ds_read16<AO + 4096>(aaddr[s]);
            a[2] = ds_read16<AO + 8192>(aaddr[s]);
            a[3] = ds_read16<AO + 12288>(aaddr[s]);
            a[4] = ds_read16<AO + 16384>(aaddr[s]);
            a[5] = ds_read16<AO + 20480>(aaddr[s]);
            a[6] = ds_read16<AO + 24576>(aaddr[s]);
            a[7] = ds_read16<AO + 28672>(aaddr[s]);
            if (s == 0 && h) q4k_scales(make_uint4((*h)[0], (*h)[1], (*h)[2], (*h)[3]), sv, nm);
            const half8 b = q4k_bfrag(w[s], sv[2 * s], nm[2 * s], sv[2 * s + 1], nm[2 * s + 1]);
            lgkm_wait<0>(a[0], a[1], a[2], a[3]);
            lgkm_wait<0>(a[4], a[5], a[6], a[7]);
#pragma unroll
            for (int mt = 0; mt < 8; ++mt)
                acc[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, a[mt]), b, acc[mt], 0, 0, 0);
        }
    };

    // This half's groups: local group li is group 4 b0 + 2 li + kh from the start of K,
    // li = 0 .. LG-1, in block b0 + li/2.  Prologue: the first block's header, local group
    // 0's activations and weights.  Local group li then issues its successor's 8 activation
    // loads and weight load (none after the last group) and, when li is even, the next
    // block's header (clamped to the last block: fetched again, never used).  So when local
    // group li starts, at most the header issued after its loads (li odd) may still be
    // outstanding.
    const int LG = 2 * (b1 - b0);
    const int glast = 4 * (b1 - 1) + 2 + kh;
    auto grp_of = [&](int li) { return min(4 * b0 + 2 * li + kh, glast); };
    u32x4 hnext = load_h(b0);
    u32x4 w0 = load_w(grp_of(0)), w1;
    load_group(grp_of(0), 0);
    for (int li = 0; li < LG; li += 2) {
        __builtin_amdgcn_sched_barrier(0);
        SXQ_WAIT_VM(0);
        barrier_nofence();  // stage 0 is filled everywhere; stage 1 is free
        __builtin_amdgcn_sched_barrier(0);
        const u32x4 h = hnext;
        load_group(grp_of(li + 1), 1);
        // The wait before the next barrier leaves exactly one load in flight, which must
        // be this header load: the scheduler may not move either register load above the
        // stage's LDS loads (were an LDS load issued last, the barrier could pass with its
        // 1 KB of the stage still unwritten).
        __builtin_amdgcn_sched_barrier(0);
        w1 = load_w(grp_of(li + 1));
        __builtin_amdgcn_sched_barrier(0);
        hnext = load_h(min(b0 + li / 2 + 1, b1 - 1));
        __builtin_amdgcn_sched_barrier(0);
        compute(std::integral_constant<int, 0>(), w0, &h);

        __builtin_amdgcn_sched_barrier(0);
        SXQ_WAIT_VM(1);
        barrier_nofence();  // stage 1 is filled everywhere; stage 0 is free
        __builtin_amdgcn_sched_barrier(0);
        if (li + 2 < LG) {  // uniform: the last pair prefetches nothing
            load_group(grp_of(li + 2), 0);
            w0 = load_w(grp_of(li + 2));
        }
        __builtin_amdgcn_sched_barrier(0);
        compute(std::integral_constant<int, 1>(), w1, nullptr);
    }
    SXQ_WAIT_VM(0);  // no global->LDS load may still be in flight past this point
    __syncthreads();

    // Add the halves, half 0's accumulator first: half 1 hands over its row tiles 0-3 and
    // keeps 4-7, half 0 the reverse.  Values 4j .. 4j+3 of row tile t of lane `lane` of
    // wave slice wv of the half that exports sit in float4 red[((half * 4 + wv) * 16 + 4t + j) * 64 + lane].
    f32x4* red = (f32x4*)lds;
    auto exchange = [&](auto keepc) {
        constexpr int KEEP = decltype(keepc)::value, GIVE = 4 - KEEP;
        f32x4* ex = red + ((kh * 4 + wv) * 16) * 64 + lane;
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                ex[(4 * t + j) * 64] = f32x4{acc[GIVE + t][4 * j], acc[GIVE + t][4 * j + 1], acc[GIVE + t][4 * j + 2],
                                             acc[GIVE + t][4 * j + 3]};
        __syncthreads();
        const f32x4* im = red + (((1 - kh) * 4 + wv) * 16) * 64 + lane;
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const f32x4 o = im[(4 * t + j) * 64];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float a = acc[KEEP + t][4 * j + e];
                    acc[KEEP + t][4 * j + e] = KEEP == 0 ? a + o[e] : o[e] + a;
                }
            }
    };
    if (kh == 0) exchange(std::integral_constant<int, 0>());
    else exchange(std::integral_constant<int, 4>());

    // A split tile stores its partial and is done: k_gemm_splitk_sum adds the S partials.
    // Row tile mt, float4 j, thread slot ts = 64 wv + lane of split z of split tile st sits
    // at float4 index ((st * S + z) * 8 + mt) * 1024 + j * 256 + ts of part.
    if (S > 1) {
        float4* mine = (float4*)part + (int64_t)((tile - full) * S + sp) * 8192 + 64 * wv + lane;
        auto store_part = [&](auto keepc) {
            constexpr int KEEP = decltype(keepc)::value;
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int mt = KEEP + t;
                    mine[(mt * 4 + j) * 256] =
                        make_float4(acc[mt][4 * j], acc[mt][4 * j + 1], acc[mt][4 * j + 2], acc[mt][4 * j + 3]);
                }
        };
        if (kh == 0) store_part(std::integral_constant<int, 0>());
        else store_part(std::integral_constant<int, 4>());
        return;
    }

    // D layout: acc[i] = D[8*(i/4) + 4*(lane/32) + i%4][lane%32].  Loads (bias, the row
    // scales, then the residual 16 values at a time) come before the stores they feed, so
    // no store has to complete before the next one is issued.  y = acc * 2^e_row (+ bias).
    const int col = n0 + 32 * wv + ln;
    if (col >= N) return;
    const float bv = bias ? bias[col] : 0.0f;
    auto store = [&](auto keepc) {
        constexpr int KEEP = decltype(keepc)::value;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int mt = KEEP + t;
            const int row0 = m0 + 32 * mt + 4 * lh;
            float v[16];
#pragma unroll
            for (int q = 0; q < 4; ++q) {  // rows row0 + 8q .. +3 (rs covers the padded rows)
                const float4 sc = *(const float4*)(rs + row0 + 8 * q);
                const float scs[4] = {sc.x, sc.y, sc.z, sc.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float a = acc[mt][4 * q + e] * scs[e];
                    v[4 * q + e] = bias ? a + bv : a;
                }
            }
            if (res) {
                float r[16];
                const float* rp = res + (int64_t)row0 * ldr + col;
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int dr = 8 * (i >> 2) + (i & 3);
                    r[i] = row0 + dr < M ? rp[(int64_t)dr * ldr] : 0.0f;
                }
#pragma unroll
                for (int i = 0; i < 16; ++i) v[i] = r[i] + v[i];
            }
            float* yp = y + (int64_t)row0 * ldy + col;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int dr = 8 * (i >> 2) + (i & 3);
                if (row0 + dr < M) yp[(int64_t)dr * ldy] = v[i];
            }
        }
    };
    if (kh == 0) store(std::integral_constant<int, 0>());
    else store(std::integral_constant<int, 4>());
}

// Second pass for split tiles: one thread per float4 slot (row tile mt, float4 j, slot
// ts) of a split tile adds the tile's S partials in split order -- the result does not
// depend on which split finished first -- and writes y like the whole-tile store:
// (sum * 2^e_row + bias), then res + that.  Slot ts = 64 wv + lane holds D[32 mt + 8 j + 4 (lane/32)
// + e][32 wv + lane % 32], e = 0..3, of the tile (the MFMA D layout above).
__global__ __launch_bounds__(256) void k_gemm_splitk_sum(const float* __restrict__ part, int S, int full,
                                                         int tiles_m, int M, int N, float* y, int64_t ldy,
                                                         const float* __restrict__ bias, const float* res, int64_t ldr,
                                                         const float* __restrict__ rs, int nslots) {
    const int g = blockIdx.x * 256 + threadIdx.x;
    if (g >= nslots) return;
    const int st = g >> 13, q = g & 8191;
    const int ts = q & 255, mt = q >> 10, j = (q >> 8) & 3;
    const int wv = ts >> 6, lane = ts & 63;
    const int tile = full + st;
    const int n0 = (tile / tiles_m) * kGemmBN, m0 = (tile % tiles_m) * kGemmBM;
    const float4* p = (const float4*)part + (int64_t)st * S * 8192 + q;
    float4 sum = p[0];
    for (int z = 1; z < S; ++z) {
        const float4 t = p[(int64_t)z * 8192];
        sum = make_float4(sum.x + t.x, sum.y + t.y, sum.z + t.z, sum.w + t.w);
    }
    const int col = n0 + 32 * wv + (lane & 31);
    if (col >= N) return;
    const float bv = bias ? bias[col] : 0.0f;
    const int row0 = m0 + 32 * mt + 8 * j + 4 * (lane >> 5);
    const float e[4] = {sum.x, sum.y, sum.z, sum.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = row0 + i;
        if (row >= M) break;
        const float a = e[i] * rs[row];
        float v = bias ? a + bv : a;
        if (res) v = res[(int64_t)row * ldr + col] + v;
        y[(int64_t)row * ldy + col] = v;
    }
}

// Work split of one GEMM over the GPU's compute units: whole tiles first, as many as fill
// every unit a whole number of times, then the remaining tiles each split along K so that
// the last round still occupies (nearly) every unit.
struct GemmPlan {
    int tiles_n = 0, tiles_m = 0, tiles = 0, full = 0, splits = 1, grid = 0;
    size_t xh_bytes = 0, rs_bytes = 0, part_bytes = 0;
};

static int device_cus() {
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

static GemmPlan gemm_plan(int64_t n, int m, int64_t k) {
    GemmPlan p;
    const int nb = (int)(k / 256);
    p.tiles_n = (int)((n + kGemmBN - 1) / kGemmBN);
    p.tiles_m = gemm_xh_rows(m) / kGemmBM;
    p.tiles = p.tiles_n * p.tiles_m;
    if (const char* e = getenv("SXQ_GEMM_SPLITS")) {  // every tile split this many ways
        p.full = 0;
        p.splits = max(1, min(atoi(e), nb));
    } else {
        const int cus = device_cus();
        p.full = p.tiles / cus * cus;
        const int rem = p.tiles - p.full;
        p.splits = rem ? max(1, min(cus / rem, nb)) : 1;
    }
    if (p.splits == 1) p.full = p.tiles;
    p.grid = p.full + (p.tiles - p.full) * p.splits;
    p.xh_bytes = ((size_t)gemm_xh_rows(m) * (size_t)k * 2 + 255) & ~(size_t)255;
    p.rs_bytes = ((size_t)gemm_xh_rows(m) * 4 + 255) & ~(size_t)255;
    const size_t split_tiles = (size_t)(p.tiles - p.full);
    p.part_bytes = split_tiles * p.splits * 128 * 256 * 4;
    return p;
}

int gemm_q4k_splits(int64_t n, int m, int64_t k) { return gemm_plan(n, m, k).splits; }

size_t gemm_q4k_workspace(int64_t n, int m, int64_t k) {
    const GemmPlan p = gemm_plan(n, m, k);
    return p.xh_bytes + p.rs_bytes + p.part_bytes;
}

hipError_t launch_gemm_q4k_prep(const float* x, int64_t ldx, int m, int64_t n, int k, void* ws, hipStream_t s) {
    const GemmPlan p = gemm_plan(n, m, k);
    const int rows = gemm_xh_rows(m);
    _Float16* xh = (_Float16*)ws;
    float* rs = (float*)((uint8_t*)ws + p.xh_bytes);
    const bool two_pass = getenv("SXQ_X2F16_TWO_PASS") != nullptr;  // A/B: the two-pass conversion
    const size_t row_lds = (size_t)k * sizeof(float);
    if (!two_pass && k <= 4096)
        hipLaunchKernelGGL(k_x_to_f16_perm1<4>, dim3((unsigned)rows), dim3(256), row_lds, s, x, ldx, m, k, xh, rs);
    else if (!two_pass && k <= 12288)
        hipLaunchKernelGGL(k_x_to_f16_perm1<12>, dim3((unsigned)rows), dim3(256), row_lds, s, x, ldx, m, k, xh, rs);
    else
        hipLaunchKernelGGL(k_x_to_f16_perm, dim3((unsigned)rows), dim3(256), 0, s, x, ldx, m, k, xh, rs);
    return hipGetLastError();
}

hipError_t launch_gemm_q4k(const QWeight& w, const void* ws, int m, float* y, int64_t ldy, const float* bias,
                           const float* res, int64_t ldr, hipStream_t s) {
    if (w.dtype != kQ4K) return hipErrorInvalidValue;
    static const hipError_t attr = hipFuncSetAttribute((const void*)k_gemm_q4k,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)gemm_q4k_lds());
    if (attr != hipSuccess) return attr;
    const GemmPlan p = gemm_plan(w.n, m, w.k);
    const float* rs = (const float*)((const uint8_t*)ws + p.xh_bytes);
    float* part = (float*)((uint8_t*)ws + p.xh_bytes + p.rs_bytes);
    hipLaunchKernelGGL(k_gemm_q4k, dim3((unsigned)p.grid), dim3(512), gemm_q4k_lds(), s, (const _Float16*)ws, m,
                       (int)w.k, (const uint4*)w.hdr, (const uint4*)w.qs, (int)w.n, y, ldy, bias, res, ldr, rs, part,
                       p.tiles_m, p.full, p.splits);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || p.full == p.tiles) return e;
    const int nslots = (p.tiles - p.full) * 8192;
    hipLaunchKernelGGL(k_gemm_splitk_sum, dim3((unsigned)((nslots + 255) / 256)), dim3(256), 0, s, (const float*)part,
                       p.splits, p.full, p.tiles_m, m, (int)w.n, y, ldy, bias, res, ldr, rs, nslots);
    return hipGetLastError();
}

}  // namespace sxq
