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
// both operands, bounded by 2^-10 * sum_k |w_k x_k| per output.
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

constexpr int kGemmBM = 128, kGemmBN = 256, kGemmStages = 4;
constexpr int kGemmStageBytes = kGemmBM * 64 * 2;   // activations of one K group: 128 rows x 64 halfs
constexpr int kGemmWStageBytes = kGemmBN * 2 * 16;  // weights of one K group: 256 rows x 2 segments
constexpr int kGemmWOff = kGemmStages * kGemmStageBytes;
constexpr int kGemmHdOff = kGemmWOff + kGemmStages * kGemmWStageBytes;  // 256 block headers

int gemm_xh_rows(int m) { return (m + kGemmBM - 1) / kGemmBM * kGemmBM; }
size_t gemm_q4k_lds() { return (size_t)kGemmHdOff + kGemmBN * 16; }

// x f32 [m][k] (row stride ldx) -> xh f16 [gemm_xh_rows(m)][k] in the GEMM K order,
// xh[r][256b + p] = f16(x[r][256b + q4k_perm_elem(p)]), rows past m zero.  Each thread
// writes 8 consecutive halfs (one MFMA operand chunk).  The first `ncount` threads also
// clear the GEMM's split counters.
__global__ __launch_bounds__(256) void k_x_to_f16_perm(const float* __restrict__ x, int64_t ldx, int m, int k,
                                                       int rows, _Float16* __restrict__ xh, unsigned* counters,
                                                       int ncount) {
    const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;  // chunk of 8 halfs
    if (c < ncount) counters[c] = 0u;
    const int kc = k >> 3;
    if (c >= (int64_t)rows * kc) return;
    const int64_t r = c / kc;
    const int p0 = (int)(c - r * kc) << 3;  // first position of the chunk within the row
    half8 v;
    if (r < m) {
        const float* src = x + r * ldx + (p0 & ~255) + q4k_perm_elem(p0 & 255);
        // j = 0..7 -> element offsets 0, 32, 8, 40, 16, 48, 24, 56 from the chunk's first
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = (_Float16)src[32 * (j & 1) + 8 * (j >> 1)];
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = (_Float16)0.0f;
    }
    *(half8*)(xh + (c << 3)) = v;
}

// The 8 (scale, min) pairs of a Q4_K block header (get_scale_min_k4), times d and dmin:
// sv[j] = d * sc_j, nm[j] = -(dmin * m_j), both exact in f32 (11-bit times 6-bit
// significands).  The 12 scale bytes are header bytes 4..15 (dwords y, z, w), taken
// with shifts so the header stays in registers; d and dmin convert in hardware.
SXQ_DEV void q4k_scales(const uint4& h, float sv[8], float nm[8]) {
    auto sc = [&](int i) -> int {
        const uint32_t d = i < 4 ? h.y : (i < 8 ? h.z : h.w);
        return (int)((d >> (8 * (i & 3))) & 0xFF);
    };
    const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(h.x & 0xFFFF));
    const float dmin = (float)__builtin_bit_cast(_Float16, (uint16_t)(h.x >> 16));
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        int scv, m;
        if (j < 4) {
            scv = sc(j) & 63;
            m = sc(j + 4) & 63;
        } else {
            scv = (sc(j + 4) & 0xF) | ((sc(j - 4) >> 6) << 4);
            m = (sc(j + 4) >> 4) | ((sc(j) >> 6) << 4);
        }
        sv[j] = d * (float)scv;
        nm[j] = -(dmin * (float)m);
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

// 16-byte global accesses coherent at agent scope (sc1: past the XCD's own L2), for the
// partial tiles one workgroup hands to another; the load's value is ready after vm_wait.
typedef float f32x4 __attribute__((ext_vector_type(4)));
SXQ_DEV void store16_agent(float* p, f32x4 v) { asm volatile("global_store_dwordx4 %0, %1, off sc1" ::"v"(p), "v"(v) : "memory"); }
SXQ_DEV f32x4 load16_agent(const float* p) {
    f32x4 r;
    asm volatile("global_load_dwordx4 %0, %1, off sc1" : "=v"(r) : "v"(p));
    return r;
}
SXQ_DEV void vm_wait0(f32x4 (&v)[6][4]) {
    asm volatile("s_waitcnt vmcnt(0)" : "+v"(v[0][0]), "+v"(v[0][1]), "+v"(v[0][2]), "+v"(v[0][3]), "+v"(v[1][0]),
                 "+v"(v[1][1]), "+v"(v[1][2]), "+v"(v[1][3]), "+v"(v[2][0]), "+v"(v[2][1]), "+v"(v[2][2]),
                 "+v"(v[2][3]));
    asm volatile("s_waitcnt vmcnt(0)" : "+v"(v[3][0]), "+v"(v[3][1]), "+v"(v[3][2]), "+v"(v[3][3]), "+v"(v[4][0]),
                 "+v"(v[4][1]), "+v"(v[4][2]), "+v"(v[4][3]), "+v"(v[5][0]), "+v"(v[5][1]), "+v"(v[5][2]),
                 "+v"(v[5][3]));
}

// Workgroup barrier without the memory fence of __syncthreads(): the fence would make
// the compiler wait for every outstanding global->LDS load, including the ones issued
// for later groups.  The caller waits for the loads it needs (SXQ_WAIT_VM); the memory
// clobber keeps the compiler from moving LDS accesses across the barrier.
SXQ_DEV void barrier_nofence() { asm volatile("s_barrier" ::: "memory"); }

// y[m][n] = x[m] . W[n] (+ bias[n], then res[m][n] + that), W Q4_K [n][k] in the device
// layout, xh from k_x_to_f16_perm (rows padded to 128).  One workgroup of 256 threads
// per tile or per split of a tile (see GemmPlan).  Wave w owns weight rows n0 + 64w .. +63 and all 128 token rows of
// the tile: 4 x 2 MFMA tiles of 32 x 32 (128 accumulators per lane).
//
// K advances in groups of 64 (a quarter block).  Every operand reaches LDS by direct
// global->LDS loads, issued 3 groups ahead into a ring of 4 stages, so no load lands in
// registers and the loop's only waits are the explicit vmcnt counts below.
//  - activations: within a stage row r's 16-byte chunk c sits at chunk slot
//    8r + (c ^ (r & 7)), so the MFMA operand reads of 32 rows spread over all banks;
//  - weights: lane (n, h) loads segment 2g + h of its two rows into its own slots and
//    reads them back itself, dequantizing each dword straight into MFMA B registers;
//  - block headers: one block ahead, decoded once per block into 16 floats per row.
// One barrier per group (for the shared activation stages).
//
// A tile split S ways: split z covers blocks [nb*z/S, nb*(z+1)/S); every split stores its
// partial tile, and the last to arrive (per-tile counter) adds the partials in split order,
// so the result does not depend on arrival order.
__global__ __launch_bounds__(256) void k_gemm_q4k(const _Float16* __restrict__ xh, int M, int K,
                                                  const uint4* __restrict__ hdr, const uint4* __restrict__ qs, int N,
                                                  float* __restrict__ y, int64_t ldy, const float* __restrict__ bias,
                                                  const float* res, int64_t ldr, float* part, unsigned* counters,
                                                  int tiles_m, int full, int splits) {
    extern __shared__ uint4 lds[];
    lds_u8* lbase = (lds_u8*)lds;
    __shared__ bool last;
    const int nb = K >> 8;
    // Workgroups 0 .. full-1 take whole tiles; the rest split the remaining tiles' K range
    // `splits` ways.  Tile t covers weight rows 256 * (t / tiles_m), token rows 128 * (t % tiles_m).
    const int id = blockIdx.x;
    const int S = id < full ? 1 : splits;
    const int tile = id < full ? id : full + (id - full) / splits;
    const int sp = id < full ? 0 : (id - full) % splits;
    const int n0 = (tile / tiles_m) * kGemmBN, m0 = (tile % tiles_m) * kGemmBM;
    const int b0 = (int)((int64_t)nb * sp / S), b1 = (int)((int64_t)nb * (sp + 1) / S);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ln = lane & 31, lh = lane >> 5;

    // Activation loads: chunk slot (4 wave + u) * 64 + lane of a stage is row
    // r = 32 wave + 8u + lane/8, chunk (lane % 8) ^ (r % 8) of the group.
    const _Float16* asrc = xh + (int64_t)(m0 + 32 * wave + (lane >> 3)) * K + 8 * ((lane & 7) ^ ((lane >> 3) & 7));
    const int64_t arow8 = (int64_t)8 * K;
    // Weight rows of this lane (rows past N clamped: loaded, never stored).
    const int64_t wr0 = min(n0 + 64 * wave + ln, N - 1), wr1 = min(n0 + 64 * wave + 32 + ln, N - 1);
    const uint4* q0 = qs + wr0 * nb * 8 + lh;
    const uint4* q1 = qs + wr1 * nb * 8 + lh;
    const uint4* hsrc = hdr + (int64_t)min(n0 + 64 * wave + lane, N - 1) * nb;  // header of row 64 wave + lane
    // LDS byte addresses of this lane's reads (stage, row tile and step offsets are
    // immediates): activation chunk of step s for row tile 0, weight segments, headers.
    uint32_t aaddr[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) aaddr[s] = lds_addr(lbase) + 16 * (8 * ln + ((2 * s + lh) ^ (ln & 7)));
    lds_u8* wlds = lbase + kGemmWOff + wave * 2048;  // + stage * kGemmWStageBytes + nt * 1024 + lane * 16
    lds_u8* hlds = lbase + kGemmHdOff + wave * 1024;  // + row-in-wave * 16
    const uint32_t waddr = lds_addr(wlds) + lane * 16, haddr = lds_addr(hlds) + ln * 16;

    auto dma = [](const void* src, lds_u8* dst) {
        __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
    };
    // the 6 loads of group grp (from the start of K) into stage st
    auto load_group = [&](int grp, int st) {
        const _Float16* src = asrc + (int64_t)grp * 64;
        lds_u8* dst = lbase + st * kGemmStageBytes + wave * 4096;
        dma(src, dst);
        dma(src + arow8, dst + 1024);
        dma(src + 2 * arow8, dst + 2048);
        dma(src + 3 * arow8, dst + 3072);
        const int wo = (grp >> 2) * 8 + 2 * (grp & 3);
        lds_u8* wd = wlds + st * kGemmWStageBytes;
        dma(q0 + wo, wd);
        dma(q1 + wo, wd + 1024);
    };
    float sv0[8], nm0[8], sv1[8], nm1[8];
    auto scales = [&]() {
        u32x4 hd0 = ds_read16<0>(haddr);
        u32x4 hd1 = ds_read16<512>(haddr);
        lgkm_wait<0>(hd0, hd1);
        q4k_scales(make_uint4(hd0[0], hd0[1], hd0[2], hd0[3]), sv0, nm0);
        q4k_scales(make_uint4(hd1[0], hd1[1], hd1[2], hd1[3]), sv1, nm1);
    };
    floatx16 acc[4][2];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[a][b][i] = 0.0f;

    // One group on stage ST.  LDS reads run ahead of the MFMAs (the 2 weight reads and
    // steps 0-1 first, step s + 2 once step s has arrived: at most 12 in flight, the lgkm
    // counter holds 15), and the B operands of step s + 1 are dequantized between the
    // MFMAs of step s, whose 32-cycle issue shadow covers about 8 VALU instructions.
    auto compute = [&](auto stc) {
        constexpr int ST = decltype(stc)::value;
        constexpr int AO = ST * kGemmStageBytes, WO = ST * kGemmWStageBytes;
        u32x4 w0 = ds_read16<WO>(waddr), w1 = ds_read16<WO + 1024>(waddr);
        u32x4 a[4][4];
        auto read_step = [&](int s) {
            a[s][0] = ds_read16<AO>(aaddr[s]);
            a[s][1] = ds_read16<AO + 4096>(aaddr[s]);
            a[s][2] = ds_read16<AO + 8192>(aaddr[s]);
            a[s][3] = ds_read16<AO + 12288>(aaddr[s]);
        };
        read_step(0);
        read_step(1);
        lgkm_wait<8>(w0, w1);
        half8 b0 = q4k_bfrag(w0[0], sv0[0], nm0[0], sv0[1], nm0[1]);
        half8 b1 = q4k_bfrag(w1[0], sv1[0], nm1[0], sv1[1], nm1[1]);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            if (s < 3) lgkm_wait<4>(a[s][0], a[s][1], a[s][2], a[s][3]);
            else lgkm_wait<0>(a[s][0], a[s][1], a[s][2], a[s][3]);
            if (s < 2) read_step(s + 2);
            half8 nb0 = b0, nb1 = b1;
            if (s < 3) {
                nb0 = q4k_bfrag(w0[s + 1], sv0[2 * s + 2], nm0[2 * s + 2], sv0[2 * s + 3], nm0[2 * s + 3]);
                nb1 = q4k_bfrag(w1[s + 1], sv1[2 * s + 2], nm1[2 * s + 2], sv1[2 * s + 3], nm1[2 * s + 3]);
            }
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                const half8 av = __builtin_bit_cast(half8, a[s][mt]);
                acc[mt][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, b0, acc[mt][0], 0, 0, 0);
                acc[mt][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, b1, acc[mt][1], 0, 0, 0);
            }
            if (s < 3) {
                // 8 x (1 MFMA, 5 VALU)
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
                }
            }
            b0 = nb0;
            b1 = nb1;
        }
    };

    // Prologue: the first block's header, groups 0..2, the first block's scales.  Every
    // group then issues exactly 6 loads and group 0 of a block also the next block's
    // header (1 load); loads past the split's end are clamped to its last group / block
    // (fetched again, never used), so the wait counts below are fixed.
    dma(hsrc + b0, hlds);
    load_group(4 * b0, 0);
    load_group(4 * b0 + 1, 1);
    load_group(4 * b0 + 2, 2);
    SXQ_WAIT_VM(18);  // the header (the 18 group loads may still be in flight)
    scales();

    const int glast = 4 * b1 - 1;  // last group of the split, from the start of K
    for (int blk = b0; blk < b1; ++blk) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            // This group's loads are complete once at most the loads issued after them
            // are outstanding: 6 for each of the next two groups, plus this block's
            // header load when that came later.  The scheduling barriers keep every load
            // in its section, so the counts stay exact.
            __builtin_amdgcn_sched_barrier(0);
            if (g == 0) SXQ_WAIT_VM(12);
            else SXQ_WAIT_VM(13);
            barrier_nofence();  // stage g is filled everywhere; stage (g + 3) % 4 is free
            __builtin_amdgcn_sched_barrier(0);
            load_group(min(4 * (g == 0 ? blk : blk + 1) + ((g + 3) & 3), glast), (g + 3) & 3);
            if (g == 0) dma(hsrc + min(blk + 1, b1 - 1), hlds);  // the header region is this wave's own
            __builtin_amdgcn_sched_barrier(0);
            if (g == 0) compute(std::integral_constant<int, 0>());
            if (g == 1) compute(std::integral_constant<int, 1>());
            if (g == 2) compute(std::integral_constant<int, 2>());
            if (g == 3) compute(std::integral_constant<int, 3>());
        }
        // the next block's header, issued in group 0: 18 group loads came after it
        __builtin_amdgcn_sched_barrier(0);
        SXQ_WAIT_VM(18);
        __builtin_amdgcn_sched_barrier(0);
        scales();
    }
    SXQ_WAIT_VM(0);  // no global->LDS load may still be in flight when the workgroup ends

    if (S > 1) {
        // Partial tile of split z of split tile st: float4 j of piece (mt, nt) of thread tid
        // at part + 4 * ((((st * S + z) * 8 + piece) * 4 + j) * 256 + tid).
        const int st = tile - full;
        float* mine = part + (int64_t)(st * S + sp) * 32768 + 4 * tid;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const f32x4 v = {acc[mt][nt][4 * j], acc[mt][nt][4 * j + 1], acc[mt][nt][4 * j + 2], acc[mt][nt][4 * j + 3]};
                    store16_agent(mine + (((mt * 2 + nt) * 4 + j) * 256) * 4, v);
                }
        if (!publish_and_count(&counters[st], (unsigned)S, &last)) return;
        // The last to arrive adds the S partials of each piece in split order (its own
        // included, read back), loading up to 6 splits' worth at once.
        const float* base = part + (int64_t)st * S * 32768 + 4 * tid;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                const int piece = mt * 2 + nt;
                f32x4 sum[4];
                for (int z0 = 0; z0 < S; z0 += 6) {
                    f32x4 t[6][4];
#pragma unroll
                    for (int dz = 0; dz < 6; ++dz)
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            t[dz][j] = z0 + dz < S ? load16_agent(base + (int64_t)(z0 + dz) * 32768 + ((piece * 4 + j) * 256) * 4)
                                                   : f32x4{0.f, 0.f, 0.f, 0.f};
                    vm_wait0(t);
#pragma unroll
                    for (int dz = 0; dz < 6; ++dz)
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            if (z0 + dz >= S) continue;
                            if (z0 + dz == 0) sum[j] = t[0][j];
                            else sum[j] = sum[j] + t[dz][j];
                        }
                }
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[mt][nt][4 * j + e] = sum[j][e];
            }
        if (tid == 0) __hip_atomic_store(&counters[st], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // D layout: acc[i] = D[8*(i/4) + 4*(lane/32) + i%4][lane%32].  Loads (bias, then the
    // residual 16 values at a time) come before the stores they feed, so no store has to
    // complete before the next one is issued.
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const int col = n0 + 64 * wave + 32 * nt + ln;
        if (col >= N) continue;
        const float bv = bias ? bias[col] : 0.0f;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            const int row0 = m0 + 32 * mt + 4 * lh;
            float v[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = bias ? acc[mt][nt][i] + bv : acc[mt][nt][i];
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
    }
}

// Work split of one GEMM over the GPU's compute units: whole tiles first, as many as fill
// every unit a whole number of times, then the remaining tiles each split along K so that
// the last round still occupies (nearly) every unit.
struct GemmPlan {
    int tiles_n = 0, tiles_m = 0, tiles = 0, full = 0, splits = 1, grid = 0;
    size_t xh_bytes = 0, part_bytes = 0, count_bytes = 0;
};

static int device_cus() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] == 0) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
        cus[dev] = v;
    }
    return cus[dev];
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
    const size_t split_tiles = (size_t)(p.tiles - p.full);
    p.part_bytes = split_tiles * p.splits * 128 * 256 * 4;
    p.count_bytes = split_tiles * 4;
    return p;
}

int gemm_q4k_splits(int64_t n, int m, int64_t k) { return gemm_plan(n, m, k).splits; }

size_t gemm_q4k_workspace(int64_t n, int m, int64_t k) {
    const GemmPlan p = gemm_plan(n, m, k);
    return p.xh_bytes + p.part_bytes + p.count_bytes;
}

hipError_t launch_gemm_q4k_prep(const float* x, int64_t ldx, int m, int64_t n, int k, void* ws, hipStream_t s) {
    const GemmPlan p = gemm_plan(n, m, k);
    const int rows = gemm_xh_rows(m);
    unsigned* counters = (unsigned*)((uint8_t*)ws + p.xh_bytes + p.part_bytes);
    const int ncount = p.tiles - p.full;
    const int64_t chunks = (int64_t)rows * (k / 8);
    const int64_t threads = chunks > ncount ? chunks : ncount;
    hipLaunchKernelGGL(k_x_to_f16_perm, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, x, ldx, m, k, rows,
                       (_Float16*)ws, counters, ncount);
    return hipGetLastError();
}

hipError_t launch_gemm_q4k(const QWeight& w, const void* ws, int m, float* y, int64_t ldy, const float* bias,
                           const float* res, int64_t ldr, hipStream_t s) {
    if (w.dtype != kQ4K) return hipErrorInvalidValue;
    static const hipError_t attr = hipFuncSetAttribute((const void*)k_gemm_q4k,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)gemm_q4k_lds());
    if (attr != hipSuccess) return attr;
    const GemmPlan p = gemm_plan(w.n, m, w.k);
    float* part = (float*)((uint8_t*)ws + p.xh_bytes);
    unsigned* counters = (unsigned*)((uint8_t*)ws + p.xh_bytes + p.part_bytes);
    hipLaunchKernelGGL(k_gemm_q4k, dim3((unsigned)p.grid), dim3(256), gemm_q4k_lds(), s, (const _Float16*)ws, m,
                       (int)w.k, (const uint4*)w.hdr, (const uint4*)w.qs, (int)w.n, y, ldy, bias, res, ldr, part,
                       counters, p.tiles_m, p.full, p.splits);
    return hipGetLastError();
}

}  // namespace sxq
