// sxq_common.h -- shared definitions for the gfx950 quantized-linear library.
//
// Block formats are GGML's (the byte layout candle-core 0.8 stores in a QTensor and
// that QTensor::quantize produces, as called at crates/syrinx-lm/src/cv2/load.rs:101-104):
//   Q8_0 {f16 d; i8 qs[32]}  Q4_0 {f16 d; u8 qs[16]}
//   Q4_K {f16 d; f16 dmin; u8 scales[12]; u8 qs[128]}  Q8_K {f32 d; i8 qs[256]; i16 bsums[16]}
// On the device the library keeps its own layouts (see DevLayout below); the canonical
// bytes only cross the C-ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#define SXQ_HD __host__ __device__ __forceinline__
#define SXQ_DEV __device__ __forceinline__

namespace sxq {

enum DType : int {
    kF32 = 0,
    kF16 = 1,
    kQ4_0 = 2,
    kQ8_0 = 8,
    kQ4K = 12,
    kQ8K = 15,
    kBF16 = 30,
};

struct BlockQ8_0 { uint16_t d; int8_t qs[32]; };
struct BlockQ4_0 { uint16_t d; uint8_t qs[16]; };
struct BlockQ8K { float d; int8_t qs[256]; int16_t bsums[16]; };
struct BlockQ4K { uint16_t d; uint16_t dmin; uint8_t scales[12]; uint8_t qs[128]; };
static_assert(sizeof(BlockQ8_0) == 34, "Q8_0 block is 34 bytes");
static_assert(sizeof(BlockQ4_0) == 18, "Q4_0 block is 18 bytes");
static_assert(sizeof(BlockQ8K) == 292, "Q8_K block is 292 bytes");
static_assert(sizeof(BlockQ4K) == 144, "Q4_K block is 144 bytes");

SXQ_HD int block_size(int dt) {
    return (dt == kQ4_0 || dt == kQ8_0) ? 32 : (dt == kQ4K || dt == kQ8K) ? 256 : (dt == kF32 || dt == kF16 || dt == kBF16) ? 1 : 0;
}
SXQ_HD int type_size(int dt) {
    switch (dt) {
    case kF32: return 4;
    case kF16: return 2;
    case kBF16: return 2;
    case kQ4_0: return 18;
    case kQ8_0: return 34;
    case kQ4K: return 144;
    case kQ8K: return 292;
    default: return 0;
    }
}
SXQ_HD int vec_dot_type(int dt) { return (dt == kQ4_0 || dt == kQ8_0) ? kQ8_0 : (dt == kQ4K ? kQ8K : -1); }

// ---------------------------------------------------------------------------------
// Device activation layouts (what the GEMV prologue copies into LDS).
//
// Q8_K activation block, 304 bytes, 16-byte aligned:
//   qs  : 256 int8 in "class-major" order: dword (8*l + j) holds the four elements
//         32*j + l + 8*t (t = 0..3) of sub-block j whose index mod 8 is l.  This is the
//         order in which Candle's generic Q4_K x Q8_K vec-dot keeps its eight integer
//         lane sums (aux32[l]), so one dword x one weight dword gives one lane partial.
//   d   : f32 scale
//   bs2 : int32[8], bs2[j] = bsums[2j] + bsums[2j+1] (the sum of sub-block j's 32 q's)
struct ActQ8K {
    int8_t qs[256];
    float d;
    int32_t pad[3];
    int32_t bs2[8];
};
static_assert(sizeof(ActQ8K) == 304, "ActQ8K is 304 bytes");

// Q8_0 activation block, 48 bytes: qs in element order, d = f32(f16(d)) (the value the
// vec-dot multiplies by), asum = sum of qs (used by Q4_0's "- 8" offset).
struct ActQ8_0 {
    int8_t qs[32];
    float d;
    int32_t asum;
    int32_t pad[2];
};
static_assert(sizeof(ActQ8_0) == 48, "ActQ8_0 is 48 bytes");

SXQ_HD size_t act_block_bytes(int vdt) { return vdt == kQ8K ? sizeof(ActQ8K) : sizeof(ActQ8_0); }

// The same Q8_K activations of up to 16 rows, one record per 256-element block column,
// laid out as the operands of the Q4_K matrix-core GEMV (v_mfma_f32_16x16x32_f16, the
// activation rows as its 16 rows), written by the quantizers next to the ActQ8K rows:
//   q  : q[l][r][g][s] = the f16 value of the q8 at qs[32 l + 8 g + {0,2,1,3,4,6,5,7}[s]]
//        of row r (class l, lane group g: the eight k-slots lane (r, g) feeds)
//   d  : d[r], the rows' scales
//   bs : bs[h][r][g] = (float) bs2[g + 4 h] of row r
// Rows a step does not have are never written and never read into a stored result.
struct MmaRec {
    _Float16 q[8][16][4][8];
    float d[16];
    float bs[2][16][4];
};
static_assert(sizeof(MmaRec) == 8768, "MmaRec is 8768 bytes");

// Weight device layouts (repacked once at QMatMul creation; same total bytes as the
// canonical blocks):
//   Q4_K: hdr[n*nb] 16 B (d, dmin, scales[12], unchanged) + qs[n*nb] 128 B where
//         dword (4*l + c) holds canonical qs bytes {32c + l + 8t, t = 0..3}: lane l of
//         an 8-lane group loads 16 contiguous bytes = its class-l bytes of all 4 chunks.
//   Q8_0: d[n*nb] f16 + qs[n*nb] 32 B.      Q4_0: d[n*nb] f16 + qs[n*nb] 16 B.
SXQ_HD size_t weight_qs_bytes(int dt) { return dt == kQ4K ? 128 : dt == kQ8_0 ? 32 : dt == kQ4_0 ? 16 : 0; }
SXQ_HD size_t weight_hdr_bytes(int dt) { return dt == kQ4K ? 16 : (dt == kQ8_0 || dt == kQ4_0) ? 2 : 0; }

// ---------------------------------------------------------------------------------
// f16 <-> f32.  f32 -> f16 is round-to-nearest-even with the `half` crate's handling
// of overflow, subnormals and NaN, written out in integer arithmetic so it does not
// depend on the hardware conversion's denormal mode.
SXQ_HD uint16_t f32_to_f16_bits(float f) {
    uint32_t x = __builtin_bit_cast(uint32_t, f);
    if ((x & 0x7FFFFFFFu) == 0) return (uint16_t)(x >> 16);
    uint32_t sign = x & 0x80000000u, exp = x & 0x7F800000u, man = x & 0x007FFFFFu;
    if (exp == 0x7F800000u) return (uint16_t)((sign >> 16) | 0x7C00u | (man ? 0x0200u : 0u) | (man >> 13));
    uint32_t hs = sign >> 16;
    int32_t he = (int32_t)(exp >> 23) - 112;
    if (he >= 0x1F) return (uint16_t)(hs | 0x7C00u);
    if (he <= 0) {
        if (14 - he > 24) return (uint16_t)hs;
        uint32_t m = man | 0x00800000u;
        uint32_t hm = m >> (14 - he);
        uint32_t rb = 1u << (13 - he);
        if ((m & rb) && (m & (3u * rb - 1u))) hm += 1;
        return (uint16_t)(hs | hm);
    }
    uint32_t h = hs | ((uint32_t)he << 10) | (man >> 13);
    if ((man & 0x1000u) && (man & 0x2FFFu)) h += 1;
    return (uint16_t)h;
}

SXQ_HD float f16_bits_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu;
    if (exp == 0) {
        float v = (float)man * 5.9604644775390625e-08f;  // man * 2^-24, exact
        return __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, v) | sign);
    }
    if (exp == 0x1F) return __builtin_bit_cast(float, sign | 0x7F800000u | (man << 13));
    return __builtin_bit_cast(float, sign | ((exp + 112u) << 23) | (man << 13));
}

// Rust `v as i8` for an already-rounded value (saturating; NaN -> 0).  Written as a
// clamp and a select so the device code has no branches.
SXQ_HD int sat_i8(float v) {
    const int c = (int)fminf(fmaxf(v, -128.0f), 127.0f);
    return v != v ? 0 : c;
}

// ---------------------------------------------------------------------------------
// Cross-lane helpers (wave64).  DPP controls: quad_perm xor1 = 0xB1, xor2 = 0x4E,
// row_half_mirror = 0x141 (lane i <-> 7 - i inside each 8-lane half row).
SXQ_DEV int dpp_xor1(int v) { return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false); }
SXQ_DEV int dpp_xor2(int v) { return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false); }
SXQ_DEV int dpp_hmirror(int v) { return __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false); }
// Integer sum over the 8 lanes of an aligned 8-lane group; every lane gets the total.
SXQ_DEV int sum8_i32(int v) {
    v += dpp_xor1(v);
    v += dpp_xor2(v);
    v += dpp_hmirror(v);
    return v;
}

}  // namespace sxq
