/*
 * sxq_oracle.c -- CPU restatement of Candle 0.8's quantized CPU path (generic order).
 *
 * TEST INFRASTRUCTURE ONLY (see sxq_oracle.h).  Compiled with -ffp-contract=off so
 * every float operation rounds exactly once, as Rust (which never contracts) does.
 *
 * Third-party source restated: candle-core 0.8 src/quantized/k_quants.rs
 * (BlockQ8_0/BlockQ4_0/BlockQ8K/BlockQ4K impl GgmlType, fn matmul) and
 * src/quantized/utils.rs (nearest_int, make_qkx1_quants, get_scale_min_k4).
 * Reference call sites: crates/syrinx-lm/src/cv2/load.rs:101-104 (quantize),
 * crates/syrinx-lm/src/cv2/mod.rs:195-211 (forward + bias).
 */
#include "sxq_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

_Static_assert(sizeof(ora_block_q8_0) == 34, "Q8_0 block is 34 bytes");
_Static_assert(sizeof(ora_block_q4_0) == 18, "Q4_0 block is 18 bytes");
_Static_assert(sizeof(ora_block_q8k) == 292, "Q8_K block is 292 bytes");
_Static_assert(sizeof(ora_block_q4k) == 144, "Q4_K block is 144 bytes");

#define QK8_0 32
#define QK4_0 32
#define QK_K 256

size_t ora_type_size(int dtype) {
    switch (dtype) {
    case ORA_F32: return 4;
    case ORA_F16: return 2;
    case ORA_Q4_0: return sizeof(ora_block_q4_0);
    case ORA_Q8_0: return sizeof(ora_block_q8_0);
    case ORA_Q4K: return sizeof(ora_block_q4k);
    case ORA_Q8K: return sizeof(ora_block_q8k);
    default: return 0;
    }
}

size_t ora_block_size(int dtype) {
    switch (dtype) {
    case ORA_F32:
    case ORA_F16: return 1;
    case ORA_Q4_0:
    case ORA_Q8_0: return 32;
    case ORA_Q4K:
    case ORA_Q8K: return 256;
    default: return 0;
    }
}

/* GgmlType::VecDotType: Q4_0 and Q8_0 dot against Q8_0 activations, Q4_K against Q8_K. */
int ora_vec_dot_type(int dtype) {
    switch (dtype) {
    case ORA_Q4_0:
    case ORA_Q8_0: return ORA_Q8_0;
    case ORA_Q4K: return ORA_Q8K;
    default: return -1;
    }
}

/* ---- half::f16 conversions (the `half` crate's software path; round to nearest even). */
uint16_t ora_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7FFFFFFFu) == 0) return (uint16_t)(x >> 16);
    uint32_t sign = x & 0x80000000u;
    uint32_t exp = x & 0x7F800000u;
    uint32_t man = x & 0x007FFFFFu;
    if (exp == 0x7F800000u) {
        uint32_t nan_bit = man == 0 ? 0 : 0x0200u;
        return (uint16_t)((sign >> 16) | 0x7C00u | nan_bit | (man >> 13));
    }
    uint32_t half_sign = sign >> 16;
    int32_t half_exp = (int32_t)(exp >> 23) - 127 + 15;
    if (half_exp >= 0x1F) return (uint16_t)(half_sign | 0x7C00u);
    if (half_exp <= 0) {
        if (14 - half_exp > 24) return (uint16_t)half_sign;
        uint32_t m = man | 0x00800000u;
        uint32_t half_man = m >> (14 - half_exp);
        uint32_t round_bit = 1u << (13 - half_exp);
        if ((m & round_bit) != 0 && (m & (3 * round_bit - 1)) != 0) half_man += 1;
        return (uint16_t)(half_sign | half_man);
    }
    uint32_t h = half_sign | ((uint32_t)half_exp << 10) | (man >> 13);
    uint32_t round_bit = 0x00001000u;
    if ((man & round_bit) != 0 && (man & (3 * round_bit - 1)) != 0) h += 1;
    return (uint16_t)h;
}

float ora_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t x;
    if (exp == 0) {
        if (man == 0) {
            x = sign;
        } else {
            /* subnormal: value = man * 2^-24, exact in f32 */
            float v = (float)man * 5.9604644775390625e-08f;
            memcpy(&x, &v, 4);
            x |= sign;
        }
    } else if (exp == 0x1F) {
        x = sign | 0x7F800000u | (man << 13);
    } else {
        x = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* Rust `f as i8` / `f as u8` / `f as i32`: truncate toward zero, saturate, NaN -> 0. */
static int8_t cast_i8(float v) {
    if (v != v) return 0;
    if (v >= 127.0f) return 127;
    if (v <= -128.0f) return -128;
    return (int8_t)v;
}
static uint8_t cast_u8(float v) {
    if (v != v) return 0;
    if (v >= 255.0f) return 255;
    if (v <= 0.0f) return 0;
    return (uint8_t)v;
}
static int32_t cast_i32(float v) {
    if (v != v) return 0;
    if (v >= 2147483647.0f) return 2147483647;
    if (v <= -2147483648.0f) return (int32_t)0x80000000u;
    return (int32_t)v;
}
/* Rust f32::max / f32::min: NaN-ignoring. */
static float fmax_rs(float a, float b) { return a != a ? b : (b != b ? a : (a > b ? a : b)); }
static float fmin_rs(float a, float b) { return a != a ? b : (b != b ? a : (a < b ? a : b)); }

/* utils.rs nearest_int: `v.round() as i32` (round half away from zero). */
static int32_t nearest_int(float v) { return cast_i32(roundf(v)); }

/* ---- Q8_0 (k_quants.rs BlockQ8_0::from_float / to_float) -------------------------- */
static void q8_0_from_float(const float *x, ora_block_q8_0 *y) {
    float amax = 0.0f;
    for (int i = 0; i < QK8_0; ++i) amax = fmax_rs(amax, fabsf(x[i]));
    float d = amax / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    y->d = ora_f32_to_f16(d);
    for (int i = 0; i < QK8_0; ++i) y->qs[i] = cast_i8(roundf(x[i] * id));
}
static void q8_0_to_float(const ora_block_q8_0 *b, float *y) {
    float d = ora_f16_to_f32(b->d);
    for (int i = 0; i < QK8_0; ++i) y[i] = (float)b->qs[i] * d;
}

/* ---- Q4_0 (k_quants.rs BlockQ4_0::from_float / to_float) -------------------------- */
static void q4_0_from_float(const float *x, ora_block_q4_0 *y) {
    float amax = 0.0f, max = 0.0f;
    for (int i = 0; i < QK4_0; ++i) {
        float a = fabsf(x[i]);
        if (amax < a) { amax = a; max = x[i]; }
    }
    float d = max / -8.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    y->d = ora_f32_to_f16(d);
    for (int j = 0; j < QK4_0 / 2; ++j) {
        float x0 = x[j] * id;
        float x1 = x[QK4_0 / 2 + j] * id;
        uint8_t xi0 = cast_u8(x0 + 8.5f);
        uint8_t xi1 = cast_u8(x1 + 8.5f);
        if (xi0 > 15) xi0 = 15;
        if (xi1 > 15) xi1 = 15;
        y->qs[j] = (uint8_t)(xi0 | (xi1 << 4));
    }
}
static void q4_0_to_float(const ora_block_q4_0 *b, float *y) {
    float d = ora_f16_to_f32(b->d);
    for (int j = 0; j < QK4_0 / 2; ++j) {
        int x0 = (b->qs[j] & 0x0F) - 8;
        int x1 = (b->qs[j] >> 4) - 8;
        y[j] = (float)x0 * d;
        y[j + QK4_0 / 2] = (float)x1 * d;
    }
}

/* ---- Q8_K (k_quants.rs BlockQ8K::from_float / to_float) --------------------------- */
static void q8k_from_float(const float *x, ora_block_q8k *y) {
    float max = 0.0f, amax = 0.0f;
    for (int j = 0; j < QK_K; ++j) {
        float a = fabsf(x[j]);
        if (amax < a) { amax = a; max = x[j]; }
    }
    if (amax == 0.0f) {
        y->d = 0.0f;
        memset(y->qs, 0, sizeof y->qs);
        /* bsums are left as they were (zeros() initialises them to 0). */
        memset(y->bsums, 0, sizeof y->bsums);
        return;
    }
    float iscale = -128.0f / max;
    for (int j = 0; j < QK_K; ++j) {
        float v = roundf(iscale * x[j]);
        y->qs[j] = cast_i8(fmin_rs(v, 127.0f));
    }
    for (int g = 0; g < QK_K / 16; ++g) {
        int32_t s = 0;
        for (int i = 0; i < 16; ++i) s += y->qs[g * 16 + i];
        y->bsums[g] = (int16_t)s;
    }
    y->d = 1.0f / iscale;
}
static void q8k_to_float(const ora_block_q8k *b, float *y) {
    for (int j = 0; j < QK_K; ++j) y[j] = b->d * (float)b->qs[j];
}

/* ---- Q4_K (k_quants.rs BlockQ4K; utils.rs get_scale_min_k4 / make_qkx1_quants) --- */
static void get_scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

void ora_make_qkx1_quants(int nmax, int ntry, const float *x, int n, float *scale_out,
                          float *min_out) {
    uint8_t l[QK_K];
    memset(l, 0, sizeof l);
    /* min_by / max_by with f32::total_cmp: the first minimum, the last maximum. */
    float mn = x[0], mx = x[0];
    for (int i = 0; i < n; ++i) {
        int32_t a, b;
        memcpy(&a, &x[i], 4);
        memcpy(&b, &mn, 4);
        a ^= (int32_t)(((uint32_t)(a >> 31)) >> 1);
        b ^= (int32_t)(((uint32_t)(b >> 31)) >> 1);
        if (a < b) mn = x[i];
        memcpy(&b, &mx, 4);
        b ^= (int32_t)(((uint32_t)(b >> 31)) >> 1);
        if (a >= b) mx = x[i];
    }
    if (mx == mn) {
        *scale_out = 0.0f;
        *min_out = 0.0f;
        return;
    }
    float min = fmin_rs(mn, 0.0f);
    float iscale = (float)nmax / (mx - min);
    float scale = 1.0f / iscale;
    for (int it = 0; it < ntry; ++it) {
        float sumlx = 0.0f;
        int32_t suml2 = 0;
        int did_change = 0;
        for (int i = 0; i < n; ++i) {
            int32_t li = nearest_int(iscale * (x[i] - min));
            if (li < 0) li = 0;
            if (li > nmax) li = nmax;
            if ((uint8_t)li != l[i]) {
                l[i] = (uint8_t)li;
                did_change = 1;
            }
            sumlx += (x[i] - min) * (float)li;
            suml2 += li * li;
        }
        scale = sumlx / (float)suml2;
        float sum = -0.0f;
        for (int i = 0; i < n; ++i) sum += x[i] - scale * (float)l[i];
        min = sum / (float)n;
        if (min > 0.0f) min = 0.0f;
        iscale = 1.0f / scale;
        if (!did_change) break;
    }
    *scale_out = scale;
    *min_out = -min;
}

static void q4k_from_float(const float *x, ora_block_q4k *b) {
    float mins[8], scales[8];
    memset(b, 0, sizeof *b);
    for (int j = 0; j < 8; ++j) ora_make_qkx1_quants(15, 5, x + 32 * j, 32, &scales[j], &mins[j]);
    float max_scale = 0.0f, max_min = 0.0f;
    for (int j = 0; j < 8; ++j) {
        max_scale = fmax_rs(scales[j], max_scale);
        max_min = fmax_rs(mins[j], max_min);
    }
    float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
    float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
    for (int j = 0; j < 8; ++j) {
        int32_t lsi = nearest_int(inv_scale * scales[j]);
        int32_t lmi = nearest_int(inv_min * mins[j]);
        uint8_t ls = (uint8_t)(lsi < 63 ? lsi : 63);
        uint8_t lm = (uint8_t)(lmi < 63 ? lmi : 63);
        if (j < 4) {
            b->scales[j] = ls;
            b->scales[j + 4] = lm;
        } else {
            b->scales[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
            b->scales[j - 4] |= (uint8_t)((ls >> 4) << 6);
            b->scales[j] |= (uint8_t)((lm >> 4) << 6);
        }
    }
    b->d = ora_f32_to_f16(max_scale / 63.0f);
    b->dmin = ora_f32_to_f16(max_min / 63.0f);
    uint8_t L[QK_K];
    memset(L, 0, sizeof L);
    for (int j = 0; j < 8; ++j) {
        uint8_t sc, m;
        get_scale_min_k4(j, b->scales, &sc, &m);
        float d = ora_f16_to_f32(b->d) * (float)sc;
        if (d != 0.0f) {
            float dm = ora_f16_to_f32(b->dmin) * (float)m;
            for (int ii = 0; ii < 32; ++ii) {
                int32_t lv = nearest_int((x[32 * j + ii] + dm) / d);
                if (lv < 0) lv = 0;
                if (lv > 15) lv = 15;
                L[32 * j + ii] = (uint8_t)lv;
            }
        }
    }
    for (int j = 0; j < QK_K; j += 64)
        for (int l = 0; l < 32; ++l) b->qs[(j / 64) * 32 + l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 4));
}

static void q4k_to_float(const ora_block_q4k *b, float *y) {
    float d = ora_f16_to_f32(b->d);
    float min = ora_f16_to_f32(b->dmin);
    int is = 0;
    for (int j = 0; j < QK_K; j += 64) {
        const uint8_t *q = b->qs + j / 2;
        uint8_t sc, m;
        get_scale_min_k4(is, b->scales, &sc, &m);
        float d1 = d * (float)sc, m1 = min * (float)m;
        get_scale_min_k4(is + 1, b->scales, &sc, &m);
        float d2 = d * (float)sc, m2 = min * (float)m;
        for (int l = 0; l < 32; ++l) *y++ = d1 * (float)(q[l] & 0xF) - m1;
        for (int l = 0; l < 32; ++l) *y++ = d2 * (float)(q[l] >> 4) - m2;
        is += 2;
    }
}

/* ---- row-level entry points ----------------------------------------------------- */
int ora_quantize_row(int dtype, const float *x, int64_t k, void *blocks) {
    size_t bs = ora_block_size(dtype);
    if (bs < 2 || k % (int64_t)bs != 0) return -1;
    int64_t nb = k / (int64_t)bs;
    for (int64_t i = 0; i < nb; ++i) {
        const float *xb = x + i * (int64_t)bs;
        switch (dtype) {
        case ORA_Q8_0: q8_0_from_float(xb, (ora_block_q8_0 *)blocks + i); break;
        case ORA_Q4_0: q4_0_from_float(xb, (ora_block_q4_0 *)blocks + i); break;
        case ORA_Q8K: q8k_from_float(xb, (ora_block_q8k *)blocks + i); break;
        case ORA_Q4K: q4k_from_float(xb, (ora_block_q4k *)blocks + i); break;
        default: return -1;
        }
    }
    return 0;
}

int ora_dequantize_row(int dtype, const void *blocks, int64_t k, float *y) {
    size_t bs = ora_block_size(dtype);
    if (bs < 2 || k % (int64_t)bs != 0) return -1;
    int64_t nb = k / (int64_t)bs;
    for (int64_t i = 0; i < nb; ++i) {
        float *yb = y + i * (int64_t)bs;
        switch (dtype) {
        case ORA_Q8_0: q8_0_to_float((const ora_block_q8_0 *)blocks + i, yb); break;
        case ORA_Q4_0: q4_0_to_float((const ora_block_q4_0 *)blocks + i, yb); break;
        case ORA_Q8K: q8k_to_float((const ora_block_q8k *)blocks + i, yb); break;
        case ORA_Q4K: q4k_to_float((const ora_block_q4k *)blocks + i, yb); break;
        default: return -1;
        }
    }
    return 0;
}

/* ---- vec_dot_unopt (generic accumulation order) --------------------------------- */
static float vec_dot_q8_0(int64_t n, const ora_block_q8_0 *x, const ora_block_q8_0 *y) {
    float sumf = 0.0f;
    for (int64_t b = 0; b < n / QK8_0; ++b) {
        int32_t s = 0;
        for (int i = 0; i < QK8_0; ++i) s += (int32_t)x[b].qs[i] * (int32_t)y[b].qs[i];
        sumf += (float)s * ora_f16_to_f32(x[b].d) * ora_f16_to_f32(y[b].d);
    }
    return sumf;
}

static float vec_dot_q4_0(int64_t n, const ora_block_q4_0 *x, const ora_block_q8_0 *y) {
    float sumf = 0.0f;
    for (int64_t b = 0; b < n / QK8_0; ++b) {
        int32_t s = 0;
        for (int j = 0; j < QK8_0 / 2; ++j) {
            int32_t v0 = (x[b].qs[j] & 0x0F) - 8;
            int32_t v1 = (x[b].qs[j] >> 4) - 8;
            s += v0 * (int32_t)y[b].qs[j] + v1 * (int32_t)y[b].qs[j + QK8_0 / 2];
        }
        sumf += (float)s * ora_f16_to_f32(x[b].d) * ora_f16_to_f32(y[b].d);
    }
    return sumf;
}

static float vec_dot_q4k(int64_t n, const ora_block_q4k *xs, const ora_block_q8k *ys) {
    const uint32_t kmask1 = 0x3f3f3f3fu, kmask2 = 0x0f0f0f0fu, kmask3 = 0x03030303u;
    int8_t aux8[QK_K];
    float sums[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float sumf = 0.0f;
    for (int64_t b = 0; b < n / QK_K; ++b) {
        const ora_block_q4k *x = xs + b;
        const ora_block_q8k *y = ys + b;
        int32_t aux32[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        const uint8_t *q4 = x->qs;
        int8_t *a = aux8;
        for (int c = 0; c < QK_K / 64; ++c) {
            for (int l = 0; l < 32; ++l) a[l] = (int8_t)(q4[l] & 0xF);
            a += 32;
            for (int l = 0; l < 32; ++l) a[l] = (int8_t)(q4[l] >> 4);
            a += 32;
            q4 += 32;
        }
        uint32_t utmp[4];
        memcpy(utmp, x->scales, 12); /* little-endian read_u32_into */
        utmp[3] = ((utmp[2] >> 4) & kmask2) | (((utmp[1] >> 6) & kmask3) << 4);
        uint32_t uaux = utmp[1] & kmask1;
        utmp[1] = (utmp[2] & kmask2) | (((utmp[0] >> 6) & kmask3) << 4);
        utmp[2] = uaux;
        utmp[0] &= kmask1;
        uint8_t scales[8], mins[8];
        memcpy(scales, &utmp[0], 8);
        memcpy(mins, &utmp[2], 8);
        int32_t sumi = 0;
        for (int j = 0; j < QK_K / 16; ++j) sumi += (int32_t)y->bsums[j] * (int32_t)mins[j / 2];
        const int8_t *q8 = y->qs;
        a = aux8;
        for (int s = 0; s < 8; ++s) {
            int32_t scale = scales[s];
            for (int g = 0; g < 4; ++g) {
                int16_t aux16[8];
                for (int l = 0; l < 8; ++l) aux16[l] = (int16_t)(q8[l] * a[l]);
                for (int l = 0; l < 8; ++l) aux32[l] += scale * (int32_t)aux16[l];
                q8 += 8;
                a += 8;
            }
        }
        float d = ora_f16_to_f32(x->d) * y->d;
        for (int l = 0; l < 8; ++l) sums[l] += d * (float)aux32[l];
        float dmin = ora_f16_to_f32(x->dmin) * y->d;
        sumf -= dmin * (float)sumi;
    }
    /* `sums.iter().sum::<f32>()` folds from -0.0 left to right. */
    float tot = -0.0f;
    for (int l = 0; l < 8; ++l) tot += sums[l];
    return sumf + tot;
}

float ora_vec_dot(int dtype, int64_t k, const void *w, const void *act) {
    switch (dtype) {
    case ORA_Q8_0: return vec_dot_q8_0(k, (const ora_block_q8_0 *)w, (const ora_block_q8_0 *)act);
    case ORA_Q4_0: return vec_dot_q4_0(k, (const ora_block_q4_0 *)w, (const ora_block_q8_0 *)act);
    case ORA_Q4K: return vec_dot_q4k(k, (const ora_block_q4k *)w, (const ora_block_q8k *)act);
    default: return NAN;
    }
}

/* ---- k_quants::matmul -------------------------------------------------------------- */
typedef struct {
    int dtype;
    int64_t k, n, rows;
    const uint8_t *rhs;
    const uint8_t *lhs_b;
    size_t w_row_bytes, a_row_bytes;
    float *dst;
    int64_t next; /* shared work counter (columns) */
    pthread_mutex_t mu;
} mm_job;

#define MM_CHUNK 256 /* rayon's with_min_len(128)/with_max_len(512) granularity */

static void *mm_worker(void *p) {
    mm_job *j = (mm_job *)p;
    int64_t total = j->rows * j->n;
    for (;;) {
        pthread_mutex_lock(&j->mu);
        int64_t s = j->next;
        j->next += MM_CHUNK;
        pthread_mutex_unlock(&j->mu);
        if (s >= total) break;
        int64_t e = s + MM_CHUNK < total ? s + MM_CHUNK : total;
        for (int64_t idx = s; idx < e; ++idx) {
            int64_t r = idx / j->n, c = idx % j->n;
            j->dst[idx] = ora_vec_dot(j->dtype, j->k, j->rhs + (size_t)c * j->w_row_bytes,
                                      j->lhs_b + (size_t)r * j->a_row_bytes);
        }
    }
    return NULL;
}

int ora_matmul(int dtype, int64_t m, int64_t k, int64_t n, const float *lhs, const void *rhs,
               float *dst, int threads) {
    int vdt = ora_vec_dot_type(dtype);
    if (vdt < 0) return -1;
    size_t bs = ora_block_size(dtype);
    if (k % (int64_t)bs != 0) return -1;
    size_t w_row_bytes = (size_t)(k / (int64_t)bs) * ora_type_size(dtype);
    size_t a_row_bytes = (size_t)(k / (int64_t)ora_block_size(vdt)) * ora_type_size(vdt);
    uint8_t *lhs_b = (uint8_t *)malloc(a_row_bytes * (size_t)(m > 0 ? m : 1));
    if (!lhs_b) return -1;
    /* (1) quantize every activation row, sequentially, to the vec-dot type. */
    for (int64_t r = 0; r < m; ++r) ora_quantize_row(vdt, lhs + r * k, k, lhs_b + (size_t)r * a_row_bytes);
    /* (2) every output is an independent vec_dot; run them on a pool of threads. */
    if (threads <= 0) threads = (int)sysconf(_SC_NPROCESSORS_ONLN);
    if (threads < 1) threads = 1;
    mm_job job;
    job.dtype = dtype;
    job.k = k;
    job.n = n;
    job.rows = m;
    job.rhs = (const uint8_t *)rhs;
    job.lhs_b = lhs_b;
    job.w_row_bytes = w_row_bytes;
    job.a_row_bytes = a_row_bytes;
    job.dst = dst;
    job.next = 0;
    pthread_mutex_init(&job.mu, NULL);
    if (threads == 1) {
        mm_worker(&job);
    } else {
        pthread_t *tid = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)threads);
        int started = 0;
        for (int t = 0; t < threads; ++t)
            if (pthread_create(&tid[t], NULL, mm_worker, &job) == 0) ++started;
        if (started == 0) mm_worker(&job);
        for (int t = 0; t < started; ++t) pthread_join(tid[t], NULL);
        free(tid);
    }
    pthread_mutex_destroy(&job.mu);
    free(lhs_b);
    return 0;
}

double ora_dot_f64(int dtype, int64_t k, const void *w, const float *x) {
    int vdt = ora_vec_dot_type(dtype);
    if (vdt < 0) return NAN;
    size_t a_bytes = (size_t)(k / (int64_t)ora_block_size(vdt)) * ora_type_size(vdt);
    uint8_t *ab = (uint8_t *)malloc(a_bytes);
    float *wf = (float *)malloc(sizeof(float) * (size_t)k);
    float *af = (float *)malloc(sizeof(float) * (size_t)k);
    ora_quantize_row(vdt, x, k, ab);
    ora_dequantize_row(vdt, ab, k, af);
    ora_dequantize_row(dtype, w, k, wf);
    double s = 0.0;
    for (int64_t i = 0; i < k; ++i) s += (double)wf[i] * (double)af[i];
    free(ab);
    free(wf);
    free(af);
    return s;
}

/* ---- glue ops ---------------------------------------------------------------------
 * RMSNorm: crates/syrinx-fish/src/s2/nn.rs:100-106 and crates/syrinx-lm/src/cv2/mod.rs:181-186.
 *   var = sum(x*x) * f32(1/n) + 0   (Tensor::mean_keepdim = sum / n as affine(1/n, 0))
 *   xn  = x / sqrt(var * 1 + f32(eps))   (Tensor + f64 = affine(1, eps))
 *   y   = xn * w
 * Candle's CPU sum over a contiguous row is a sequential f32 loop in a non-AVX build. */
void ora_rms_norm(const float *x, const float *w, int64_t n, double eps, float *y) {
    float s = 0.0f;
    for (int64_t i = 0; i < n; ++i) s += x[i] * x[i];
    float var = s * (float)(1.0 / (double)n) + 0.0f;
    float den = sqrtf(var * 1.0f + (float)eps);
    for (int64_t i = 0; i < n; ++i) y[i] = (x[i] / den) * w[i];
}

/* crates/syrinx-fish/src/s2/nn.rs:117-141 precompute_rope: [seq_len, head_dim/2]. */
void ora_rope_tables_interleaved(int64_t seq_len, int64_t head_dim, double base, float *cos_out,
                                 float *sin_out) {
    int64_t half = head_dim / 2;
    for (int64_t t = 0; t < seq_len; ++t)
        for (int64_t i = 0; i < half; ++i) {
            float inv = 1.0f / powf((float)base, 2.0f * (float)i / (float)head_dim);
            float a = (float)t * inv;
            cos_out[t * half + i] = cosf(a);
            sin_out[t * half + i] = sinf(a);
        }
}

/* crates/syrinx-lm/src/cv2/attention.rs:108-119 rope_cos_sin_at: [t, head_dim/2]
 * (the table there is the same half duplicated along the last dim). */
void ora_rope_tables_half(int64_t seq_len, int64_t head_dim, float theta, float *cos_out,
                          float *sin_out) {
    int64_t half = head_dim / 2;
    for (int64_t t = 0; t < seq_len; ++t)
        for (int64_t i = 0; i < half; ++i) {
            float inv = 1.0f / powf(theta, 2.0f * (float)i / (float)head_dim);
            float a = (float)t * inv;
            cos_out[t * half + i] = cosf(a);
            sin_out[t * half + i] = sinf(a);
        }
}

/* crates/syrinx-fish/src/s2/nn.rs:154-166: pairs (2i, 2i+1). */
void ora_rope_interleaved(float *x, int64_t n_heads, int64_t hd, const float *c, const float *s) {
    for (int64_t h = 0; h < n_heads; ++h) {
        float *v = x + h * hd;
        for (int64_t i = 0; i < hd / 2; ++i) {
            float x0 = v[2 * i], x1 = v[2 * i + 1];
            v[2 * i] = x0 * c[i] - x1 * s[i];
            v[2 * i + 1] = x1 * c[i] + x0 * s[i];
        }
    }
}

/* crates/syrinx-lm/src/cv2/attention.rs:82-88: x*cos + cat(-x2, x1)*sin. */
void ora_rope_half(float *x, int64_t n_heads, int64_t hd, const float *c, const float *s) {
    int64_t half = hd / 2;
    for (int64_t h = 0; h < n_heads; ++h) {
        float *v = x + h * hd;
        for (int64_t i = 0; i < half; ++i) {
            float x1 = v[i], x2 = v[i + half];
            v[i] = x1 * c[i] + (-x2) * s[i];
            v[i + half] = x2 * c[i] + x1 * s[i];
        }
    }
}

/* candle_nn::ops::softmax over the last dim: max, exp(x - max), sum, divide. */
void ora_softmax(float *x, int64_t n) {
    float m = -INFINITY;
    for (int64_t i = 0; i < n; ++i) m = fmax_rs(m, x[i]);
    float s = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        x[i] = expf(x[i] - m);
        s += x[i];
    }
    for (int64_t i = 0; i < n; ++i) x[i] = x[i] / s;
}

/* candle's unary silu: v / (1 + exp(-v)). */
float ora_silu(float v) { return v / (1.0f + expf(-v)); }

void ora_silu_mul(const float *g, const float *u, int64_t n, float *out) {
    for (int64_t i = 0; i < n; ++i) out[i] = ora_silu(g[i]) * u[i];
}

/* crates/syrinx-fish/src/s2/nn.rs:340-351 (and cv2/attention.rs:67-75) for one
 * decode query: scores = (q . k_j) * f32(1/sqrt(hd)), softmax, sum_j p_j v_j. */
void ora_attend_one(const float *q, const float *kc, const float *vc, int64_t L, int64_t hd,
                    float *out) {
    float *sc = (float *)malloc(sizeof(float) * (size_t)(L > 0 ? L : 1));
    float scale = (float)(1.0 / sqrt((double)hd));
    for (int64_t j = 0; j < L; ++j) {
        float d = 0.0f;
        for (int64_t i = 0; i < hd; ++i) d += q[i] * kc[j * hd + i];
        sc[j] = d * scale + 0.0f;
    }
    ora_softmax(sc, L);
    for (int64_t i = 0; i < hd; ++i) {
        float a = 0.0f;
        for (int64_t j = 0; j < L; ++j) a += sc[j] * vc[j * hd + i];
        out[i] = a;
    }
    free(sc);
}
