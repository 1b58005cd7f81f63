/* Drives every function of the CPU oracle (oracle/sxq_oracle.c) over random and edge-case
 * inputs under AddressSanitizer + UndefinedBehaviorSanitizer (tests/sanitize/Makefile).
 * Test infrastructure only: any out-of-bounds access, use of freed memory, signed
 * overflow, misaligned load or invalid shift aborts the run; "ok" on success. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../oracle/sxq_oracle.h"

static uint64_t rng_state = 0x1234567u;
static float frand(void) {  /* xorshift64, uniform in [-1, 1) */
    rng_state ^= rng_state << 13;
    rng_state ^= rng_state >> 7;
    rng_state ^= rng_state << 17;
    return (float)((rng_state >> 11) * (1.0 / 9007199254740992.0)) * 2.0f - 1.0f;
}

static void fill(float *x, int64_t n, int kind) {
    for (int64_t i = 0; i < n; ++i) {
        switch (kind) {
        case 0: x[i] = frand(); break;                          /* plain */
        case 1: x[i] = 0.0f; break;                             /* all-zero blocks */
        case 2: x[i] = frand() * 1e30f; break;                  /* huge */
        case 3: x[i] = frand() * 1e-30f; break;                 /* tiny (f16 underflow) */
        default: x[i] = (i % 7 == 0) ? 3.0f : -3.0f; break;     /* ties at the maximum */
        }
    }
}

static int check_dtype(int dt, int64_t k, int64_t n, int64_t m, int kind) {
    const int vdt = ora_vec_dot_type(dt);
    const size_t bs = ora_block_size(dt), ts = ora_type_size(dt);
    const size_t vbs = ora_block_size(vdt), vts = ora_type_size(vdt);
    const size_t wrow = (size_t)(k / (int64_t)bs) * ts, arow = (size_t)(k / (int64_t)vbs) * vts;
    float *w = malloc(sizeof(float) * n * k), *x = malloc(sizeof(float) * m * k), *y = malloc(sizeof(float) * k);
    float *dst1 = malloc(sizeof(float) * m * n), *dst4 = malloc(sizeof(float) * m * n);
    uint8_t *wb = malloc(wrow * n), *ab = malloc(arow);
    fill(w, n * k, kind);
    fill(x, m * k, kind == 2 ? 0 : kind);
    for (int64_t r = 0; r < n; ++r)
        if (ora_quantize_row(dt, w + r * k, k, wb + r * wrow)) return 1;
    if (ora_dequantize_row(dt, wb, k, y)) return 2;
    if (ora_quantize_row(vdt, x, k, ab)) return 3;
    volatile float d = ora_vec_dot(dt, k, wb, ab);
    volatile double d64 = ora_dot_f64(dt, k, wb, x);
    (void)d;
    (void)d64;
    if (ora_matmul(dt, m, k, n, x, wb, dst1, 1) || ora_matmul(dt, m, k, n, x, wb, dst4, 4)) return 4;
    if (memcmp(dst1, dst4, sizeof(float) * m * n)) return 5;  /* thread count never changes a bit */
    if (ora_quantize_row(dt, w, k + 1, wb) != -1) return 6;    /* misaligned k is refused */
    free(w), free(x), free(y), free(dst1), free(dst4), free(wb), free(ab);
    return 0;
}

int main(void) {
    const int dts[] = {2, 8, 12};  /* Q4_0, Q8_0, Q4_K */
    for (int i = 0; i < 3; ++i)
        for (int kind = 0; kind < 5; ++kind) {
            const int64_t k = dts[i] == 12 ? 512 : 96;
            const int rc = check_dtype(dts[i], k, 37, 3, kind);
            if (rc) {
                fprintf(stderr, "dtype %d kind %d: check %d failed\n", dts[i], kind, rc);
                return 1;
            }
        }
    float xs[32], sc = 0.0f, mn = 0.0f;
    fill(xs, 32, 0);
    ora_make_qkx1_quants(15, 5, xs, 32, &sc, &mn);
    fill(xs, 32, 1);
    ora_make_qkx1_quants(15, 5, xs, 32, &sc, &mn);
    for (int i = 0; i < 4096; ++i) {
        const uint16_t h = ora_f32_to_f16(frand() * 70000.0f);
        (void)ora_f16_to_f32(h);
    }
    (void)ora_f16_to_f32(0x7C00u), (void)ora_f16_to_f32(0x0001u), (void)ora_f32_to_f16(NAN);
    enum { H = 4, HD = 64, L = 9, S = 12 };
    float q[H * HD], w[HD], out[HD], cs[S * HD / 2], sn[S * HD / 2], kc[L * HD], vc[L * HD], g[HD], u[HD];
    fill(q, H * HD, 0), fill(w, HD, 0), fill(kc, L * HD, 0), fill(vc, L * HD, 0), fill(g, HD, 0), fill(u, HD, 0);
    ora_rms_norm(q, w, HD, 1e-6, out);
    ora_rope_tables_interleaved(S, HD, 1e6, cs, sn);
    ora_rope_interleaved(q, H, HD, cs + 5 * HD / 2, sn + 5 * HD / 2);
    ora_rope_tables_half(S, HD, 1e6f, cs, sn);
    ora_rope_half(q, H, HD, cs + 7 * HD / 2, sn + 7 * HD / 2);
    ora_softmax(q, H * HD);
    (void)ora_silu(-100.0f), (void)ora_silu(100.0f);
    ora_silu_mul(g, u, HD, out);
    ora_attend_one(q, kc, vc, L, HD, out);
    ora_attend_one(q, kc, vc, 1, HD, out);
    puts("ok");
    return 0;
}
