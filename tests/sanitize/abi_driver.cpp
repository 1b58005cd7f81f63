// Drives libsxq's host code through the C-ABI calls that need no GPU -- argument checks,
// Candle's error texts, the thread-local error string, block geometry, embedding schemes,
// handle-less calls -- under AddressSanitizer + UndefinedBehaviorSanitizer, against a
// host-only build of every source (tests/sanitize/Makefile).  Test infrastructure only;
// prints "ok" on success.
#include <cstdio>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/sxq.h"

#define EXPECT(c)                                                  \
    do {                                                           \
        if (!(c)) {                                                \
            std::fprintf(stderr, "failed: %s (line %d)\n", #c, __LINE__); \
            return 1;                                              \
        }                                                          \
    } while (0)

static int checks() {
    EXPECT(sxq_block_size(SXQ_Q4K) == 256 && sxq_type_size(SXQ_Q4K) == 144 && sxq_block_size(99) == 0);
    EXPECT(sxq_version() != nullptr && std::strlen(sxq_version()) > 0);
    sxq_qmm* h = nullptr;
    EXPECT(sxq_qmm_create(0, SXQ_Q4K, 10, 896, nullptr, 0, 0, &h) == SXQ_ERR_BLOCK_ALIGN && !h);
    EXPECT(std::strcmp(sxq_last_error(),
                       "quantized tensor must have their last dim divisible by block size [10, 896] 256") == 0);
    EXPECT(sxq_qmm_create(0, 3, 10, 896, nullptr, 0, 0, &h) == SXQ_ERR_DTYPE);
    EXPECT(sxq_qmm_create(0, SXQ_Q8_0, 10, 896, nullptr, 100, 0, &h) == SXQ_ERR_SHAPE);
    EXPECT(std::strstr(sxq_last_error(), "needs 9520") != nullptr);
    EXPECT(sxq_qmm_create(0, SXQ_Q8_0, 0, 896, nullptr, 0, 0, &h) == SXQ_ERR_INVALID);
    int64_t shape[2] = {1, 896};
    EXPECT(sxq_qmm_forward(nullptr, nullptr, shape, 2, nullptr, nullptr, nullptr, 0, nullptr) == SXQ_ERR_INVALID);
    EXPECT(sxq_qmm_destroy(nullptr) == SXQ_OK);
    EXPECT(sxq_quantize_rows(0, SXQ_Q4K, nullptr, 4, 896, nullptr, nullptr) == SXQ_ERR_BLOCK_ALIGN);
    size_t sz = 7;
    EXPECT(sxq_qmm_workspace_size(nullptr, 1, 0, &sz) == SXQ_ERR_INVALID);
    EXPECT(sxq_qmm_forward_ws(nullptr, nullptr, shape, 2, nullptr, nullptr, nullptr, 0, nullptr, 0, nullptr) ==
           SXQ_ERR_INVALID);
    EXPECT(std::strstr(sxq_last_error(), "null handle") != nullptr);
    int eff = 0;
    EXPECT(sxq_embed_scheme(4, 896, &eff) == SXQ_OK && eff == 4);
    EXPECT(sxq_embed_scheme(4, 81, &eff) == SXQ_OK && eff == 8);
    EXPECT(sxq_embed_scheme(5, 896, &eff) == SXQ_ERR_INVALID);
    EXPECT(sxq_lm_reset(nullptr, 1, nullptr) == SXQ_ERR_INVALID);
    EXPECT(sxq_lm_create(0, nullptr, nullptr) == SXQ_ERR_INVALID);
    sxq_lm_config c{};
    sxq_lm* lm = nullptr;
    c.n_layers = 1;  // every other size left 0: refused before any device call
    EXPECT(sxq_lm_create(0, &c, &lm) == SXQ_ERR_INVALID && !lm);
    EXPECT(sxq_fish_fast_expand(nullptr, 1, nullptr, nullptr, 1, nullptr, nullptr, nullptr, 10, nullptr, 1, 0,
                                nullptr) == SXQ_ERR_INVALID);
    sxq_fish_sampling p{};
    p.top_k = -1;
    EXPECT(sxq_sample_codebook(0, nullptr, 0, 1, 16, &p, nullptr, nullptr, 0, nullptr, nullptr, 1, nullptr) ==
           SXQ_ERR_INVALID);
    EXPECT(sxq_sample_ras(0, nullptr, 0, 1, 16, 0, 0, 0, 0.8f, 65, 10, 0.1f, nullptr, nullptr, nullptr, nullptr, 1,
                          nullptr) == SXQ_ERR_INVALID);
    return 0;
}

int main() {
    if (checks()) return 1;
    // the error text is thread-local: concurrent failures never see each other's message
    std::vector<std::thread> ts;
    int bad = 0;
    for (int t = 0; t < 8; ++t)
        ts.emplace_back([t, &bad] {
            for (int i = 0; i < 200; ++i) {
                sxq_qmm* h = nullptr;
                const int64_t k = 896 + 32 * (2 * t + 1);  // never a multiple of 256
                sxq_qmm_create(0, SXQ_Q4K, 10 + t, k, nullptr, 0, 0, &h);
                char want[128];
                std::snprintf(want, sizeof want,
                              "quantized tensor must have their last dim divisible by block size [%d, %lld] 256",
                              10 + t, (long long)k);
                if (std::strcmp(sxq_last_error(), want) != 0) __atomic_add_fetch(&bad, 1, __ATOMIC_RELAXED);
            }
        });
    for (auto& th : ts) th.join();
    if (bad) {
        std::fprintf(stderr, "%d thread-local error texts crossed threads\n", bad);
        return 1;
    }
    std::puts("ok");
    return 0;
}
