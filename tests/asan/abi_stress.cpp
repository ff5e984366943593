// abi_stress.cpp -- drives the host code of libenchip's C ABI (include/enchip.h) for a
// host AddressSanitizer build (tests/asan/Makefile): every host-buffer entry point, the
// weight swizzle and image round trip at ragged shapes, scratch growth and the scratch-cap
// decline, every argument-error path, truncated name buffers, the thread-local error
// messages from 8 threads, releases and a close with weights still registered. The
// numerics are checked elsewhere (tests/test_gpu_*.py); here a result is only checked for
// what needs no reference: finite outputs, exact ones where the inputs make them exact.
// Exit status 0 when every check holds; AddressSanitizer aborts on a memory error.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <thread>
#include <vector>

#include "enchip.h"

static int g_fail = 0;

#define CHECK(cond, ...)                                                   \
    do {                                                                   \
        if (!(cond)) {                                                     \
            std::fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__);      \
            std::fprintf(stderr, __VA_ARGS__);                             \
            std::fprintf(stderr, "\n");                                    \
            ++g_fail;                                                      \
        }                                                                  \
    } while (0)

static std::vector<float> randf(std::mt19937 &g, size_t n, float sd = 1.0f) {
    std::normal_distribution<float> d(0.0f, sd);
    std::vector<float> v(n);
    for (auto &x : v) x = d(g);
    return v;
}

static std::vector<int8_t> randq(std::mt19937 &g, size_t n) {
    std::uniform_int_distribution<int> d(-128, 127);
    std::vector<int8_t> v(n);
    for (auto &x : v) x = (int8_t)d(g);
    return v;
}

static bool all_finite(const std::vector<float> &v) {
    for (float x : v)
        if (!std::isfinite(x)) return false;
    return true;
}

// Weight registration, shape query, export and re-registration of the image, at ragged N, K.
static void weights(enchip_ctx *ctx, std::mt19937 &g) {
    const int64_t shapes[][2] = {{1, 1}, {33, 7}, {300, 100}, {257, 1000}, {768, 768}, {64, 0}};
    for (auto &s : shapes) {
        const int64_t N = s[0], K = s[1];
        auto wq = randq(g, (size_t)(N * K));
        std::vector<float> ws(N, 0.01f);
        enchip_weight w = 0;
        CHECK(enchip_weight_register(ctx, K ? wq.data() : nullptr, ws.data(), N, K, &w) == ENCHIP_OK,
              "register N=%lld K=%lld: %s", (long long)N, (long long)K, enchip_last_error(ctx));
        int64_t n = -1, k = -1;
        CHECK(enchip_weight_shape(ctx, w, &n, &k) == ENCHIP_OK && n == N && k == K, "shape");
        const int64_t bytes = enchip_weight_image_bytes(N, K);
        CHECK(bytes > 0, "image bytes");
        std::vector<int8_t> img((size_t)bytes);
        std::vector<float> sc(N);
        CHECK(enchip_weight_export(ctx, w, img.data(), bytes, sc.data()) == ENCHIP_OK, "export");
        CHECK(enchip_weight_export(ctx, w, img.data(), bytes - 1, nullptr) == ENCHIP_ERR_ARG, "export short");
        enchip_weight w2 = 0;
        CHECK(enchip_weight_register_image(ctx, img.data(), bytes, sc.data(), N, K, &w2) == ENCHIP_OK, "image");
        CHECK(enchip_weight_register_image(ctx, img.data(), bytes + 1, sc.data(), N, K, &w2) == ENCHIP_ERR_ARG,
              "image size");
        std::vector<int8_t> img2((size_t)bytes);
        enchip_weight w3 = 0;
        CHECK(enchip_weight_register_image(ctx, img.data(), bytes, sc.data(), N, K, &w3) == ENCHIP_OK, "image 2");
        CHECK(enchip_weight_export(ctx, w3, img2.data(), bytes, nullptr) == ENCHIP_OK && img == img2, "round trip");
        CHECK(enchip_weight_release(ctx, w) == ENCHIP_OK, "release");
        CHECK(enchip_weight_release(ctx, w) == ENCHIP_ERR_HANDLE, "double release");
        enchip_weight_release(ctx, w3);
        // w2 stays registered: enchip_close frees it
    }
    enchip_weight w = 0;
    CHECK(enchip_weight_register(ctx, nullptr, nullptr, 4, 4, &w) == ENCHIP_ERR_ARG, "null register");
    CHECK(enchip_weight_register(ctx, nullptr, nullptr, 0, 4, &w) == ENCHIP_ERR_ARG, "N=0");
    CHECK(enchip_weight_register(ctx, nullptr, nullptr, 4, 4, nullptr) == ENCHIP_ERR_ARG, "null out");
    CHECK(enchip_weight_image_bytes(-1, 4) == -1, "bad image shape");
}

// The host-buffer compute entry points at several shapes (each routing to other kernels).
static void compute(enchip_ctx *ctx, std::mt19937 &g) {
    const int64_t shapes[][3] = {{1, 768, 768}, {16, 768, 3072}, {33, 100, 257}, {200, 768, 300}, {1000, 384, 1536}};
    for (auto &s : shapes) {
        const int64_t M = s[0], K = s[1], N = s[2];
        auto wq = randq(g, (size_t)(N * K));
        std::vector<float> ws(N, 0.003f);
        enchip_weight w = 0;
        CHECK(enchip_weight_register(ctx, wq.data(), ws.data(), N, K, &w) == ENCHIP_OK, "register");
        auto a = randf(g, (size_t)(M * K));
        auto bias = randf(g, (size_t)N, 0.1f);
        std::vector<float> dst((size_t)(M * N)), dst2((size_t)(M * N));
        std::vector<int32_t> acc((size_t)(M * N));
        CHECK(enchip_w8a8_linear(ctx, w, a.data(), M, bias.data(), ENCHIP_ACT_GELU, dst.data(), acc.data()) == ENCHIP_OK,
              "linear: %s", enchip_last_error(ctx));
        CHECK(all_finite(dst), "linear finite");
        // the batch of two ops equals two single calls, bit for bit
        enchip_op ops[2] = {{w, bias.data(), ENCHIP_ACT_NONE, dst.data()}, {w, nullptr, ENCHIP_ACT_GELU, dst2.data()}};
        CHECK(enchip_w8a8_batch(ctx, a.data(), M, K, ops, 2) == ENCHIP_OK, "batch");
        std::vector<float> one((size_t)(M * N));
        CHECK(enchip_w8a8_linear(ctx, w, a.data(), M, nullptr, ENCHIP_ACT_GELU, one.data(), nullptr) == ENCHIP_OK, "l");
        CHECK(std::memcmp(one.data(), dst2.data(), one.size() * 4) == 0, "batch == single");
        // weight-only product and its finite result
        CHECK(enchip_matmul_bt_q8(ctx, w, a.data(), M, dst.data()) == ENCHIP_OK, "q8: %s", enchip_last_error(ctx));
        CHECK(all_finite(dst), "q8 finite");
        // quantizer alone
        std::vector<int8_t> aq((size_t)(M * K));
        std::vector<float> as((size_t)M);
        CHECK(enchip_quant_rows(ctx, a.data(), M, K, aq.data(), as.data()) == ENCHIP_OK, "quant");
        // f32 MatmulBT on integer operands (exact in any order): against a host loop
        std::vector<float> ai((size_t)(M * K)), bi((size_t)(N * K)), c((size_t)(M * N));
        for (size_t i = 0; i < ai.size(); ++i) ai[i] = (float)((int)(i * 7 % 9) - 4);
        for (size_t i = 0; i < bi.size(); ++i) bi[i] = (float)((int)(i * 5 % 7) - 3);
        CHECK(enchip_matmul_bt_f32(ctx, ai.data(), bi.data(), c.data(), M, K, N) == ENCHIP_OK, "f32");
        bool exact = true;
        for (int64_t m = 0; m < M && exact; m += 97)
            for (int64_t n = 0; n < N; n += 31) {
                double r = 0;
                for (int64_t k = 0; k < K; ++k) r += (double)ai[m * K + k] * bi[n * K + k];
                exact &= (double)c[m * N + n] == r;
            }
        CHECK(exact, "f32 exact on integers");
        // kernel names, truncated
        char name[8];
        CHECK(enchip_gemm_kernel_name(ctx, w, M, ENCHIP_ACT_GELU, name, (int)sizeof name) == ENCHIP_OK, "name");
        CHECK(std::strlen(name) < sizeof name, "name truncated");
        // argument errors leave dst alone
        std::vector<float> keep((size_t)(M * N), 7.0f);
        CHECK(enchip_w8a8_linear(ctx, w, a.data(), M, nullptr, 9, keep.data(), nullptr) == ENCHIP_ERR_ARG, "act");
        CHECK(enchip_w8a8_linear(ctx, w + 1000, a.data(), M, nullptr, 0, keep.data(), nullptr) == ENCHIP_ERR_HANDLE,
              "handle");
        CHECK(enchip_w8a8_linear(ctx, w, nullptr, M, nullptr, 0, keep.data(), nullptr) == ENCHIP_ERR_ARG, "null a");
        CHECK(enchip_matmul_bt_q8(ctx, w, a.data(), -1, keep.data()) == ENCHIP_ERR_ARG, "q8 M");
        bool kept = true;
        for (float x : keep) kept &= x == 7.0f;
        CHECK(kept, "declines leave dst");
        CHECK(enchip_weight_release(ctx, w) == ENCHIP_OK, "release");
    }
    // ann top-k on a small index (two-pass route), and the stats
    {
        const int64_t n = 4096, K = 64, M = 5, k = 7;
        auto wq = randq(g, (size_t)(n * K));
        std::vector<float> ws(n, 0.01f);
        enchip_weight idx = 0;
        CHECK(enchip_weight_register(ctx, wq.data(), ws.data(), n, K, &idx) == ENCHIP_OK, "index");
        auto q = randf(g, (size_t)(M * K));
        std::vector<int32_t> hi((size_t)(M * k));
        std::vector<float> hs((size_t)(M * k));
        CHECK(enchip_ann_topk(ctx, idx, q.data(), M, k, hi.data(), hs.data()) == ENCHIP_OK, "topk");
        for (int32_t i : hi) CHECK(i >= 0 && i < n, "hit index %d", i);
        int64_t fused = -1, fb = -1;
        CHECK(enchip_ann_topk_stats(ctx, &fused, &fb) == ENCHIP_OK && fused >= 0 && fb >= 0, "stats");
        CHECK(enchip_ann_topk(ctx, idx, q.data(), M, 2000, hi.data(), hs.data()) == ENCHIP_ERR_ARG, "k too big");
        enchip_weight_release(ctx, idx);
    }
    // scratch cap: a call needing more than the cap declines, dst untouched, then lifts
    {
        const int64_t M = 4096, K = 768, N = 768;
        auto wq = randq(g, (size_t)(N * K));
        std::vector<float> ws(N, 0.003f);
        enchip_weight w = 0;
        enchip_weight_register(ctx, wq.data(), ws.data(), N, K, &w);
        auto a = randf(g, (size_t)(M * K));
        std::vector<float> dst((size_t)(M * N), 3.0f);
        CHECK(enchip_set_scratch_limit(ctx, 1 << 16) == ENCHIP_OK, "cap");
        CHECK(enchip_w8a8_linear(ctx, w, a.data(), M, nullptr, 0, dst.data(), nullptr) == ENCHIP_ERR_OOM, "oom");
        CHECK(dst[0] == 3.0f && dst.back() == 3.0f, "oom dst");
        CHECK(enchip_set_scratch_limit(ctx, 0) == ENCHIP_OK, "uncap");
        CHECK(enchip_w8a8_linear(ctx, w, a.data(), M, nullptr, 0, dst.data(), nullptr) == ENCHIP_OK, "after cap");
        enchip_weight_release(ctx, w);
    }
}

// 8 threads on one context: linears that succeed and calls that fail with messages of
// their own, read on the failing thread.
static void threads(enchip_ctx *ctx) {
    std::vector<std::thread> ts;
    std::vector<int> bad(8, 0);
    for (int t = 0; t < 8; ++t)
        ts.emplace_back([ctx, t, &bad] {
            std::mt19937 g(100 + t);
            const int64_t M = 17 + 40 * t, K = 256, N = 96 * (1 + t % 3);
            auto wq = randq(g, (size_t)(N * K));
            std::vector<float> ws(N, 0.004f);
            enchip_weight w = 0;
            if (enchip_weight_register(ctx, wq.data(), ws.data(), N, K, &w) != ENCHIP_OK) { bad[t]++; return; }
            auto a = randf(g, (size_t)(M * K));
            std::vector<float> dst((size_t)(M * N));
            for (int it = 0; it < 20; ++it) {
                if (enchip_w8a8_linear(ctx, w, a.data(), M, nullptr, it & 1, dst.data(), nullptr) != ENCHIP_OK) bad[t]++;
                if (enchip_matmul_bt_q8(ctx, w, a.data(), M, dst.data()) != ENCHIP_OK) bad[t]++;
                const int act = 50 + t;
                if (enchip_w8a8_linear(ctx, w, a.data(), M, nullptr, act, dst.data(), nullptr) != ENCHIP_ERR_ARG) bad[t]++;
                const std::string msg = enchip_last_error(ctx);
                if (msg.find("bad act " + std::to_string(act)) == std::string::npos) bad[t]++;
            }
            if (enchip_weight_release(ctx, w) != ENCHIP_OK) bad[t]++;
        });
    for (auto &th : ts) th.join();
    for (int t = 0; t < 8; ++t) CHECK(bad[t] == 0, "thread %d: %d failures", t, bad[t]);
}

int main() {
    CHECK(enchip_abi_version() == ENCHIP_ABI_VERSION, "abi");
    enchip_ctx *ctx = nullptr;
    CHECK(enchip_open(99, &ctx) != ENCHIP_OK && ctx == nullptr, "open of a missing device");
    CHECK(std::strlen(enchip_last_error(nullptr)) > 0, "open error");
    if (enchip_open(0, &ctx) != ENCHIP_OK) {
        std::fprintf(stderr, "enchip_open(0) failed: %s\n", enchip_last_error(nullptr));
        return 2;
    }
    int cus = 0, clk = 0;
    char name[4];
    CHECK(enchip_device_info(ctx, &cus, &clk, name, (int)sizeof name) == ENCHIP_OK && cus > 0, "device info");
    CHECK(std::strlen(name) < sizeof name, "device name truncated");
    std::mt19937 g(7);
    weights(ctx, g);
    std::printf("weights: %d failures so far\n", g_fail);
    std::fflush(stdout);
    compute(ctx, g);
    std::printf("compute: %d failures so far\n", g_fail);
    std::fflush(stdout);
    threads(ctx);
    std::printf("threads: %d failures so far\n", g_fail);
    std::fflush(stdout);
    CHECK(enchip_set_small_m(ctx, 8) == ENCHIP_OK && enchip_set_small_m(ctx, 32) == ENCHIP_OK, "small m");
    CHECK(enchip_set_attention_products(ctx, 77) == ENCHIP_ERR_ARG, "attention mode");
    CHECK(enchip_close(ctx) == ENCHIP_OK, "close");  // with weights still registered
    enchip_close(nullptr);
    std::printf("abi_stress: %s (%d failures)\n", g_fail ? "FAILED" : "ok", g_fail);
    std::fflush(nullptr);
    // Skip the exit-time destructors: the HSA runtime's own teardown trips this
    // AddressSanitizer runtime's device-allocator check (inside libhsa-runtime64, after
    // every enchip call has returned and the context is closed).
    std::_Exit(g_fail ? 1 : 0);
}
