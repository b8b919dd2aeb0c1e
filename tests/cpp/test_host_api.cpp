// Tests of the C++ host API (include/irontensor.hpp), written like the reference's inline Rust
// tests: each KAT follows the test it names (file:line in the reference), with the expected values
// computed by the same inline CPU loops those tests use.
//   test_host_api --cpu   error types, BF16 rounding and argument checks; no device needed
//   test_host_api         everything, on device 0
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "irontensor.hpp"

using namespace irontensor;

static int g_failed = 0, g_passed = 0;

#define CHECK(cond)                                                              \
    do {                                                                         \
        if (!(cond)) {                                                           \
            std::printf("  FAILED %s:%d: %s\n", __FILE__, __LINE__, #cond);      \
            throw std::runtime_error("check failed");                            \
        }                                                                        \
    } while (0)

static void run(const char *name, const std::function<void()> &fn) {
    try {
        fn();
        ++g_passed;
        std::printf("ok   %s\n", name);
    } catch (const std::exception &e) {
        ++g_failed;
        std::printf("FAIL %s: %s\n", name, e.what());
    }
    std::fflush(stdout);
}

template <typename E, typename F>
static std::string expect_throw(F &&f) {
    try {
        f();
    } catch (const E &e) {
        return e.what();
    }
    throw std::runtime_error("expected exception not thrown");
}

static void cpu_tests() {
    run("error_display_formats", [] {  // src/error.rs:43-66
        CHECK(std::string(ShapeMismatch("op", "a", "b").what()) == "op: shape mismatch, expected a, got b");
        CHECK(std::string(UnsupportedDimensions("op", "2D", {1, 2}).what()) == "op: unsupported dimensions, expected 2D, got [1, 2]");
        CHECK(std::string(PrecisionMismatch("op", "FP32", "BF16").what()) == "op: precision mismatch, expected FP32, got BF16");
        CHECK(std::string(InnerDimensionMismatch("op", {1, 2}, {3, 4}).what()) == "op: inner dimensions don't match, A=[1, 2], B=[3, 4]");
        CHECK(std::string(EmptyTensor("op").what()) == "op: empty tensor not supported");
    });
    run("bf16_conversion_roundtrip", [] {  // src/precision.rs:51-65
        for (float v : {0.0f, 1.0f, -1.0f, 0.5f, -0.5f, 100.0f, -100.0f, 1e-5f, 1e5f}) {
            float back = bf16_to_f32(f32_to_bf16(v));
            float rel = std::fabs(v) > 1e-10f ? std::fabs((back - v) / v) : std::fabs(back - v);
            CHECK(rel < 0.01f);
        }
        CHECK(f32_to_bf16(1.0f + 1.0f / 256) == 0x3F80);       // tie -> even
        CHECK(f32_to_bf16(1.0f + 3.0f / 256) == 0x3F82);       // tie -> even (up)
        CHECK(std::isinf(bf16_to_f32(f32_to_bf16(INFINITY))));
        CHECK(std::isnan(bf16_to_f32(f32_to_bf16(NAN))));
    });
    run("gemm_check_rejects_bad_arguments", [] {
        int dummy;
        CHECK(it_gemm_check(IT_F16, IT_F32, IT_OP_N, IT_OP_N, 2, 2, 2, &dummy, 2, 0, &dummy, 2, 0, 0.f, &dummy, 2, 0, 1, nullptr) == IT_ERR_PRECISION);
        CHECK(it_gemm_check(IT_F32, IT_F32, IT_OP_N, IT_OP_N, 2, 2, 3, &dummy, 2, 0, &dummy, 2, 0, 0.f, &dummy, 2, 0, 1, nullptr) == IT_ERR_INVALID);
        CHECK(it_gemm_check(IT_F32, IT_F32, IT_OP_N, IT_OP_N, 2, 2, 2, &dummy, 2, 0, &dummy, 2, 0, 0.f, nullptr, 2, 0, 1, nullptr) == IT_ERR_NULL);
        CHECK(it_gemm_check(IT_F32, IT_F32, IT_OP_N, IT_OP_N, 2, 2, 2, &dummy, 2, 0, &dummy, 2, 0, 0.f, &dummy, 2, 0, 1, nullptr) == IT_OK);
        CHECK(std::string(it_last_error()).find("C is NULL") != std::string::npos);
    });
}

static std::vector<float> cpu_matmul(const std::vector<float> &a, const std::vector<float> &b, size_t m, size_t k, size_t n) {
    std::vector<float> c(m * n);
    for (size_t i = 0; i < m; ++i)
        for (size_t j = 0; j < n; ++j) {
            float acc = 0.0f;
            for (size_t p = 0; p < k; ++p) acc += a[i * k + p] * b[p * n + j];
            c[i * n + j] = acc;
        }
    return c;
}

static void gpu_tests() {
    run("matmul_2x2", [] {  // src/ops/gemm.rs:291-306
        Tensor a = Tensor::from_f32_slice({1, 2, 3, 4}, {2, 2}), b = Tensor::from_f32_slice({5, 6, 7, 8}, {2, 2});
        auto r = matmul(a, b).as_f32_slice();
        CHECK(r.size() == 4 && r[0] == 19 && r[1] == 22 && r[2] == 43 && r[3] == 50);
    });
    run("matmul_larger", [] {  // src/ops/gemm.rs:308-351
        const size_t m = 64, k = 32, n = 48;
        std::vector<float> a(m * k), b(k * n);
        for (size_t i = 0; i < m; ++i)
            for (size_t j = 0; j < k; ++j) a[i * k + j] = (float)(i + j) * 0.01f;
        for (size_t i = 0; i < k; ++i)
            for (size_t j = 0; j < n; ++j) b[i * n + j] = (float)(i * j) * 0.01f;
        auto r = matmul(Tensor::from_f32_slice(a, {m, k}), Tensor::from_f32_slice(b, {k, n})).as_f32_slice();
        auto e = cpu_matmul(a, b, m, k, n);
        for (size_t i = 0; i < m * n; ++i) CHECK(std::fabs(r[i] - e[i]) < 1e-3f);
    });
    run("matmul_batched", [] {  // src/ops/gemm.rs:353-386
        const size_t bt = 2, m = 3, k = 4, n = 2;
        std::vector<float> a(bt * m * k), b(bt * k * n);
        for (size_t i = 0; i < a.size(); ++i) a[i] = (float)i * 0.1f;
        for (size_t i = 0; i < b.size(); ++i) b[i] = (float)i * 0.1f;
        Tensor c = matmul(Tensor::from_f32_slice(a, {bt, m, k}), Tensor::from_f32_slice(b, {bt, k, n}));
        CHECK((c.shape() == std::vector<size_t>{bt, m, n}));
        auto r = c.as_f32_slice();
        for (size_t q = 0; q < bt; ++q) {
            std::vector<float> aa(a.begin() + q * m * k, a.begin() + (q + 1) * m * k);
            std::vector<float> bb(b.begin() + q * k * n, b.begin() + (q + 1) * k * n);
            auto e = cpu_matmul(aa, bb, m, k, n);
            for (size_t i = 0; i < m * n; ++i) CHECK(std::fabs(r[q * m * n + i] - e[i]) < 1e-3f);
        }
    });
    run("mps_matches_reference", [] {  // src/ops/mps_gemm.rs:637-668 (exact integers)
        const size_t m = 16, k = 8, n = 12;
        std::vector<float> a(m * k), b(k * n);
        for (size_t i = 0; i < a.size(); ++i) a[i] = (float)(i % 7) - 3.0f;
        for (size_t i = 0; i < b.size(); ++i) b[i] = (float)(i % 5) - 2.0f;
        auto r = matmul_mps(Tensor::from_f32_slice(a, {m, k}), Tensor::from_f32_slice(b, {k, n})).as_f32_slice();
        CHECK(r == cpu_matmul(a, b, m, k, n));
    });
    run("matmul_backward_2d", [] {  // src/ops/backward/gemm.rs:457-509
        const size_t m = 3, k = 4, n = 2;
        std::vector<float> a(m * k), b(k * n), gc(m * n, 1.0f);
        for (size_t i = 0; i < a.size(); ++i) a[i] = (float)i * 0.1f;
        for (size_t i = 0; i < b.size(); ++i) b[i] = (float)i * 0.1f;
        auto g = matmul_backward(Tensor::from_f32_slice(gc, {m, n}), Tensor::from_f32_slice(a, {m, k}),
                                 Tensor::from_f32_slice(b, {k, n}));
        auto ga = g.first.as_f32_slice(), gb = g.second.as_f32_slice();
        for (size_t i = 0; i < m; ++i)
            for (size_t j = 0; j < k; ++j) {
                float e = 0;
                for (size_t l = 0; l < n; ++l) e += gc[i * n + l] * b[j * n + l];
                CHECK(std::fabs(ga[i * k + j] - e) < 1e-4f);
            }
        for (size_t i = 0; i < k; ++i)
            for (size_t j = 0; j < n; ++j) {
                float e = 0;
                for (size_t l = 0; l < m; ++l) e += a[l * k + i] * gc[l * n + j];
                CHECK(std::fabs(gb[i * n + j] - e) < 1e-4f);
            }
    });
    run("matmul_backward_4d", [] {  // src/ops/backward/gemm.rs:548-586
        const size_t b1 = 2, b2 = 3, m = 4, k = 5, n = 6;
        std::vector<float> a(b1 * b2 * m * k), b(b1 * b2 * k * n), gc(b1 * b2 * m * n, 1.0f);
        for (size_t i = 0; i < a.size(); ++i) a[i] = std::fmod((float)i * 0.01f, 1.0f);
        for (size_t i = 0; i < b.size(); ++i) b[i] = std::fmod((float)i * 0.01f, 1.0f);
        auto g = matmul_backward(Tensor::from_f32_slice(gc, {b1, b2, m, n}), Tensor::from_f32_slice(a, {b1, b2, m, k}),
                                 Tensor::from_f32_slice(b, {b1, b2, k, n}));
        CHECK((g.first.shape() == std::vector<size_t>{b1, b2, m, k}));
        CHECK((g.second.shape() == std::vector<size_t>{b1, b2, k, n}));
        float e = 0;
        for (size_t l = 0; l < n; ++l) e += gc[l] * b[l];
        CHECK(std::fabs(g.first.as_f32_slice()[0] - e) < 1e-3f);
    });
    run("matmul_bf16", [] {  // src/ops/bf16_ops/mod.rs:34-49
        Tensor c = matmul_bf16(Tensor::from_f32_as_bf16({1, 2, 3, 4, 5, 6}, {2, 3}),
                               Tensor::from_f32_as_bf16({1, 2, 3, 4, 5, 6}, {3, 2}));
        CHECK(c.precision() == Precision::BF16);
        auto r = c.as_bf16_slice();
        CHECK(bf16_to_f32(r[0]) == 22 && bf16_to_f32(r[1]) == 28 && bf16_to_f32(r[2]) == 49 && bf16_to_f32(r[3]) == 64);
    });
    run("linear_with_bias", [] {  // src/nn/linear.rs:224-238
        Tensor w = Tensor::from_f32_slice({1, 0, 0, 1}, {2, 2}), bias = Tensor::from_f32_slice({1, 2}, {2});
        auto r = linear(Tensor::from_f32_slice({1, 2}, {1, 2}), w, &bias).as_f32_slice();
        CHECK(r[0] == 2 && r[1] == 4);
    });
    run("linear_forward_backward_shapes", [] {  // src/train/helpers.rs:48-76
        Tensor x = Tensor::from_f32_slice(std::vector<float>(8 * 4, 0.5f), {8, 4});
        Tensor w = Tensor::from_f32_slice(std::vector<float>(3 * 4, 0.25f), {3, 4});
        Tensor y = linear_forward(x, w);
        CHECK((y.shape() == std::vector<size_t>{8, 3}) && y.as_f32_slice()[0] == 0.5f);
        auto g = linear_backward(Tensor::from_f32_slice(std::vector<float>(8 * 3, 1.0f), {8, 3}), x, w);
        CHECK((g.first.shape() == std::vector<size_t>{8, 4}) && g.first.as_f32_slice()[0] == 0.75f);
        CHECK((g.second.shape() == std::vector<size_t>{3, 4}) && g.second.as_f32_slice()[0] == 4.0f);
    });
    run("attention_causal_rows", [] {  // src/ops/attention.rs:653-679 inputs, closed-form check
        const size_t b = 1, s = 4, h = 1, d = 4;
        std::vector<float> q(b * s * h * d, 0.0f), v(b * s * h * d);
        for (size_t i = 0; i < v.size(); ++i) v[i] = (float)(i + 1) * 0.1f;
        // Q = 0: uniform weights over the visible keys, so row r is the mean of V rows 0..r.
        auto o = attention(Tensor::from_f32_slice(q, {b, s, h, d}), Tensor::from_f32_slice(v, {b, s, h, d}),
                           Tensor::from_f32_slice(v, {b, s, h, d}), true).as_f32_slice();
        for (size_t r = 0; r < s; ++r)
            for (size_t c = 0; c < d; ++c) {
                float mean = 0;
                for (size_t j = 0; j <= r; ++j) mean += v[j * d + c];
                mean /= (float)(r + 1);
                CHECK(std::fabs(o[r * d + c] - mean) < 1e-5f);
            }
    });
    run("flash_attention_causal_rows", [] {  // same closed form at head_dim 64, ragged seq 70
        const size_t b = 1, s = 70, h = 2, d = 64;
        std::vector<float> q(b * s * h * d, 0.0f), v(b * s * h * d);
        for (size_t i = 0; i < v.size(); ++i) v[i] = (float)((i * 37) % 101) * 0.01f - 0.5f;
        auto o = flash_attention_bshd(Tensor::from_f32_slice(q, {b, s, h, d}), Tensor::from_f32_slice(v, {b, s, h, d}),
                                      Tensor::from_f32_slice(v, {b, s, h, d}), true).as_f32_slice();
        for (size_t r = 0; r < s; ++r)
            for (size_t hh = 0; hh < h; ++hh)
                for (size_t c = 0; c < d; ++c) {
                    double mean = 0;
                    for (size_t j = 0; j <= r; ++j) mean += v[(j * h + hh) * d + c];
                    mean /= (double)(r + 1);
                    CHECK(std::fabs(o[(r * h + hh) * d + c] - mean) < 1e-5);
                }
    });
    // flash_attention (src/ops/flash_attention.rs:76-98) on [batch, heads, seq, head_dim]: Q = 0 gives
    // causal prefix means of V at a fused (64) and a materialised (32) head size; its assertions.
    for (size_t d : {size_t(64), size_t(32)})
        run(("flash_attention_bhsd_d" + std::to_string(d)).c_str(), [d] {
            const size_t b = 1, h = 2, s = 70;
            std::vector<float> q(b * h * s * d, 0.0f), v(b * h * s * d);
            for (size_t i = 0; i < v.size(); ++i) v[i] = (float)((i * 37) % 101) * 0.01f - 0.5f;
            auto o = flash_attention(Tensor::from_f32_slice(q, {b, h, s, d}), Tensor::from_f32_slice(v, {b, h, s, d}),
                                     Tensor::from_f32_slice(v, {b, h, s, d}), true).as_f32_slice();
            for (size_t hh = 0; hh < h; ++hh)
                for (size_t r = 0; r < s; ++r)
                    for (size_t c = 0; c < d; ++c) {
                        double mean = 0;
                        for (size_t j = 0; j <= r; ++j) mean += v[(hh * s + j) * d + c];
                        mean /= (double)(r + 1);
                        CHECK(std::fabs(o[(hh * s + r) * d + c] - mean) < 1e-5);
                    }
            Tensor big = Tensor::zeros({1, 1, 4, 129}, Precision::FP32);
            expect_throw<Panic>([&] { flash_attention(big, big, big, false); });
            Tensor a = Tensor::zeros({1, 2, 4, d}, Precision::FP32), c = Tensor::zeros({1, 2, 5, d}, Precision::FP32);
            expect_throw<Panic>([&] { flash_attention(a, c, a, false); });
            auto z = flash_attention(Tensor::zeros({1, 2, 0, d}, Precision::FP32), Tensor::zeros({1, 2, 0, d}, Precision::FP32),
                                     Tensor::zeros({1, 2, 0, d}, Precision::FP32), true);
            CHECK(z.shape() == std::vector<size_t>({1, 2, 0, d}));
        });
    run("flash_attention_backward_zero_grad", [] {  // dO = 0 gives dQ = dK = dV = 0 exactly
        const size_t b = 1, h = 2, n = 100, d = 64;
        std::vector<float> x(b * h * n * d);
        for (size_t i = 0; i < x.size(); ++i) x[i] = (float)((i * 13) % 29) * 0.05f - 0.7f;
        Tensor t = Tensor::from_f32_slice(x, {b, h, n, d});
        auto g = flash_attention_backward(Tensor::zeros({b, h, n, d}, Precision::FP32), t, t, t);
        for (const Tensor *r : {&g.dq, &g.dk, &g.dv})
            for (float f : r->as_f32_slice()) CHECK(f == 0.0f);
    });
    run("transpose_3d_gpu", [] {  // src/ops/attention.rs:395-449, ragged tiles
        const size_t b = 3, m = 70, n = 130;
        std::vector<float> x(b * m * n);
        for (size_t i = 0; i < x.size(); ++i) x[i] = (float)i;
        auto t = transpose_3d_gpu(Tensor::from_f32_slice(x, {b, m, n}), b, m, n);
        CHECK((t.shape() == std::vector<size_t>{b, n, m}));
        auto y = t.as_f32_slice();
        for (size_t z = 0; z < b; ++z)
            for (size_t i = 0; i < m; ++i)
                for (size_t j = 0; j < n; ++j) CHECK(y[(z * n + j) * m + i] == x[(z * m + i) * n + j]);
        expect_throw<Panic>([&] { transpose_3d_gpu(Tensor::from_f32_slice(x, {b, m, n}), b, m, n + 1); });
    });
    run("causal_mask_3d_gpu", [] {  // src/ops/attention.rs:455-517
        const size_t b = 2, s = 37;
        std::vector<float> x(b * s * s);
        for (size_t i = 0; i < x.size(); ++i) x[i] = (float)(i % 101) - 50.f;
        auto y = causal_mask_3d_gpu(Tensor::from_f32_slice(x, {b, s, s}), b, s).as_f32_slice();
        for (size_t z = 0; z < b; ++z)
            for (size_t r = 0; r < s; ++r)
                for (size_t c = 0; c < s; ++c) {
                    const size_t i = (z * s + r) * s + c;
                    CHECK(c > r ? (std::isinf(y[i]) && y[i] < 0) : y[i] == x[i]);
                }
    });
    run("typed_errors", [] {  // src/ops/mps_gemm.rs:45-108
        Tensor f = Tensor::zeros({2, 3}, Precision::FP32), g = Tensor::zeros({4, 5}, Precision::FP32);
        CHECK(expect_throw<InnerDimensionMismatch>([&] { matmul(f, g); }).find("A=[2, 3], B=[4, 5]") != std::string::npos);
        Tensor h = Tensor::zeros({2, 2}, Precision::BF16);
        expect_throw<PrecisionMismatch>([&] { matmul(h, h); });
        Tensor t4 = Tensor::zeros({1, 1, 2, 2}, Precision::FP32);
        expect_throw<UnsupportedDimensions>([&] { matmul(t4, t4); });
        expect_throw<Panic>([&] { matmul_mps_nt(f, g); });
        expect_throw<Panic>([&] { Tensor::from_f32_slice({1, 2, 3}, {2, 2}); });
    });
    run("command_batch_async", [] {  // src/command_batch.rs:174-390
        CommandBatch::begin();
        CHECK(CommandBatch::is_active());
        Tensor a = Tensor::from_f32_slice(std::vector<float>(64 * 64, 1.0f), {64, 64});
        Tensor c = matmul(a, a);
        CommandBatch::commit_async();
        CommandBatch::wait_for_completion();
        CHECK(CommandBatch::is_async_complete());
        CommandBatch::end();
        CHECK(!CommandBatch::is_active());
        CHECK(c.as_f32_slice()[0] == 64.0f);
        CHECK(gpu_memory_allocated() > 0);
    });
    run("rmsnorm_closed_forms", [] {  // src/ops/norm.rs:31
        Tensor x = Tensor::from_f32_slice(std::vector<float>(3 * 8, 2.0f), {3, 8});
        Tensor g = Tensor::from_f32_slice({1, 2, 3, 4, 5, 6, 7, 8}, {8});
        std::vector<float> y = rmsnorm(x, g, 0.f).as_f32_slice();
        for (int r = 0; r < 3; ++r)
            for (int c = 0; c < 8; ++c) CHECK(std::fabs(y[r * 8 + c] - (c + 1)) < 1e-6f);
        auto [dx, dg] = rmsnorm_backward(Tensor::zeros({3, 8}, Precision::FP32), x, g, 1e-5f);
        for (float v : dx.as_f32_slice()) CHECK(v == 0.f);
        for (float v : dg.as_f32_slice()) CHECK(v == 0.f);
    });
    run("rope_inverse_and_position_zero", [] {  // src/ops/rope.rs:22, src/ops/backward/rope.rs:16
        std::vector<float> h(2 * 5 * 2 * 8);
        for (size_t i = 0; i < h.size(); ++i) h[i] = std::sin(0.37f * (float)i);
        Tensor x = Tensor::from_f32_slice(h, {2, 5, 2, 8});
        std::vector<float> y = rope(x, 10000.f, 0).as_f32_slice();
        std::vector<float> back = rope_backward(rope(x, 10000.f, 0), 10000.f, 0).as_f32_slice();
        for (size_t i = 0; i < h.size(); ++i) CHECK(std::fabs(back[i] - h[i]) < 1e-5f);
        for (int b = 0; b < 2; ++b)
            for (int i = 0; i < 16; ++i) CHECK(y[b * 80 + i] == h[b * 80 + i]);  // position 0 unrotated
    });
    run("embedding_gather_scatter", [] {  // src/ops/embedding.rs:21, src/ops/backward/embedding.rs:21
        Tensor w = Tensor::from_f32_slice({0, 1, 10, 11, 20, 21}, {3, 2});
        std::vector<float> e = embedding(w, {2, 0, 2}).as_f32_slice();
        CHECK((e == std::vector<float>{20, 21, 0, 1, 20, 21}));
        Tensor dy = Tensor::from_f32_slice({1, 2, 3, 4, 5, 6}, {3, 2});
        CHECK((embedding_backward(dy, {2, 0, 2}, 3).as_f32_slice() == std::vector<float>{3, 4, 0, 0, 6, 8}));
        expect_throw<Panic>([&] { embedding(w, {3}); });
    });
    run("cross_entropy_uniform_logits", [] {  // src/ops/backward/loss.rs:248
        CrossEntropy ce = cross_entropy_fused(Tensor::zeros({4, 10}, Precision::FP32), {0, 3, 9, 5});
        CHECK(std::fabs(ce.loss - std::log(10.f)) < 1e-6f);
        std::vector<float> g = ce.grad.as_f32_slice();
        CHECK(std::fabs(g[0] - (0.1f - 1.f) / 4.f) < 1e-7f && std::fabs(g[1] - 0.1f / 4.f) < 1e-7f);
    });
    run("cross_entropy_stats_uniform_logits", [] {  // the loss half of src/ops/backward/loss.rs:248
        CrossEntropyStats ce = cross_entropy_stats(Tensor::zeros({4, 10}, Precision::FP32), {0, 3, 9, 5});
        CHECK(std::fabs(ce.loss - std::log(10.f)) < 1e-6f);
        std::vector<float> st = ce.stats.as_f32_slice();  // {max, 1/sum} per row: {0, 1/10}
        for (int r = 0; r < 4; ++r) CHECK(st[2 * r] == 0.f && std::fabs(st[2 * r + 1] - 0.1f) < 1e-7f);
    });
    run("swiglu_backward_at_zero", [] {  // src/shaders/backward/elementwise.metal:101-126
        Tensor one = Tensor::from_f32_slice({1, 1}, {1, 2}), zero = Tensor::zeros({1, 2}, Precision::FP32);
        auto [gg, gu] = swiglu_backward(one, zero, one);
        for (float v : gg.as_f32_slice()) CHECK(v == 0.5f);  // sig(0) * (1 + 0) * up
        for (float v : gu.as_f32_slice()) CHECK(v == 0.f);   // silu(0)
    });
    run("fused_rmsnorm_linear_matches_separate", [] {  // src/ops/fused_rmsnorm_linear.rs:279-316
        std::vector<float> x(8 * 128), g(128), w(64 * 128);
        for (size_t i = 0; i < x.size(); ++i) x[i] = ((float)(i % 100) - 50.f) * 0.01f;
        for (size_t i = 0; i < g.size(); ++i) g[i] = 1.f + std::sin((float)i) * 0.1f;
        for (size_t i = 0; i < w.size(); ++i) w[i] = ((float)(i % 200) - 100.f) * 0.001f;
        Tensor tx = Tensor::from_f32_slice(x, {8, 128}), tg = Tensor::from_f32_slice(g, {128});
        Tensor tw = Tensor::from_f32_slice(w, {64, 128});
        std::vector<float> fused = fused_rmsnorm_linear(tx, tg, tw, 1e-5f).as_f32_slice();
        std::vector<float> sep = matmul_mps_nt(rmsnorm(tx, tg, 1e-5f), tw).as_f32_slice();
        for (size_t i = 0; i < fused.size(); ++i) CHECK(std::fabs(fused[i] - sep[i]) < 1e-4f);
    });
    run("fused_linear_cross_entropy_ignore_index", [] {  // src/ops/fused_linear_cross_entropy.rs:454-490
        std::vector<float> h(4 * 16), w(32 * 16);
        for (size_t i = 0; i < h.size(); ++i) h[i] = std::sin((float)i * 0.1f);
        for (size_t i = 0; i < w.size(); ++i) w[i] = std::cos((float)i * 0.05f);
        FusedLinearCE r = fused_linear_cross_entropy(Tensor::from_f32_slice(h, {4, 16}),
                                                     Tensor::from_f32_slice(w, {32, 16}), {5, -100, 10, -100});
        CHECK(r.loss > 0.f);
        std::vector<float> gh = r.grad_hidden.as_f32_slice();
        for (int d = 0; d < 16; ++d) CHECK(gh[16 + d] == 0.f && gh[48 + d] == 0.f);
    });
    run("l2_norm_and_lion", [] {  // src/ops/reduction.rs:94, src/shaders/lion.metal
        Tensor a = Tensor::from_f32_slice({3, 0}, {2}), b = Tensor::from_f32_slice({4}, {1});
        CHECK(total_l2_norm_gpu({&a, &b}) == 5.f);
        Tensor w = Tensor::from_f32_slice({1.f, -2.f}, {2}), g = Tensor::from_f32_slice({1.f, -1.f}, {2});
        ParamState st(w);
        Lion opt(LionConfig{0.5f, 0.9f, 0.99f, 0.f});
        opt.step(w, g, st);
        CHECK((w.as_f32_slice() == std::vector<float>{0.5f, -1.5f}));
        std::vector<float> m = st.momentum.as_f32_slice();
        CHECK(std::fabs(m[0] - 0.1f) < 1e-7f && std::fabs(m[1] + 0.1f) < 1e-7f);
    });
}

int main(int argc, char **argv) {
    const bool cpu_only = argc > 1 && std::strcmp(argv[1], "--cpu") == 0;
    cpu_tests();
    if (!cpu_only) {
        if (it_device_count() == 0) {
            std::printf("FAIL no HIP device visible\n");
            return 2;
        }
        gpu_tests();
    }
    std::printf("%d passed, %d failed\n", g_passed, g_failed);
    return g_failed ? 1 : 0;
}
