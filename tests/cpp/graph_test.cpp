// GPU test of the C++ host layer's storage, pool and autograd:
//  1. Storage / Tensor: host -> HIP -> host round trips, clone, moves, and
//     pool reuse (same size class on the same stream comes back from cache);
//  2. the 3-layer MLP (784 -> 1024 -> 1024 -> 10, batch 256) trained 3 SGD
//     steps through the GradientFlow graph (matmul, add_bias, relu,
//     softmax_cross_entropy, backward, sgd) must agree with the fused
//     cxm_mlp3_step_f32: losses within 1e-5 relative, weights and biases
//     within 1e-4 of their layer's weight scale.  The two are not bit for
//     bit alike: the fused step's output layer forms the logits, dH2 and gW3
//     on the 16x16x4 MFMA in another summation order than the graph's GEMMs;
//     both are held to the CPU oracle in the Python GPU tests;
//  3. gradient accumulation: y = x W + x W gives dW = 2 x^T dY exactly.
// Prints ALL OK and returns 0 when every check passes.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <vector>

#include "cortex_hip_graph.hpp"

namespace hip = cortex::_fw::hip;

static int failures = 0;
#define EXPECT(cond, ...)                      \
    do {                                       \
        if (!(cond)) {                         \
            std::printf("FAIL %d: ", __LINE__); \
            std::printf(__VA_ARGS__);          \
            std::printf("\n");                 \
            ++failures;                        \
        }                                      \
    } while (0)

// deterministic host data: an LCG mapped to [-1, 1)
static std::vector<float> rnd(size_t n, unsigned seed, float scale) {
    std::vector<float> v(n);
    unsigned long long s = 0x9E3779B97F4A7C15ull ^ seed;
    for (size_t i = 0; i < n; ++i) {
        s = s * 6364136223846793005ull + 1442695040888963407ull;
        v[i] = scale * (static_cast<float>((s >> 40) & 0xFFFFFF) / 8388608.0f - 1.0f);
    }
    return v;
}

// max |a - b| <= tol * max |w| (w: the layer's weight)
static bool close_to(const std::vector<float> &a, const std::vector<float> &b, const std::vector<float> &w, float tol) {
    if (a.size() != b.size()) return false;
    float scale = 0.0f, err = 0.0f;
    for (float v : w) scale = std::fmax(scale, std::fabs(v));
    for (size_t i = 0; i < a.size(); ++i) err = std::fmax(err, std::fabs(a[i] - b[i]));
    return err <= tol * scale;
}

int main() {
    int ndev = 0;
    if (cxm_device_count(&ndev) != CXM_OK || ndev < 1) {
        std::printf("no device\n");
        return 2;
    }
    // ---------------------------------------------------------- 1. storage
    {
        const std::vector<float> h = rnd(1000, 1, 1.0f);
        hip::Tensor t({10, 100}, hip::DType::Float32, hip::DeviceType::HOST);
        std::memcpy(t.data(), h.data(), h.size() * sizeof(float));
        t.to(hip::DeviceType::HIP);
        EXPECT(t.device() == hip::DeviceType::HIP, "to(HIP)");
        hip::Storage c = t.storage()->clone();
        EXPECT(c.device() == hip::DeviceType::HIP && c.bytes() == 4000, "clone");
        hip::Storage moved(std::move(c));
        EXPECT(c.isEmpty() && moved.bytes() == 4000, "move leaves the source empty");
        hip::Storage back = moved.copy_to(hip::DeviceType::HOST);
        EXPECT(std::memcmp(back.raw(), h.data(), 4000) == 0, "host -> HIP -> clone -> host round trip");
        t.to(hip::DeviceType::HOST);
        EXPECT(std::memcmp(t.data(), h.data(), 4000) == 0, "Tensor::to(HOST)");

        cxm_pool_stats_t s0, s1;
        cxm_pool_stats(&s0);
        void *p = nullptr, *q = nullptr;
        cxm_pool_alloc(&p, 3000, hip::stream());
        cxm_pool_free(p);
        cxm_pool_alloc(&q, 4000, hip::stream());  // same 4 KiB class
        cxm_pool_stats(&s1);
        // p may itself come from the cache (t's device storage, same class, was freed by to(HOST))
        EXPECT(q == p && s1.hits >= s0.hits + 1 && s1.allocs == s0.allocs + 2, "pool reuses the block on the same stream");
        cxm_pool_free(q);
        EXPECT(cxm_pool_free(q) == CXM_E_INVALID, "double free rejected");
    }

    // ----------------------------------------------------- 2. MLP graph
    const size_t B = 256, d0 = 784, d1 = 1024, d2 = 1024, d3 = 10;
    const float lr = 0.01f;
    const std::vector<float> x = rnd(B * d0, 2, 0.5f);
    std::vector<int32_t> labels(B);
    for (size_t r = 0; r < B; ++r) labels[r] = static_cast<int32_t>((r * 7) % d3);
    const std::vector<float> w1 = rnd(d0 * d1, 3, 0.05f), w2 = rnd(d1 * d2, 4, 0.04f), w3 = rnd(d2 * d3, 5, 0.04f);
    const std::vector<float> b1 = rnd(d1, 6, 0.1f), b2 = rnd(d2, 7, 0.1f), b3 = rnd(d3, 8, 0.1f);

    int32_t *dlab = nullptr;
    hip::check(cxm_dev_malloc(reinterpret_cast<void **>(&dlab), B * sizeof(int32_t)), "labels");
    hip::check(cxm_memcpy_h2d(dlab, labels.data(), B * sizeof(int32_t), hip::stream()), "labels");

    // graph path
    auto X = std::make_shared<hip::Tensor>(hip::Tensor::from_host({(int64_t)B, (int64_t)d0}, x.data()));
    auto W1 = std::make_shared<hip::Tensor>(hip::Tensor::from_host({(int64_t)d0, (int64_t)d1}, w1.data(), true));
    auto W2 = std::make_shared<hip::Tensor>(hip::Tensor::from_host({(int64_t)d1, (int64_t)d2}, w2.data(), true));
    auto W3 = std::make_shared<hip::Tensor>(hip::Tensor::from_host({(int64_t)d2, (int64_t)d3}, w3.data(), true));
    auto B1 = std::make_shared<hip::Tensor>(hip::Tensor::from_host({(int64_t)d1}, b1.data(), true));
    auto B2 = std::make_shared<hip::Tensor>(hip::Tensor::from_host({(int64_t)d2}, b2.data(), true));
    auto B3 = std::make_shared<hip::Tensor>(hip::Tensor::from_host({(int64_t)d3}, b3.data(), true));
    const std::vector<hip::TensorPtr> params = {W1, B1, W2, B2, W3, B3};

    // fused path
    hip::Tensor fW1 = hip::Tensor::from_host({(int64_t)d0, (int64_t)d1}, w1.data());
    hip::Tensor fW2 = hip::Tensor::from_host({(int64_t)d1, (int64_t)d2}, w2.data());
    hip::Tensor fW3 = hip::Tensor::from_host({(int64_t)d2, (int64_t)d3}, w3.data());
    hip::Tensor fB1 = hip::Tensor::from_host({(int64_t)d1}, b1.data());
    hip::Tensor fB2 = hip::Tensor::from_host({(int64_t)d2}, b2.data());
    hip::Tensor fB3 = hip::Tensor::from_host({(int64_t)d3}, b3.data());
    hip::Tensor floss({1}, hip::DType::Float32, hip::DeviceType::HIP);
    cxm_mlp3 *net = nullptr;
    hip::check(cxm_mlp3_create(&net, B, d0, d1, d2, d3), "mlp3_create");

    for (int step = 0; step < 3; ++step) {
        auto h1 = hip::relu(hip::add_bias(hip::matmul(X, W1), B1));
        auto h2 = hip::relu(hip::add_bias(hip::matmul(h1, W2), B2));
        auto logits = hip::add_bias(hip::matmul(h2, W3), B3);
        auto loss = hip::softmax_cross_entropy(logits, dlab);
        EXPECT(loss->flow() && loss->flow()->ToString() == "SoftmaxCrossEntropy", "loss flow");
        hip::backward(loss);
        EXPECT(W1->has_grad() && B3->has_grad() && !X->has_grad(), "gradients reach the parameters only");
        hip::sgd(params, lr);

        hip::check(cxm_mlp3_step_f32(net, X->data(), dlab, fW1.data(), fB1.data(), fW2.data(), fB2.data(), fW3.data(),
                                     fB3.data(), lr, floss.data(), hip::stream()),
                   "mlp3_step");
        const float lg = loss->host()[0], lf = floss.host()[0];
        EXPECT(std::fabs(lg - lf) <= 1e-5f * std::fabs(lf), "step %d loss: graph %.9g fused %.9g", step, lg, lf);
        EXPECT(std::isfinite(lg), "finite loss");
    }
    {
        const auto w1h = fW1.host(), w2h = fW2.host(), w3h = fW3.host();
        EXPECT(close_to(W1->host(), w1h, w1h, 1e-4f), "W1 within 1e-4 of scale");
        EXPECT(close_to(W2->host(), w2h, w2h, 1e-4f), "W2 within 1e-4 of scale");
        EXPECT(close_to(W3->host(), w3h, w3h, 1e-4f), "W3 within 1e-4 of scale");
        EXPECT(close_to(B1->host(), fB1.host(), w1h, 1e-4f), "b1 within 1e-4 of W1's scale");
        EXPECT(close_to(B2->host(), fB2.host(), w2h, 1e-4f), "b2 within 1e-4 of W2's scale");
        EXPECT(close_to(B3->host(), fB3.host(), w3h, 1e-4f), "b3 within 1e-4 of W3's scale");
    }
    cxm_mlp3_destroy(net);

    // ------------------------------------------------- 3. accumulation
    {
        const size_t M = 64, K = 48, N = 32;
        const std::vector<float> xa = rnd(M * K, 9, 1.0f), wa = rnd(K * N, 10, 1.0f);
        auto Xa = std::make_shared<hip::Tensor>(hip::Tensor::from_host({(int64_t)M, (int64_t)K}, xa.data()));
        auto Wa = std::make_shared<hip::Tensor>(hip::Tensor::from_host({(int64_t)K, (int64_t)N}, wa.data(), true));
        auto y = hip::add(hip::matmul(Xa, Wa), hip::matmul(Xa, Wa));
        hip::backward(y);  // seed dY = 1
        const std::vector<float> g = Wa->grad().host();
        // single path: dW = X^T 1, computed by the same GEMM
        hip::Tensor ones({(int64_t)M, (int64_t)N}, hip::DType::Float32, hip::DeviceType::HIP);
        const std::vector<float> one(M * N, 1.0f);
        hip::check(cxm_memcpy_h2d(ones.data(), one.data(), one.size() * 4, hip::stream()), "ones");
        hip::Tensor single({(int64_t)K, (int64_t)N}, hip::DType::Float32, hip::DeviceType::HIP);
        hip::check(cxm_gemm_f32(Xa->data(), ones.data(), single.data(), K, M, N, 1, 0, nullptr, CXM_ACT_NONE, nullptr,
                                hip::stream()),
                   "single");
        const std::vector<float> s = single.host();
        bool ok = true;
        for (size_t i = 0; i < s.size(); ++i) ok = ok && g[i] == s[i] + s[i];
        EXPECT(ok, "two consumers: dW = 2 X^T dY exactly");
    }
    cxm_dev_free(dlab);
    hip::check(cxm_device_sync(), "sync");
    if (failures == 0) std::printf("ALL OK\n");
    return failures == 0 ? 0 : 1;
}
