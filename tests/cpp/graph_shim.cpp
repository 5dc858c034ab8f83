// Test-only C entry points over the autograd graph (include/cortex_hip_graph.hpp),
// so that the Python parity tests can drive the graph with seeded host
// inputs and compare what it produces with the CPU oracle.  Each function
// uploads its host inputs, builds the graph with the graph's own ops, runs
// forward and backward(root, seed) and downloads the results into the
// caller's host arrays.  Errors exit the process (the C++ layer's
// convention), which a test reports as a crash.
#include <cstring>
#include <vector>

#include "cortex_hip_graph.hpp"

namespace hip = cortex::_fw::hip;
using hip::TensorPtr;

namespace {

std::int64_t I(std::size_t v) { return static_cast<std::int64_t>(v); }

TensorPtr up(std::vector<std::int64_t> shape, const float *h, bool grad) {
    return std::make_shared<hip::Tensor>(hip::Tensor::from_host(std::move(shape), h, grad));
}

void down(const hip::Tensor &t, float *h) {
    const std::vector<float> v = t.host();
    std::memcpy(h, v.data(), v.size() * sizeof(float));
}

struct DevLabels {
    std::int32_t *p = nullptr;
    DevLabels(const std::int32_t *h, std::size_t n) {
        hip::check(cxm_dev_malloc(reinterpret_cast<void **>(&p), n * sizeof(std::int32_t)), "labels");
        hip::check(cxm_memcpy_h2d(p, h, n * sizeof(std::int32_t), hip::stream()), "labels");
        hip::check(cxm_stream_sync(hip::stream()), "labels");
    }
    ~DevLabels() { (void)cxm_dev_free(p); }
};

}  // namespace

extern "C" {

// `steps` SGD steps of the 3-layer ReLU MLP built from graph ops
// (matmul, add_bias, relu, softmax_cross_entropy, backward, sgd); the six
// parameters are updated in place, losses[s] is step s's loss.
int gs_mlp_steps(const float *x, const std::int32_t *labels, float *w1, float *b1, float *w2, float *b2, float *w3,
                 float *b3, std::size_t b, std::size_t d0, std::size_t d1, std::size_t d2, std::size_t d3, float lr,
                 int steps, float *losses) {
    DevLabels lab(labels, b);
    auto X = up({I(b), I(d0)}, x, false);
    auto W1 = up({I(d0), I(d1)}, w1, true), B1 = up({I(d1)}, b1, true);
    auto W2 = up({I(d1), I(d2)}, w2, true), B2 = up({I(d2)}, b2, true);
    auto W3 = up({I(d2), I(d3)}, w3, true), B3 = up({I(d3)}, b3, true);
    for (int s = 0; s < steps; ++s) {
        auto h1 = hip::relu(hip::add_bias(hip::matmul(X, W1), B1));
        auto h2 = hip::relu(hip::add_bias(hip::matmul(h1, W2), B2));
        auto logits = hip::add_bias(hip::matmul(h2, W3), B3);
        auto loss = hip::softmax_cross_entropy(logits, lab.p);
        hip::backward(loss);
        hip::sgd({W1, B1, W2, B2, W3, B3}, lr);
        down(*loss, losses + s);
    }
    down(*W1, w1), down(*B1, b1), down(*W2, w2), down(*B2, b2), down(*W3, w3), down(*B3, b3);
    return 0;
}

// y = act(x * scale + bias) over [m, n], as one fused op (fused = 1) or as
// the composition mul_row -> add_bias -> activation (fused = 0, act not
// NONE), then backward with seed dy: dx, dscale, dbias.
int gs_affine(const float *x, const float *scale, const float *bias, const float *dy, std::size_t m, std::size_t n,
              int act, int fused, float *y, float *dx, float *dscale, float *dbias) {
    auto X = up({I(m), I(n)}, x, true), S = up({I(n)}, scale, true), Bv = up({I(n)}, bias, true);
    TensorPtr Y;
    if (fused) {
        Y = hip::affine_act(X, S, Bv, act);
    } else {
        auto t = hip::add_bias(hip::mul_row(X, S), Bv);
        Y = act == CXM_ACT_NONE ? t : hip::activate(t, act);
    }
    const hip::Tensor seed = hip::Tensor::from_host({I(m), I(n)}, dy);
    hip::backward(Y, seed);
    down(*Y, y), down(X->grad(), dx), down(S->grad(), dscale), down(Bv->grad(), dbias);
    return 0;
}

// y = softmax / log_softmax(x) over rows, then backward with seed dy.
int gs_softmax(const float *x, const float *dy, std::size_t rows, std::size_t cols, int log_mode, float *y, float *dx) {
    auto X = up({I(rows), I(cols)}, x, true);
    auto Y = log_mode ? hip::log_softmax(X) : hip::softmax(X);
    const hip::Tensor seed = hip::Tensor::from_host({I(rows), I(cols)}, dy);
    hip::backward(Y, seed);
    down(*Y, y), down(X->grad(), dx);
    return 0;
}

// z = sum / mean of x [outer, dim, inner] over dim, then backward with seed dz.
int gs_reduce(const float *x, const float *dz, std::size_t outer, std::size_t dim, std::size_t inner, int mean,
              float *z, float *dx) {
    auto X = up({I(outer), I(dim), I(inner)}, x, true);
    auto Z = mean ? hip::mean(X, outer, dim, inner) : hip::sum(X, outer, dim, inner);
    const hip::Tensor seed = hip::Tensor::from_host({I(outer), I(inner)}, dz);
    hip::backward(Z, seed);
    down(*Z, z), down(X->grad(), dx);
    return 0;
}

// loss = softmax_cross_entropy(logits, labels), backward with the seed
// gradient `seed` (1.0 is the default seed of backward(loss)).
int gs_xent(const float *logits, const std::int32_t *labels, std::size_t b, std::size_t c, float seed, float *loss,
            float *dlogits) {
    DevLabels lab(labels, b);
    auto L = up({I(b), I(c)}, logits, true);
    auto loss_t = hip::softmax_cross_entropy(L, lab.p);
    const hip::Tensor s = hip::Tensor::from_host({1}, &seed);
    hip::backward(loss_t, s);
    down(*loss_t, loss), down(L->grad(), dlogits);
    return 0;
}

// y = add(mul_scalar(x, a), mul_scalar(x, c)): x's gradient gets two
// contributions, dy*a then dy*c added in (the accumulation path).
int gs_two_paths(const float *x, const float *dy, std::size_t n, float a, float c, float *y, float *dx) {
    auto X = up({I(n)}, x, true);
    auto Y = hip::add(hip::mul_scalar(X, a), hip::mul_scalar(X, c));
    const hip::Tensor seed = hip::Tensor::from_host({I(n)}, dy);
    hip::backward(Y, seed);
    down(*Y, y), down(X->grad(), dx);
    return 0;
}

}  // extern "C"
