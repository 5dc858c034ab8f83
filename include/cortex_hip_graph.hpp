// cortex_hip_graph.hpp -- reverse-mode autograd over the gfx950 backend:
// the concrete GradientFlows the reference declares but never implements,
// a backward driver and SGD.
//
// The reference's autograd is the abstract meta::GradientFlow with
// `virtual void backward(const Tensor& _grad) = 0` and a name
// (source/CortexMind/framework/Graph/flow.hpp:15-24); GradientLink attaches a
// flow to a tensor (Graph/link.cpp:11-13).  No subclass, no driver and no
// optimizer exist there.  This header keeps that interface (GradientFlow,
// backward(const Tensor&), ToString()) and adds the flows of the MLP
// training path -- MatMul, AddBias, Add, ReLU, SoftmaxCrossEntropy -- each
// running the library's kernels through the C ABI on hip::stream(), plus
// backward(loss) and sgd().  Tensors are shared handles (TensorPtr) so that
// a flow can reach its inputs' gradients.
//
// Gradients accumulate: the first contribution to a tensor's gradient is
// written directly, later ones are added (matrix_t::add in place).
// Header-only; link with -lcxm_hip.
#ifndef CORTEX_HIP_GRAPH_HPP
#define CORTEX_HIP_GRAPH_HPP

#include <cstdint>
#include <functional>
#include <memory>
#include <string>
#include <string_view>
#include <unordered_set>
#include <utility>
#include <vector>

#include "cortex_hip.hpp"

namespace cortex::_fw::hip {

using TensorPtr = std::shared_ptr<Tensor>;

inline TensorPtr make_tensor(std::vector<std::int64_t> shape, bool requires_grad = false) {
    return std::make_shared<Tensor>(std::move(shape), DeviceType::HIP, requires_grad);
}

// meta::GradientFlow (Graph/flow.hpp:15-24).  `inputs` are the tensors the
// flow sends gradients to; the driver walks them to order the flows.
struct GradientFlow {
    explicit GradientFlow(std::string name) : name_(std::move(name)) {}
    virtual ~GradientFlow() = default;
    virtual void backward(const Tensor &grad) = 0;
    std::string_view ToString() const noexcept { return name_; }
    std::vector<TensorPtr> inputs;

private:
    std::string name_;
};

// A tensor takes part in the backward pass when it asks for a gradient or
// was produced by a flow.
inline bool needs_grad(const TensorPtr &t) { return t->isRequired() || t->flow() != nullptr; }

// Adds a gradient contribution to t: `write(dst)` fills a buffer of t's
// shape; the first contribution writes t's gradient directly.
inline void accumulate(const TensorPtr &t, const std::function<void(float *)> &write) {
    auto &g = t->grad_ptr();
    if (!g) {
        g = make_tensor(t->shape());
        write(g->data());
        return;
    }
    Tensor tmp(t->shape());
    write(tmp.data());
    matrix_t::add(g->data(), tmp.data(), g->len());
}

// GradientLink (Graph/link.cpp:11-13): attach a flow to the tensor it produced.
inline void link(const TensorPtr &out, std::shared_ptr<GradientFlow> flow) { out->flow() = std::move(flow); }

// ------------------------------------------------------------------ flows

// C[M,N] = A[M,K] B[K,N]: dA = dC B^T, dB = A^T dC (cxm_gemm_f32 with the
// transposed operand forms).
struct MatMulFlow : GradientFlow {
    TensorPtr a, b;
    MatMulFlow(TensorPtr a_, TensorPtr b_) : GradientFlow("MatMul"), a(std::move(a_)), b(std::move(b_)) {
        inputs = {a, b};
    }
    void backward(const Tensor &dc) override {
        const std::size_t M = a->dim(0), K = a->dim(1), N = b->dim(1);
        if (needs_grad(a))
            accumulate(a, [&](float *da) {
                check(cxm_gemm_f32(dc.data(), b->data(), da, M, N, K, 0, 1, nullptr, CXM_ACT_NONE, nullptr, stream()),
                      "MatMulFlow: dA");
            });
        if (needs_grad(b))
            accumulate(b, [&](float *db) {
                check(cxm_gemm_f32(a->data(), dc.data(), db, K, M, N, 1, 0, nullptr, CXM_ACT_NONE, nullptr, stream()),
                      "MatMulFlow: dB");
            });
    }
};

// Y[M,N] = X + b[N] (Broadcast::row::add): dX = dY, db = sum over rows of dY.
struct AddBiasFlow : GradientFlow {
    TensorPtr x, bias;
    AddBiasFlow(TensorPtr x_, TensorPtr b_) : GradientFlow("AddBias"), x(std::move(x_)), bias(std::move(b_)) {
        inputs = {x, bias};
    }
    void backward(const Tensor &dy) override {
        const std::size_t M = x->dim(0), N = x->dim(1);
        if (needs_grad(x))
            accumulate(x, [&](float *dx) {
                check(cxm_memcpy_d2d(dx, dy.data(), M * N * sizeof(float), stream()), "AddBiasFlow: dX");
            });
        if (needs_grad(bias))
            accumulate(bias, [&](float *db) { reduce::sum(dy.data(), db, 1, M, N); });
    }
};

// Y = A + B (same shape, matrix_t::add): dA = dY, dB = dY.
struct AddFlow : GradientFlow {
    TensorPtr a, b;
    AddFlow(TensorPtr a_, TensorPtr b_) : GradientFlow("Add"), a(std::move(a_)), b(std::move(b_)) { inputs = {a, b}; }
    void backward(const Tensor &dy) override {
        for (const TensorPtr &t : {a, b})
            if (needs_grad(t))
                accumulate(t, [&](float *d) {
                    check(cxm_memcpy_d2d(d, dy.data(), dy.len() * sizeof(float), stream()), "AddFlow");
                });
    }
};

// Y = relu(X): dX = dY * (Y > 0) from the saved output.  The flow keeps
// Y's storage, not Y itself: Y owns the flow, and a handle back would make
// a reference cycle.
struct ReLUFlow : GradientFlow {
    TensorPtr x;
    std::shared_ptr<Storage> y;
    ReLUFlow(TensorPtr x_, std::shared_ptr<Storage> y_) : GradientFlow("ReLU"), x(std::move(x_)), y(std::move(y_)) {
        inputs = {x};
    }
    void backward(const Tensor &dy) override {
        if (!needs_grad(x)) return;
        accumulate(x, [&](float *dx) {
            check(cxm_act_bwd_f32(y->as<float>(), dy.data(), dx, dy.len(), CXM_ACT_RELU, stream()), "ReLUFlow");
        });
    }
};

// loss = mean over rows of -log_softmax(logits)[r, label_r]; the forward
// kernel also writes dloss/dlogits = (softmax - onehot) / rows, which the
// backward passes on for the seed gradient 1 of a scalar loss.
struct SoftmaxCrossEntropyFlow : GradientFlow {
    TensorPtr logits;
    Tensor dlogits;
    SoftmaxCrossEntropyFlow(TensorPtr l, Tensor d)
        : GradientFlow("SoftmaxCrossEntropy"), logits(std::move(l)), dlogits(std::move(d)) {
        inputs = {logits};
    }
    void backward(const Tensor &) override {
        if (!needs_grad(logits)) return;
        accumulate(logits, [&](float *dl) {
            check(cxm_memcpy_d2d(dl, dlogits.data(), dlogits.len() * sizeof(float), stream()),
                  "SoftmaxCrossEntropyFlow");
        });
    }
};

// ---------------------------------------------------------------- ops

inline TensorPtr matmul(const TensorPtr &a, const TensorPtr &b) {
    auto c = make_tensor({a->dim(0), b->dim(1)});
    matrix_t::matmul(a->data(), b->data(), c->data(), a->dim(0), a->dim(1), b->dim(1));
    if (needs_grad(a) || needs_grad(b)) link(c, std::make_shared<MatMulFlow>(a, b));
    return c;
}

inline TensorPtr add_bias(const TensorPtr &x, const TensorPtr &b) {
    auto y = make_tensor(x->shape());
    Broadcast::row::add(x->data(), b->data(), y->data(), x->dim(0), x->dim(1));
    if (needs_grad(x) || needs_grad(b)) link(y, std::make_shared<AddBiasFlow>(x, b));
    return y;
}

inline TensorPtr add(const TensorPtr &a, const TensorPtr &b) {
    auto y = make_tensor(a->shape());
    matrix_t::add(a->data(), b->data(), y->data(), a->len());
    if (needs_grad(a) || needs_grad(b)) link(y, std::make_shared<AddFlow>(a, b));
    return y;
}

inline TensorPtr relu(const TensorPtr &x) {
    auto y = make_tensor(x->shape());
    activation::relu(x->data(), y->data(), x->len());
    if (needs_grad(x)) link(y, std::make_shared<ReLUFlow>(x, y->storage()));
    return y;
}

// labels: device int32 [rows].
inline TensorPtr softmax_cross_entropy(const TensorPtr &logits, const std::int32_t *labels) {
    auto loss = make_tensor({1});
    Tensor dl(logits->shape());
    check(cxm_softmax_xent_f32(logits->data(), labels, loss->data(), dl.data(), logits->dim(0), logits->dim(1),
                               stream()),
          "softmax_cross_entropy");
    if (needs_grad(logits)) link(loss, std::make_shared<SoftmaxCrossEntropyFlow>(logits, std::move(dl)));
    return loss;
}

// ------------------------------------------------------------ backward

// Runs every flow reachable from `root` once, each after all flows that
// consume its output: reverse topological order of the graph.
inline void backward(const TensorPtr &root) {
    std::vector<TensorPtr> order;
    std::unordered_set<const Tensor *> seen;
    std::function<void(const TensorPtr &)> visit = [&](const TensorPtr &t) {
        if (!t->flow() || !seen.insert(t.get()).second) return;
        for (const auto &in : t->flow()->inputs) visit(in);
        order.push_back(t);
    };
    visit(root);
    if (!root->has_grad()) {  // seed: d root / d root = 1
        root->grad_ptr() = make_tensor(root->shape());
        const std::vector<float> ones(root->len(), 1.0f);
        check(cxm_memcpy_h2d(root->grad().data(), ones.data(), ones.size() * sizeof(float), stream()), "backward: seed");
        check(cxm_stream_sync(stream()), "backward: seed");
    }
    for (auto it = order.rbegin(); it != order.rend(); ++it) {
        const TensorPtr &t = *it;
        if (t->has_grad()) t->flow()->backward(t->grad());
    }
}

// W -= lr * dW for every parameter with a gradient (matrix_t::sub of
// ScalarOp::mul: two roundings), then the gradients are dropped.
inline void sgd(const std::vector<TensorPtr> &params, float lr) {
    for (const auto &p : params) {
        if (!p->has_grad()) continue;
        check(cxm_sgd_f32(p->data(), p->grad().data(), lr, p->len(), stream()), "sgd");
        p->grad_ptr().reset();
    }
}

}  // namespace cortex::_fw::hip

#endif  // CORTEX_HIP_GRAPH_HPP
