// cortex_hip_graph.hpp -- reverse-mode autograd over the gfx950 backend:
// the concrete GradientFlows the reference declares but never implements,
// a backward driver and SGD.
//
// The reference's autograd is the abstract meta::GradientFlow with
// `virtual void backward(const Tensor& _grad) = 0` and a name
// (source/CortexMind/framework/Graph/flow.hpp:15-24); GradientLink attaches a
// flow to a tensor (Graph/link.cpp:11-13).  No subclass, no driver and no
// optimizer exist there.  This header keeps that interface (GradientFlow,
// backward(const Tensor&), ToString()) and adds flows for every operator on
// the path -- MatMul, AddBias, Add, MulRow (Broadcast::row::mul), MulScalar
// (ScalarOp::mul), ReLU / Sigmoid / Tanh, the fused AffineAct, Softmax and
// LogSoftmax, Sum and Mean over an axis, SoftmaxCrossEntropy -- each
// running the library's kernels through the C ABI on hip::stream(), plus
// backward(root[, seed]) and sgd().  Tensors are shared handles (TensorPtr)
// so that a flow can reach its inputs' gradients.
//
// Gradients accumulate: the first contribution to a tensor's gradient is
// written directly, later ones are added (matrix_t::add in place).
// Flows that need a forward output keep its storage, not the tensor: the
// output owns the flow, and a handle back would make a reference cycle.
// Header-only; link with -lcxm_hip.
#ifndef CORTEX_HIP_GRAPH_HPP
#define CORTEX_HIP_GRAPH_HPP

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <initializer_list>
#include <memory>
#include <string>
#include <string_view>
#include <unordered_set>
#include <utility>
#include <vector>

#include "cortex_hip.hpp"

namespace cortex::_fw::hip {

using TensorPtr = std::shared_ptr<Tensor>;

// An fp32 tensor on the HIP device.
inline TensorPtr make_tensor(std::vector<std::int64_t> shape, bool requires_grad = false) {
    return std::make_shared<Tensor>(std::move(shape), DType::Float32, DeviceType::HIP, requires_grad);
}
inline Tensor device_tensor(std::vector<std::int64_t> shape) {
    return Tensor(std::move(shape), DType::Float32, DeviceType::HIP);
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
    Tensor tmp = device_tensor(t->shape());
    write(tmp.data());
    matrix_t::add(g->data(), tmp.data(), g->len());
}

// Where a kernel that forms several gradients at once writes t's
// contribution: t's gradient itself when it has none yet, else `tmp`, which
// grad_done then adds in; a scratch buffer when t takes no gradient.
inline float *grad_dst(const TensorPtr &t, Tensor &tmp) {
    if (needs_grad(t) && !t->has_grad()) {
        t->grad_ptr() = make_tensor(t->shape());
        return t->grad().data();
    }
    tmp = device_tensor(t->shape());
    return tmp.data();
}
inline void grad_done(const TensorPtr &t, Tensor &tmp) {
    if (needs_grad(t) && !tmp.empty()) matrix_t::add(t->grad().data(), tmp.data(), t->len());
}

// GradientLink (Graph/link.cpp:11-13): attach a flow to the tensor it produced.
inline void link(const TensorPtr &out, std::shared_ptr<GradientFlow> flow) { out->flow() = std::move(flow); }

// The graph's ops run device kernels on their operands' storage: a tensor
// that is not fp32 HIP memory is refused on the host (CXM_ASSERT's exit)
// before any launch could touch it.
inline void on_device(std::initializer_list<const Tensor *> ts, const char *what) {
    for (const Tensor *t : ts)
        if (t->device() != DeviceType::HIP || t->dtype() != DType::Float32) {
            std::fprintf(stderr, "[ERROR] %s: operand is not an fp32 HIP tensor\n", what);
            std::exit(1);
        }
}

// Rows and columns of a 2-D tensor.
inline std::size_t rows_of(const Tensor &t) { return static_cast<std::size_t>(t.dim(0)); }
inline std::size_t cols_of(const Tensor &t) { return static_cast<std::size_t>(t.dim(1)); }

// ------------------------------------------------------------------ flows

// C[M,N] = A[M,K] B[K,N]: dA = dC B^T, dB = A^T dC (cxm_gemm_f32 with the
// transposed operand forms).
struct MatMulFlow : GradientFlow {
    TensorPtr a, b;
    MatMulFlow(TensorPtr a_, TensorPtr b_) : GradientFlow("MatMul"), a(std::move(a_)), b(std::move(b_)) {
        inputs = {a, b};
    }
    void backward(const Tensor &dc) override {
        const std::size_t M = rows_of(*a), K = cols_of(*a), N = cols_of(*b);
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
        const std::size_t M = rows_of(*x), N = cols_of(*x);
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

// Y[M,N] = X * s[N] (Broadcast::row::mul): dX = dY * s, ds = sum over rows
// of dY * X.  One pass of the fused affine backward with no activation
// (cxm_affine_act_bwd_f32, ACT_NONE) forms both; its bias sum is dropped.
struct MulRowFlow : GradientFlow {
    TensorPtr x, scale;
    MulRowFlow(TensorPtr x_, TensorPtr s_) : GradientFlow("MulRow"), x(std::move(x_)), scale(std::move(s_)) {
        inputs = {x, scale};
    }
    void backward(const Tensor &dy) override {
        const std::size_t M = rows_of(*x), N = cols_of(*x);
        Tensor tx, ts, db = device_tensor({static_cast<std::int64_t>(N)});
        float *dx = grad_dst(x, tx), *ds = grad_dst(scale, ts);
        check(cxm_affine_act_bwd_f32(x->data(), scale->data(), x->data(), dy.data(), dx, ds, db.data(), M, N,
                                     CXM_ACT_NONE, stream()),
              "MulRowFlow");
        grad_done(x, tx);
        grad_done(scale, ts);
    }
};

// Y = X * c (ScalarOp::mul): dX = dY * c.
struct MulScalarFlow : GradientFlow {
    TensorPtr x;
    float c;
    MulScalarFlow(TensorPtr x_, float c_) : GradientFlow("MulScalar"), x(std::move(x_)), c(c_) { inputs = {x}; }
    void backward(const Tensor &dy) override {
        if (!needs_grad(x)) return;
        accumulate(x, [&](float *dx) { ScalarOp::mul(dy.data(), c, dx, dy.len()); });
    }
};

// Y = act(X) for act in RELU, SIGMOID, TANH: dX = dY * act'(Y) from the
// saved output (relu' = [Y > 0], sigmoid' = Y (1 - Y), tanh' = 1 - Y^2).
struct ActFlow : GradientFlow {
    TensorPtr x;
    std::shared_ptr<Storage> y;
    int act;
    static const char *name_of(int a) { return a == CXM_ACT_RELU ? "ReLU" : a == CXM_ACT_SIGMOID ? "Sigmoid" : "Tanh"; }
    ActFlow(TensorPtr x_, std::shared_ptr<Storage> y_, int a)
        : GradientFlow(name_of(a)), x(std::move(x_)), y(std::move(y_)), act(a) {
        inputs = {x};
    }
    void backward(const Tensor &dy) override {
        if (!needs_grad(x)) return;
        accumulate(x, [&](float *dx) {
            check(cxm_act_bwd_f32(y->as<float>(), dy.data(), dx, dy.len(), act, stream()), "ActFlow");
        });
    }
};

// Y = act(X * s[N] + b[N]) in one pass (cxm_affine_act_fwd_f32): the
// backward forms dX, ds and db in one pass too (cxm_affine_act_bwd_f32)
// from X, s, the saved Y and dY.
struct AffineActFlow : GradientFlow {
    TensorPtr x, scale, bias;
    std::shared_ptr<Storage> y;
    int act;
    AffineActFlow(TensorPtr x_, TensorPtr s_, TensorPtr b_, std::shared_ptr<Storage> y_, int a)
        : GradientFlow("AffineAct"), x(std::move(x_)), scale(std::move(s_)), bias(std::move(b_)), y(std::move(y_)),
          act(a) {
        inputs = {x, scale, bias};
    }
    void backward(const Tensor &dy) override {
        const std::size_t M = rows_of(*x), N = cols_of(*x);
        Tensor tx, ts, tb;
        float *dx = grad_dst(x, tx), *ds = grad_dst(scale, ts), *db = grad_dst(bias, tb);
        check(cxm_affine_act_bwd_f32(x->data(), scale->data(), y->as<float>(), dy.data(), dx, ds, db, M, N, act,
                                     stream()),
              "AffineActFlow");
        grad_done(x, tx);
        grad_done(scale, ts);
        grad_done(bias, tb);
    }
};

// Row softmax (log_mode 0) or log-softmax (1) over the last axis of
// [rows, cols]: dX from the saved output (cxm_softmax_bwd_f32).
struct SoftmaxFlow : GradientFlow {
    TensorPtr x;
    std::shared_ptr<Storage> y;
    int log_mode;
    SoftmaxFlow(TensorPtr x_, std::shared_ptr<Storage> y_, int log)
        : GradientFlow(log ? "LogSoftmax" : "Softmax"), x(std::move(x_)), y(std::move(y_)), log_mode(log) {
        inputs = {x};
    }
    void backward(const Tensor &dy) override {
        if (!needs_grad(x)) return;
        accumulate(x, [&](float *dx) {
            check(cxm_softmax_bwd_f32(y->as<float>(), dy.data(), dx, rows_of(*x), cols_of(*x), log_mode, stream()),
                  "SoftmaxFlow");
        });
    }
};

// Z[outer, inner] = reduce::sum / reduce::mean of X[outer, dim, inner] over
// dim: dX[o, d, i] = dZ[o, i] (/ dim for the mean).
struct SumFlow : GradientFlow {
    TensorPtr x;
    std::size_t outer, dim, inner;
    int mean;
    SumFlow(TensorPtr x_, std::size_t o, std::size_t d, std::size_t i, int m)
        : GradientFlow(m ? "Mean" : "Sum"), x(std::move(x_)), outer(o), dim(d), inner(i), mean(m) {
        inputs = {x};
    }
    void backward(const Tensor &dz) override {
        if (!needs_grad(x)) return;
        accumulate(x, [&](float *dx) {
            check(cxm_reduce_sum_bwd_f32(dz.data(), dx, outer, dim, inner, mean, stream()), "SumFlow");
        });
    }
};

// loss = mean over rows of -log_softmax(logits)[r, label_r]; the forward
// kernel also writes dloss/dlogits = (softmax - onehot) / rows, which the
// backward scales by the incoming gradient (a one-element device tensor,
// read on the device: dlogits * g[0], one rounding; exact for the seed 1).
struct SoftmaxCrossEntropyFlow : GradientFlow {
    TensorPtr logits;
    Tensor dlogits;
    SoftmaxCrossEntropyFlow(TensorPtr l, Tensor d)
        : GradientFlow("SoftmaxCrossEntropy"), logits(std::move(l)), dlogits(std::move(d)) {
        inputs = {logits};
    }
    void backward(const Tensor &g) override {
        if (!needs_grad(logits)) return;
        if (g.len() != 1) check(CXM_E_INVALID, "SoftmaxCrossEntropyFlow: the loss gradient is not a scalar");
        accumulate(logits, [&](float *dl) {
            // column broadcast over one row: dl[0, j] = dlogits[0, j] * g[0]
            check(cxm_bcast_col_f32(dlogits.data(), g.data(), dl, 1, dlogits.len(), CXM_OP_MUL, stream()),
                  "SoftmaxCrossEntropyFlow");
        });
    }
};

// ---------------------------------------------------------------- ops

inline TensorPtr matmul(const TensorPtr &a, const TensorPtr &b) {
    on_device({a.get(), b.get()}, "matmul");
    auto c = make_tensor({a->dim(0), b->dim(1)});
    matrix_t::matmul(a->data(), b->data(), c->data(), rows_of(*a), cols_of(*a), cols_of(*b));
    if (needs_grad(a) || needs_grad(b)) link(c, std::make_shared<MatMulFlow>(a, b));
    return c;
}

inline TensorPtr add_bias(const TensorPtr &x, const TensorPtr &b) {
    on_device({x.get(), b.get()}, "add_bias");
    auto y = make_tensor(x->shape());
    Broadcast::row::add(x->data(), b->data(), y->data(), rows_of(*x), cols_of(*x));
    if (needs_grad(x) || needs_grad(b)) link(y, std::make_shared<AddBiasFlow>(x, b));
    return y;
}

inline TensorPtr add(const TensorPtr &a, const TensorPtr &b) {
    on_device({a.get(), b.get()}, "add");
    auto y = make_tensor(a->shape());
    matrix_t::add(a->data(), b->data(), y->data(), a->len());
    if (needs_grad(a) || needs_grad(b)) link(y, std::make_shared<AddFlow>(a, b));
    return y;
}

// X[M,N] * s[N] (Broadcast::row::mul)
inline TensorPtr mul_row(const TensorPtr &x, const TensorPtr &s) {
    on_device({x.get(), s.get()}, "mul_row");
    auto y = make_tensor(x->shape());
    Broadcast::row::mul(x->data(), s->data(), y->data(), rows_of(*x), cols_of(*x));
    if (needs_grad(x) || needs_grad(s)) link(y, std::make_shared<MulRowFlow>(x, s));
    return y;
}

// X * c (ScalarOp::mul)
inline TensorPtr mul_scalar(const TensorPtr &x, float c) {
    on_device({x.get()}, "mul_scalar");
    auto y = make_tensor(x->shape());
    ScalarOp::mul(x->data(), c, y->data(), x->len());
    if (needs_grad(x)) link(y, std::make_shared<MulScalarFlow>(x, c));
    return y;
}

inline TensorPtr activate(const TensorPtr &x, int act) {
    on_device({x.get()}, "activation");
    auto y = make_tensor(x->shape());
    check(cxm_unary_f32(x->data(), y->data(), x->len(), act, stream()), "activation");
    if (needs_grad(x)) link(y, std::make_shared<ActFlow>(x, y->storage(), act));
    return y;
}
inline TensorPtr relu(const TensorPtr &x) { return activate(x, CXM_ACT_RELU); }
inline TensorPtr sigmoid(const TensorPtr &x) { return activate(x, CXM_ACT_SIGMOID); }
inline TensorPtr tanh(const TensorPtr &x) { return activate(x, CXM_ACT_TANH); }

// act(X * s + b) as one kernel each way; act in NONE, RELU, SIGMOID, TANH.
inline TensorPtr affine_act(const TensorPtr &x, const TensorPtr &s, const TensorPtr &b, int act) {
    on_device({x.get(), s.get(), b.get()}, "affine_act");
    auto y = make_tensor(x->shape());
    check(cxm_affine_act_fwd_f32(x->data(), s->data(), b->data(), y->data(), rows_of(*x), cols_of(*x), act, stream()),
          "affine_act");
    if (needs_grad(x) || needs_grad(s) || needs_grad(b))
        link(y, std::make_shared<AffineActFlow>(x, s, b, y->storage(), act));
    return y;
}

inline TensorPtr softmax_rows(const TensorPtr &x, int log_mode) {
    on_device({x.get()}, "softmax");
    auto y = make_tensor(x->shape());
    check(cxm_softmax_fwd_f32(x->data(), y->data(), rows_of(*x), cols_of(*x), log_mode, stream()), "softmax");
    if (needs_grad(x)) link(y, std::make_shared<SoftmaxFlow>(x, y->storage(), log_mode));
    return y;
}
inline TensorPtr softmax(const TensorPtr &x) { return softmax_rows(x, 0); }
inline TensorPtr log_softmax(const TensorPtr &x) { return softmax_rows(x, 1); }

// reduce::sum / reduce::mean over the middle axis of X viewed as
// [outer, dim, inner] (X's element count must be outer * dim * inner);
// the result has shape [outer, inner].
inline TensorPtr reduce_axis(const TensorPtr &x, std::size_t outer, std::size_t dim, std::size_t inner, int mean) {
    on_device({x.get()}, "reduce");
    if (outer * dim * inner != x->len()) check(CXM_E_INVALID, "reduce: outer * dim * inner != element count");
    auto z = make_tensor({static_cast<std::int64_t>(outer), static_cast<std::int64_t>(inner)});
    if (mean) reduce::mean(x->data(), z->data(), outer, dim, inner);
    else reduce::sum(x->data(), z->data(), outer, dim, inner);
    if (needs_grad(x)) link(z, std::make_shared<SumFlow>(x, outer, dim, inner, mean));
    return z;
}
inline TensorPtr sum(const TensorPtr &x, std::size_t outer, std::size_t dim, std::size_t inner) {
    return reduce_axis(x, outer, dim, inner, 0);
}
inline TensorPtr mean(const TensorPtr &x, std::size_t outer, std::size_t dim, std::size_t inner) {
    return reduce_axis(x, outer, dim, inner, 1);
}

// labels: device int32 [rows].
inline TensorPtr softmax_cross_entropy(const TensorPtr &logits, const std::int32_t *labels) {
    on_device({logits.get()}, "softmax_cross_entropy");
    auto loss = make_tensor({1});
    Tensor dl = device_tensor(logits->shape());
    check(cxm_softmax_xent_f32(logits->data(), labels, loss->data(), dl.data(), rows_of(*logits), cols_of(*logits),
                               stream()),
          "softmax_cross_entropy");
    if (needs_grad(logits)) link(loss, std::make_shared<SoftmaxCrossEntropyFlow>(logits, std::move(dl)));
    return loss;
}

// ------------------------------------------------------------ backward

// Runs every flow reachable from `root` once, each after all flows that
// consume its output: reverse topological order of the graph.  The root's
// gradient is `seed` (a device fp32 tensor of the root's element count),
// or ones when the root has no gradient yet and no seed is given.
inline void backward(const TensorPtr &root, const Tensor *seed = nullptr) {
    std::vector<TensorPtr> order;
    std::unordered_set<const Tensor *> seen;
    std::function<void(const TensorPtr &)> visit = [&](const TensorPtr &t) {
        if (!t->flow() || !seen.insert(t.get()).second) return;
        for (const auto &in : t->flow()->inputs) visit(in);
        order.push_back(t);
    };
    visit(root);
    if (seed) {
        if (seed->len() != root->len() || seed->device() != DeviceType::HIP)
            check(CXM_E_INVALID, "backward: seed does not match the root");
        root->grad_ptr() = make_tensor(root->shape());
        check(cxm_memcpy_d2d(root->grad().data(), seed->data(), seed->len() * sizeof(float), stream()), "backward: seed");
    } else if (!root->has_grad()) {  // d root / d root = 1
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
inline void backward(const TensorPtr &root, const Tensor &seed) { backward(root, &seed); }

// W -= lr * dW for every parameter with a gradient (matrix_t::sub of
// ScalarOp::mul: two roundings), then the gradients are dropped.
inline void sgd(const std::vector<TensorPtr> &params, float lr) {
    for (const auto &p : params) {
        if (!p->has_grad()) continue;
        on_device({p.get(), &p->grad()}, "sgd");
        check(cxm_sgd_f32(p->data(), p->grad().data(), lr, p->len(), stream()), "sgd");
        p->grad_ptr().reset();
    }
}

}  // namespace cortex::_fw::hip

#endif  // CORTEX_HIP_GRAPH_HPP
