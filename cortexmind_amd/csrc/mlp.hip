// Training step of the 3-layer ReLU MLP (784 -> 1024 -> 1024 -> 10 at the
// C5 workload), composed on the host from the library's own kernels.
//
// The reference has no layers, loss, optimizer or concrete autograd flows:
// only the abstract meta::GradientFlow::backward(const Tensor&)
// (source/CortexMind/framework/Graph/flow.hpp:15-24).  The step below is
// the forward pass, the reverse-mode backward of each op in reverse order
// (the job a chain of concrete GradientFlows would do), and SGD:
//   h1 = relu(x W1 + b1), h2 = relu(h1 W2 + b2), logits = h2 W3 + b3
//   loss, dlogits = softmax cross-entropy
//   dh2 = (dl W3^T) * [h2 > 0], gW3 = h2^T dl, gb3 = colsum(dl)
//   dh1 = (dh2 W2^T) * [h1 > 0], gW2 = h1^T dh2, gb2 = colsum(dh2)
//   gW1 = x^T dh1, gb1 = colsum(dh1)
//   W -= lr * gW, b -= lr * gb
// Bias add and ReLU ride in the forward GEMM epilogue, the ReLU backward
// mask in the dX GEMM epilogue, and each SGD update in the epilogue of the
// kernel that produces its gradient (weights: the dW GEMM; biases: the
// column sum), so no gradient is ever written out.  A layer's weights are
// updated only after its dX product has read them, which gives the same
// values as taking every gradient first.  Everything is enqueued on one
// stream without host synchronisation.
#include <new>

#include "cxm_common.hpp"

struct cxm_mlp3 {
    size_t b, d0, d1, d2, d3;
    float *h1, *h2, *lg, *dl, *dh2, *dh1;
    void *block;  // one allocation holding all of the above
};

extern "C" {

int cxm_mlp3_create(cxm_mlp3 **handle, size_t batch, size_t d0, size_t d1, size_t d2, size_t d3) {
    if (!handle || !batch || !d0 || !d1 || !d2 || !d3) return CXM_E_INVALID;
    *handle = nullptr;
    cxm_mlp3 *h = new (std::nothrow) cxm_mlp3{};
    if (!h) return CXM_E_INVALID;
    h->b = batch;
    h->d0 = d0;
    h->d1 = d1;
    h->d2 = d2;
    h->d3 = d3;
    // sizes in floats, each rounded to 64 floats (256 B) to keep 128-bit alignment
    auto r = [](size_t n) { return (n + 63) / 64 * 64; };
    const size_t sizes[6] = {r(batch * d1), r(batch * d2), r(batch * d3),
                             r(batch * d3), r(batch * d2), r(batch * d1)};
    size_t total = 0;
    for (size_t s : sizes) total += s;
    void *p = nullptr;
    int rc = cxm_dev_malloc(&p, total * sizeof(float));
    if (rc) {
        delete h;
        return rc;
    }
    h->block = p;
    float *f = static_cast<float *>(p);
    float **slots[6] = {&h->h1, &h->h2, &h->lg, &h->dl, &h->dh2, &h->dh1};
    for (int i = 0; i < 6; ++i) {
        *slots[i] = f;
        f += sizes[i];
    }
    *handle = h;
    return CXM_OK;
}

int cxm_mlp3_destroy(cxm_mlp3 *h) {
    if (!h) return CXM_E_INVALID;
    int rc = cxm_dev_free(h->block);
    delete h;
    return rc;
}

int cxm_mlp3_step_f32(cxm_mlp3 *h, const float *x, const int32_t *labels, float *w1, float *b1,
                      float *w2, float *b2, float *w3, float *b3, float lr, float *loss,
                      cxm_stream_t s) {
    if (!h || !x || !labels || !w1 || !b1 || !w2 || !b2 || !w3 || !b3 || !loss) return CXM_E_INVALID;
    const size_t B = h->b, d0 = h->d0, d1 = h->d1, d2 = h->d2, d3 = h->d3;
    int rc;
#define CXM_TRY(call)        \
    if ((rc = (call)) != 0) \
        return rc
    using cxm::Epilogue;
    const Epilogue sgd{nullptr, nullptr, CXM_ACT_NONE, 1, lr};
    // forward
    CXM_TRY(cxm::gemm_ex(x, w1, h->h1, B, d0, d1, 0, 0, Epilogue{b1, nullptr, CXM_ACT_RELU, 0, 0.0f}, s));
    CXM_TRY(cxm::gemm_ex(h->h1, w2, h->h2, B, d1, d2, 0, 0, Epilogue{b2, nullptr, CXM_ACT_RELU, 0, 0.0f}, s));
    CXM_TRY(cxm::gemm_ex(h->h2, w3, h->lg, B, d2, d3, 0, 0, Epilogue{b3, nullptr, CXM_ACT_NONE, 0, 0.0f}, s));
    CXM_TRY(cxm_softmax_xent_f32(h->lg, labels, loss, h->dl, B, d3, s));
    // layer 3: dX first (reads W3), then W3 -= lr * h2^T dl, b3 -= lr * colsum(dl)
    CXM_TRY(cxm::gemm_ex(h->dl, w3, h->dh2, B, d3, d2, 0, 1, Epilogue{nullptr, h->h2, CXM_ACT_NONE, 0, 0.0f}, s));
    CXM_TRY(cxm::gemm_ex(h->h2, h->dl, w3, d2, B, d3, 1, 0, sgd, s));
    CXM_TRY(cxm::colsum_sgd(h->dl, b3, B, d3, lr, s));
    // layer 2
    CXM_TRY(cxm::gemm_ex(h->dh2, w2, h->dh1, B, d2, d1, 0, 1, Epilogue{nullptr, h->h1, CXM_ACT_NONE, 0, 0.0f}, s));
    CXM_TRY(cxm::gemm_ex(h->h1, h->dh2, w2, d1, B, d2, 1, 0, sgd, s));
    CXM_TRY(cxm::colsum_sgd(h->dh2, b2, B, d2, lr, s));
    // layer 1
    CXM_TRY(cxm::gemm_ex(x, h->dh1, w1, d0, B, d1, 1, 0, sgd, s));
    CXM_TRY(cxm::colsum_sgd(h->dh1, b1, B, d1, lr, s));
#undef CXM_TRY
    return CXM_OK;
}

}  // extern "C"
