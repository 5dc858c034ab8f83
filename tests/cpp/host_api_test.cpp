// Drives the backend through the C++ host layer (include/cortex_hip.hpp),
// the way a C++ caller of the reference engine would: device buffers from
// cxm_dev_malloc, operators named as in Engine/AVX2, results copied back
// and checked against values computed here.  Inputs are small integers, so
// every sum is exact whatever the summation order.  Prints "ALL OK" and
// returns 0 when every check passes; a failed check prints what differed
// and returns 1; a failed call exits(1) inside the host layer.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <vector>

#include "cortex_hip.hpp"

namespace hip = cortex::_fw::hip;

template <class T>
struct Dev {
    T *p = nullptr;
    size_t n;
    explicit Dev(size_t n_) : n(n_) { hip::check(cxm_dev_malloc(reinterpret_cast<void **>(&p), n * sizeof(T)), "malloc"); }
    Dev(const std::vector<T> &h) : Dev(h.size()) { hip::check(cxm_memcpy_h2d(p, h.data(), n * sizeof(T), nullptr), "h2d"); }
    std::vector<T> get() const {
        std::vector<T> h(n);
        hip::check(cxm_memcpy_d2h(h.data(), p, n * sizeof(T), nullptr), "d2h");
        return h;
    }
    ~Dev() { cxm_dev_free(p); }
};

static int failures = 0;
#define EXPECT(cond, ...)                     \
    do {                                      \
        if (!(cond)) {                        \
            std::printf("FAIL: " __VA_ARGS__); \
            std::printf("\n");                \
            ++failures;                       \
        }                                     \
    } while (0)

int main() {
    int n = 0;
    if (cxm_device_count(&n) != CXM_OK || n < 1) {
        std::printf("no device\n");
        return 2;
    }
    const size_t R = 300, C = 1028;
    std::vector<float> x(R * C);
    for (size_t i = 0; i < x.size(); ++i) x[i] = static_cast<float>(static_cast<int>((i * 2654435761u) % 201) - 100);
    x[5 * C + 77] = 1000.0f;  // row 5 maximum at column 77
    x[9 * C + 3] = 1000.0f;   // column 3 maximum at row 9
    Dev<float> dx(x);

    // reduce::sum / max / argmax, row and column forms
    Dev<float> zr(R), zc(C);
    Dev<int32_t> ar(R), ac(C);
    hip::reduce::sum(dx.p, zr.p, R, C, 1);
    hip::reduce::sum(dx.p, zc.p, 1, R, C);
    hip::reduce::argmax(dx.p, ar.p, R, C, 1);
    hip::reduce::argmax(dx.p, ac.p, 1, R, C);
    auto hr = zr.get(), hc = zc.get();
    auto har = ar.get(), hac = ac.get();
    for (size_t r = 0; r < R; ++r) {
        double s = 0;
        for (size_t c = 0; c < C; ++c) s += x[r * C + c];
        EXPECT(hr[r] == static_cast<float>(s), "row sum %zu: %f vs %f", r, hr[r], s);
    }
    for (size_t c = 0; c < C; ++c) {
        double s = 0;
        for (size_t r = 0; r < R; ++r) s += x[r * C + c];
        EXPECT(hc[c] == static_cast<float>(s), "col sum %zu", c);
    }
    EXPECT(har[5] == 77, "row argmax 5 = %d", har[5]);
    EXPECT(hac[3] == 9, "col argmax 3 = %d", hac[3]);
    Dev<float> g(1);
    hip::reduce::max(dx.p, g.p, R * C);
    EXPECT(g.get()[0] == 1000.0f, "global max");
    hip::reduce::min(dx.p, g.p, R * C);
    EXPECT(g.get()[0] == -100.0f, "global min");
    hip::reduce::norm1(dx.p, zr.p, R, C, 1);
    auto hn = zr.get();
    for (size_t r = 0; r < R; ++r) {
        double s = 0;
        for (size_t c = 0; c < C; ++c) s += std::fabs(x[r * C + c]);
        EXPECT(hn[r] == static_cast<float>(s), "row norm1 %zu", r);
    }

    // Broadcast::row::add in place, then matrix_t::mul and activation::relu
    std::vector<float> b(C);
    for (size_t c = 0; c < C; ++c) b[c] = static_cast<float>(c % 7) - 3.0f;
    Dev<float> db(b), dy(R * C);
    hip::Broadcast::row::add(dx.p, db.p, R, C);
    hip::activation::relu(dx.p, dy.p, R * C);
    auto hy = dy.get();
    for (size_t i = 0; i < hy.size(); ++i) {
        const float t = x[i] + b[i % C];
        EXPECT(hy[i] == (0.0f > t ? 0.0f : t), "relu(x+b) at %zu", i);
        if (failures > 10) break;
    }

    // matrix_t::matmul on small integers (exact in fp32)
    const size_t M = 70, K = 33, N = 45;
    std::vector<float> A(M * K), B(K * N);
    for (size_t i = 0; i < A.size(); ++i) A[i] = static_cast<float>(static_cast<int>(i % 9) - 4);
    for (size_t i = 0; i < B.size(); ++i) B[i] = static_cast<float>(static_cast<int>(i % 5) - 2);
    Dev<float> dA(A), dB(B), dC(M * N);
    hip::matrix_t::matmul(dA.p, dB.p, dC.p, M, K, N);
    auto hC = dC.get();
    for (size_t i = 0; i < M; ++i)
        for (size_t j = 0; j < N; ++j) {
            float s = 0;
            for (size_t k = 0; k < K; ++k) s += A[i * K + k] * B[k * N + j];
            EXPECT(hC[i * N + j] == s, "matmul %zu,%zu", i, j);
        }

    // wise::square / abs / sign and the pow and gather forms on small integers (exact)
    std::vector<float> w(1000);
    for (size_t i = 0; i < w.size(); ++i) w[i] = static_cast<float>(static_cast<int>(i % 23) - 11);
    Dev<float> dw(w), dq(w.size()), dp(w.size()), ds(w.size());
    hip::wise::square(dw.p, dq.p, w.size());
    hip::wise::pow(dw.p, 3.0f, dp.p, w.size());
    hip::wise::sign(dw.p, ds.p, w.size());
    std::vector<int32_t> gi(500);
    for (size_t i = 0; i < gi.size(); ++i) gi[i] = static_cast<int32_t>((i * 37) % w.size());
    Dev<int32_t> dgi(gi);
    Dev<float> dg(gi.size());
    hip::wise::gather(dw.p, w.size(), dgi.p, dg.p, gi.size());
    auto hq = dq.get(), hp = dp.get(), hs = ds.get(), hg = dg.get();
    for (size_t i = 0; i < w.size(); ++i) {
        EXPECT(hq[i] == w[i] * w[i], "square %zu", i);
        const float cube = w[i] * w[i] * w[i];  // exact for these integers
        EXPECT(std::fabs(hp[i] - cube) <= 2.4e-7f * std::fabs(cube), "pow %zu: %f", i, hp[i]);
        EXPECT(hs[i] == static_cast<float>((w[i] > 0) - (w[i] < 0)), "sign %zu", i);
        if (failures > 10) break;
    }
    for (size_t i = 0; i < gi.size(); ++i) EXPECT(hg[i] == w[gi[i]], "gather %zu", i);

    // ScalarOp and wise over TensorViews (Engine/AVX2/scalar.hpp:36-104,
    // wise.hpp:27-41), out of place and in place, on Tensors of each
    // supported DType placed on the device (Tensor(shape, DType, DeviceType))
    for (hip::DType t : {hip::DType::Float32, hip::DType::BFloat16, hip::DType::Float16}) {
        const size_t L = 777;
        std::vector<float> v(L);
        for (size_t i = 0; i < L; ++i) v[i] = static_cast<float>(static_cast<int>(i % 31) - 15);
        hip::Tensor a({static_cast<int64_t>(L)}, hip::DType::Float32, hip::DeviceType::HOST);
        std::memcpy(a.data(), v.data(), L * sizeof(float));
        a.to(hip::DeviceType::HIP);
        hip::Tensor ta({static_cast<int64_t>(L)}, t, hip::DeviceType::HIP), tz({static_cast<int64_t>(L)}, t, hip::DeviceType::HIP);
        EXPECT(ta.dtype() == t && ta.device() == hip::DeviceType::HIP && ta.storage()->bytes() == L * hip::size_of(t),
               "Tensor(shape, DType, HIP) storage");
        hip::check(cxm_convert(ta.raw(), t == hip::DType::Float32 ? CXM_DT_F32 : t == hip::DType::BFloat16 ? CXM_DT_BF16 : CXM_DT_F16,
                               a.raw(), CXM_DT_F32, L, hip::stream()),
                   "convert");
        {
            auto va = ta.view();
            auto vz = tz.view();
            hip::ScalarOp::mul(va, 3.0f, vz);  // out of place
            hip::ScalarOp::add(vz, 1.0f);      // in place
            hip::ScalarOp::sub(vz, 2.0f);
            hip::ScalarOp::div(vz, 2.0f);
        }
        hip::Tensor back({static_cast<int64_t>(L)}, hip::DType::Float32, hip::DeviceType::HIP);
        auto convert_back = [&](hip::Tensor &src) {
            hip::check(cxm_convert(back.raw(), CXM_DT_F32, src.raw(),
                                   t == hip::DType::Float32 ? CXM_DT_F32 : t == hip::DType::BFloat16 ? CXM_DT_BF16 : CXM_DT_F16,
                                   L, hip::stream()),
                       "convert back");
            return back.host();
        };
        auto h = convert_back(tz);
        for (size_t i = 0; i < L; ++i) {
            const float want = (v[i] * 3.0f + 1.0f - 2.0f) / 2.0f;  // exact in all three types
            EXPECT(h[i] == want, "ScalarOp over TensorView dtype %d at %zu: %f vs %f", static_cast<int>(t), i, h[i], want);
            if (failures > 10) break;
        }
        {
            auto va = ta.view();
            auto vz = tz.view();
            hip::wise::abs(va, vz);
            hip::wise::square(vz, vz);
            hip::wise::neg(vz, vz);
        }
        h = convert_back(tz);
        for (size_t i = 0; i < L; ++i) {
            EXPECT(h[i] == -(v[i] * v[i]), "wise over TensorView dtype %d at %zu", static_cast<int>(t), i);
            if (failures > 10) break;
        }
        {
            auto va = ta.view();
            auto vz = tz.view();
            hip::wise::pow(va, 2.0f, vz);
            hip::wise::sign(va, va);
        }
        h = convert_back(tz);
        const auto hsg = convert_back(ta);
        for (size_t i = 0; i < L; ++i) {
            EXPECT(std::fabs(h[i] - v[i] * v[i]) <= 1e-2f * v[i] * v[i], "wise::pow dtype %d at %zu", static_cast<int>(t), i);
            EXPECT(hsg[i] == static_cast<float>((v[i] > 0) - (v[i] < 0)), "wise::sign in place dtype %d", static_cast<int>(t));
            if (failures > 10) break;
        }
    }

    if (failures == 0) std::printf("ALL OK\n");
    return failures == 0 ? 0 : 1;
}
