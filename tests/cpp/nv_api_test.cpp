// Drives the backend through the reference's GPU operator API as mirrored
// in include/cortex_hip_nv.hpp (nv::ElementWise / Matrix / ScalarKernel over
// TensorView, Engine/CUDA/*.cuh), for Float32, BFloat16 and Float16 views.
// Inputs are small integers, so every result checked here is exact in all
// three types whatever the order of operations.  Prints "ALL OK" and
// returns 0 when every check passes; a failed check prints what differed
// and returns 1; a failed call exits(1) inside the host layer.
#include <cmath>
#include <cstdio>
#include <vector>

#include "cortex_hip_nv.hpp"

namespace hip = cortex::_fw::hip;
using hip::DType;
using hip::TensorView;

static int failures = 0;
#define EXPECT(cond, ...)                      \
    do {                                       \
        if (!(cond)) {                         \
            std::printf("FAIL: " __VA_ARGS__); \
            std::printf("\n");                 \
            ++failures;                        \
        }                                      \
    } while (0)

static int dt_code(DType t) { return t == DType::Float32 ? CXM_DT_F32 : t == DType::BFloat16 ? CXM_DT_BF16 : CXM_DT_F16; }
static size_t esize(DType t) { return t == DType::Float32 ? 4 : 2; }

// A device buffer of n elements of type t, filled from fp32 host values
// (converted on the device; the conversions are tested elsewhere).
struct Buf {
    void *p = nullptr;
    size_t n;
    DType t;
    Buf(size_t n_, DType t_) : n(n_), t(t_) { hip::check(cxm_dev_malloc(&p, n * esize(t) + 16), "malloc"); }
    Buf(const std::vector<float> &h, DType t_) : Buf(h.size(), t_) { set(h); }
    void set(const std::vector<float> &h) {
        void *tmp = nullptr;
        hip::check(cxm_dev_malloc(&tmp, n * 4), "malloc");
        hip::check(cxm_memcpy_h2d(tmp, h.data(), n * 4, nullptr), "h2d");
        hip::check(cxm_convert(p, dt_code(t), tmp, CXM_DT_F32, n, nullptr), "convert");
        hip::check(cxm_stream_sync(nullptr), "sync");
        cxm_dev_free(tmp);
    }
    std::vector<float> get() const {
        void *tmp = nullptr;
        hip::check(cxm_dev_malloc(&tmp, n * 4), "malloc");
        hip::check(cxm_convert(tmp, CXM_DT_F32, p, dt_code(t), n, nullptr), "convert");
        std::vector<float> h(n);
        hip::check(cxm_memcpy_d2h(h.data(), tmp, n * 4, nullptr), "d2h");
        cxm_dev_free(tmp);
        return h;
    }
    TensorView view() { return TensorView(static_cast<std::byte *>(p), t, hip::DeviceType::HIP, n); }
    ~Buf() { cxm_dev_free(p); }
};

static const char *name(DType t) { return t == DType::Float32 ? "f32" : t == DType::BFloat16 ? "bf16" : "f16"; }

static void run(DType t) {
    const size_t N = 1000;
    std::vector<float> x(N), y(N);
    for (size_t i = 0; i < N; ++i) {
        x[i] = static_cast<float>(static_cast<int>((i * 37) % 17) - 8);
        y[i] = static_cast<float>(static_cast<int>((i * 11) % 7) + 1);  // 1..7, no zero
    }
    Buf bx(x, t), by(y, t), bz(N, t);
    TensorView vx = bx.view(), vy = by.view(), vz = bz.view();

    hip::Matrix::add(vx, vy, vz);
    auto z = bz.get();
    for (size_t i = 0; i < N; ++i) EXPECT(z[i] == x[i] + y[i], "%s Matrix::add %zu", name(t), i);
    hip::Matrix::mul(vx, vy, vz);
    z = bz.get();
    for (size_t i = 0; i < N; ++i) EXPECT(z[i] == x[i] * y[i], "%s Matrix::mul %zu", name(t), i);
    hip::Matrix::max(vx, vy, vz);
    z = bz.get();
    for (size_t i = 0; i < N; ++i) EXPECT(z[i] == (x[i] > y[i] ? x[i] : y[i]), "%s Matrix::max %zu", name(t), i);

    hip::ScalarKernel::mul(vx, 2.0f, vz);
    z = bz.get();
    for (size_t i = 0; i < N; ++i) EXPECT(z[i] == 2.0f * x[i], "%s ScalarKernel::mul %zu", name(t), i);
    hip::ScalarKernel::add(vz, 3.0f);  // in place
    z = bz.get();
    for (size_t i = 0; i < N; ++i) EXPECT(z[i] == 2.0f * x[i] + 3.0f, "%s ScalarKernel::add %zu", name(t), i);

    hip::ElementWise::square(vx, vz);
    z = bz.get();
    for (size_t i = 0; i < N; ++i) EXPECT(z[i] == x[i] * x[i], "%s ElementWise::square %zu", name(t), i);
    hip::ElementWise::abs(vx, vz);
    z = bz.get();
    for (size_t i = 0; i < N; ++i) EXPECT(z[i] == std::fabs(x[i]), "%s ElementWise::abs %zu", name(t), i);
    hip::ElementWise::sqrt(vz, vz);  // of |x|^2 computed below: use squares
    hip::ElementWise::square(vx, vz);
    hip::ElementWise::sqrt(vz, vz);
    z = bz.get();
    for (size_t i = 0; i < N; ++i) EXPECT(z[i] == std::fabs(x[i]), "%s ElementWise::sqrt %zu", name(t), i);
    hip::ElementWise::pow(vy, 2.0f, vz);
    z = bz.get();
    for (size_t i = 0; i < N; ++i) EXPECT(z[i] == y[i] * y[i], "%s ElementWise::pow %zu", name(t), i);

    hip::Matrix::sub(vx, vy);  // in place: x - y
    auto xs = bx.get();
    for (size_t i = 0; i < N; ++i) EXPECT(xs[i] == x[i] - y[i], "%s Matrix::sub in place %zu", name(t), i);

    // matmul with M, K, N implied by the element counts
    const size_t M = 40, K = 24, Nn = 56;
    std::vector<float> a(M * K), b(K * Nn), ref(M * Nn, 0.0f);
    for (size_t i = 0; i < a.size(); ++i) a[i] = static_cast<float>(static_cast<int>((i * 7) % 5) - 2);
    for (size_t i = 0; i < b.size(); ++i) b[i] = static_cast<float>(static_cast<int>((i * 3) % 5) - 2);
    for (size_t i = 0; i < M; ++i)
        for (size_t j = 0; j < Nn; ++j)
            for (size_t k = 0; k < K; ++k) ref[i * Nn + j] += a[i * K + k] * b[k * Nn + j];
    Buf ba(a, t), bb(b, t), bc(M * Nn, t);
    TensorView va = ba.view(), vb = bb.view(), vc = bc.view();
    hip::Matrix::matmul(va, vb, vc);
    auto c = bc.get();
    for (size_t i = 0; i < c.size(); ++i) EXPECT(c[i] == ref[i], "%s Matrix::matmul %zu: %g vs %g", name(t), i, c[i], ref[i]);
    hip::Matrix::matmul(va, vb, vc, M, K, Nn);
    c = bc.get();
    for (size_t i = 0; i < c.size(); ++i) EXPECT(c[i] == ref[i], "%s Matrix::matmul(M,K,N) %zu", name(t), i);
}

int main() {
    // shape inference of Matrix::matmul (host only)
    size_t m = 0, k = 0, n = 0;
    EXPECT(hip::nv_detail::dims(40 * 24, 24 * 56, 40 * 56, &m, &k, &n) && m == 40 && k == 24 && n == 56, "dims 40x24x56");
    EXPECT(hip::nv_detail::dims(1, 1, 1, &m, &k, &n) && m == 1 && k == 1 && n == 1, "dims 1x1x1");
    EXPECT(hip::nv_detail::dims(4096ull * 8192, 8192ull * 1024, 4096ull * 1024, &m, &k, &n) && m == 4096 && k == 8192 &&
               n == 1024,
           "dims 4096x8192x1024");
    EXPECT(!hip::nv_detail::dims(6, 10, 7, &m, &k, &n), "dims inconsistent");
    EXPECT(!hip::nv_detail::dims(0, 10, 7, &m, &k, &n), "dims zero");

    int dc = 0;
    if (cxm_device_count(&dc) != CXM_OK || dc < 1) {
        std::printf("no device\n");
        return 2;
    }
    for (DType t : {DType::Float32, DType::BFloat16, DType::Float16}) run(t);
    if (failures) {
        std::printf("%d failures\n", failures);
        return 1;
    }
    std::printf("ALL OK\n");
    return 0;
}
