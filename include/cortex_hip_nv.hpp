// cortex_hip_nv.hpp -- the reference's GPU operator API (nv::ElementWise,
// nv::Matrix, nv::ScalarKernel over TensorView) on the gfx950 backend.
//
// Mirrors source/CortexMind/framework/Engine/CUDA/element_wise.cuh:11-27,
// matrix.cuh:11-26 and scalar.cuh:25-99: static operators taking
// non-owning, non-copyable views (Tools/view.hpp:25-83) of device data,
// dispatched on the view's dtype (view.hpp:107-117: Float32, Float16,
// BFloat16; anything else is an error).  DeviceType::HIP takes the place of
// DeviceType::CUDA (Memory/type.hpp:22-26): every view passed here must be
// HIP device memory.  Each call is queued on hip::stream().  Errors print a
// message and exit(1), as the reference's CXM_ASSERT does
// (Tools/Error/errors.cpp:14-23).
//
// Differences from the reference, all on purpose:
//  * Matrix::matmul(Xx, Xy, Xz) derives M, K, N from the three element
//    counts (M*K, K*N, M*N determine them) instead of taking the counts
//    themselves as the dimensions (matrix.cu:114-116); an explicit
//    (M, K, N) overload is added.
//  * fp32 matmul is true fp32 (the reference asks cuBLAS for TF32), and
//    fp16 matmul accumulates in fp32 (the reference in fp16).
//  * operands must agree in dtype and element count (the reference does not
//    check).
#ifndef CORTEX_HIP_NV_HPP
#define CORTEX_HIP_NV_HPP

#include <cstddef>
#include <cstdint>

#include "cortex_hip.hpp"

namespace cortex::_fw::hip {

// Type/dtype.hpp:21-33 (same values).
enum class DType : std::uint8_t {
    Unknown = 0,
    Int32 = 1,
    Int64 = 2,
    Float32 = 3,
    Float64 = 4,
    BFloat16 = 5,
    Float16 = 6,
    QInt16 = 7,
    QInt8 = 8,
    QUInt16 = 9,
    QUInt8 = 10,
};

// Tools/view.hpp:25-83: non-owning view of `size` elements of `type`.
class TensorView {
public:
    TensorView(std::byte *data, DType type, DeviceType device, std::size_t size)
        : m_data(data), m_type(type), m_device(device), m_size(size) {}
    TensorView(TensorView const &) = delete;
    TensorView(TensorView &&) = delete;
    TensorView &operator=(TensorView const &) = delete;
    TensorView &operator=(TensorView &&) = delete;
    ~TensorView() = default;

    [[nodiscard]] std::byte *data() noexcept { return m_data; }
    [[nodiscard]] const std::byte *data() const noexcept { return m_data; }
    [[nodiscard]] DType dtype() const noexcept { return m_type; }
    [[nodiscard]] DeviceType device() const noexcept { return m_device; }
    [[nodiscard]] std::size_t size() const noexcept { return m_size; }

private:
    std::byte *m_data;
    DType m_type;
    DeviceType m_device;
    std::size_t m_size;
};

namespace nv_detail {

[[noreturn]] inline void fail(const char *what, const char *why) {
    std::fprintf(stderr, "[ERROR] %s: %s\n", what, why);
    std::exit(1);
}

// view.hpp:107-117's dispatch, as the ABI's dtype code.
inline int code(const TensorView &v, const char *what) {
    if (v.device() != DeviceType::HIP) fail(what, "view is not HIP device memory");
    switch (v.dtype()) {
        case DType::Float32: return CXM_DT_F32;
        case DType::BFloat16: return CXM_DT_BF16;
        case DType::Float16: return CXM_DT_F16;
        default: fail(what, "unsupported DType");
    }
}

inline int same(const TensorView &a, const TensorView &b, const char *what) {
    const int c = code(a, what);
    if (code(b, what) != c) fail(what, "operands differ in dtype");
    if (a.size() != b.size()) fail(what, "operands differ in element count");
    return c;
}

inline int same(const TensorView &a, const TensorView &b, const TensorView &c, const char *what) {
    same(a, b, what);
    return same(a, c, what);
}

inline void unary(const TensorView &Xx, TensorView &Xz, int fn, const char *what) {
    const int dt = same(Xx, Xz, what);
    check(cxm_wise_t(Xx.data(), Xz.data(), Xx.size(), fn, dt, stream()), what);
}

inline void binary(const TensorView &Xx, const TensorView &Xy, TensorView &Xz, int op, const char *what) {
    const int dt = same(Xx, Xy, Xz, what);
    check(cxm_binary_t(Xx.data(), Xy.data(), Xz.data(), Xx.size(), op, dt, stream()), what);
}

inline void scalar(const TensorView &Xx, float value, TensorView &Xz, int op, const char *what) {
    const int dt = same(Xx, Xz, what);
    check(cxm_scalar_t(Xx.data(), value, Xz.data(), Xx.size(), op, dt, stream()), what);
}

// M, K, N from |A| = M*K, |B| = K*N, |C| = M*N: M*M = |A|*|C| / |B|.
inline bool dims(std::size_t sa, std::size_t sb, std::size_t sc, std::size_t *m, std::size_t *k, std::size_t *n) {
    if (sa == 0 || sb == 0 || sc == 0) return false;
    const unsigned __int128 p = static_cast<unsigned __int128>(sa) * sc;
    if (p % sb != 0) return false;
    const unsigned __int128 q = p / sb;
    // integer square root of q (q < 2^128): Newton from above
    unsigned __int128 x = q, y = (x + 1) / 2;
    while (y < x) {
        x = y;
        y = (x + q / x) / 2;
    }
    if (x * x != q || x == 0) return false;
    const std::size_t M = static_cast<std::size_t>(x);
    if (sa % M != 0 || sc % M != 0) return false;
    const std::size_t K = sa / M, N = sc / M;
    if (static_cast<unsigned __int128>(K) * N != sb) return false;
    *m = M;
    *k = K;
    *n = N;
    return true;
}

}  // namespace nv_detail

// nv::ElementWise (element_wise.cuh:11-27, element_wise.cu:17-181).
struct ElementWise {
    static void square(const TensorView &Xx, TensorView &Xz) { nv_detail::unary(Xx, Xz, CXM_FN_SQUARE, "ElementWise::square"); }
    static void pow(const TensorView &Xx, float value, TensorView &Xz) {
        nv_detail::scalar(Xx, value, Xz, CXM_OP_POW, "ElementWise::pow");
    }
    static void pow(const TensorView &Xx, const TensorView &Xy, TensorView &Xz) {
        nv_detail::binary(Xx, Xy, Xz, CXM_OP_POW, "ElementWise::pow");
    }
    static void sqrt(const TensorView &Xx, TensorView &Xz) { nv_detail::unary(Xx, Xz, CXM_FN_SQRT, "ElementWise::sqrt"); }
    static void rsqrt(const TensorView &Xx, TensorView &Xz) { nv_detail::unary(Xx, Xz, CXM_FN_RSQRT, "ElementWise::rsqrt"); }
    static void log(const TensorView &Xx, TensorView &Xz) { nv_detail::unary(Xx, Xz, CXM_FN_LOG, "ElementWise::log"); }
    static void exp(const TensorView &Xx, TensorView &Xz) { nv_detail::unary(Xx, Xz, CXM_FN_EXP, "ElementWise::exp"); }
    static void erf(const TensorView &Xx, TensorView &Xz) { nv_detail::unary(Xx, Xz, CXM_FN_ERF, "ElementWise::erf"); }
    static void sin(const TensorView &Xx, TensorView &Xz) { nv_detail::unary(Xx, Xz, CXM_FN_SIN, "ElementWise::sin"); }
    static void cos(const TensorView &Xx, TensorView &Xz) { nv_detail::unary(Xx, Xz, CXM_FN_COS, "ElementWise::cos"); }
    static void abs(const TensorView &Xx, TensorView &Xz) { nv_detail::unary(Xx, Xz, CXM_FN_ABS, "ElementWise::abs"); }
    static void neg(const TensorView &Xx, TensorView &Xz) { nv_detail::unary(Xx, Xz, CXM_FN_NEG, "ElementWise::neg"); }
    static void rcp(const TensorView &Xx, TensorView &Xz) { nv_detail::unary(Xx, Xz, CXM_FN_RCP, "ElementWise::rcp"); }
    static void inverse(const TensorView &Xx, TensorView &Xz) {
        nv_detail::unary(Xx, Xz, CXM_FN_INVERSE, "ElementWise::inverse");
    }
    static void sign(const TensorView &Xx, TensorView &Xz) { nv_detail::unary(Xx, Xz, CXM_FN_SIGN, "ElementWise::sign"); }
};

// nv::Matrix (matrix.cuh:11-26, matrix.cu:40-202).
struct Matrix {
    static void add(const TensorView &Xx, const TensorView &Xy, TensorView &Xz) {
        nv_detail::binary(Xx, Xy, Xz, CXM_OP_ADD, "Matrix::add");
    }
    static void sub(const TensorView &Xx, const TensorView &Xy, TensorView &Xz) {
        nv_detail::binary(Xx, Xy, Xz, CXM_OP_SUB, "Matrix::sub");
    }
    static void mul(const TensorView &Xx, const TensorView &Xy, TensorView &Xz) {
        nv_detail::binary(Xx, Xy, Xz, CXM_OP_MUL, "Matrix::mul");
    }
    static void div(const TensorView &Xx, const TensorView &Xy, TensorView &Xz) {
        nv_detail::binary(Xx, Xy, Xz, CXM_OP_DIV, "Matrix::div");
    }
    static void max(const TensorView &Xx, const TensorView &Xy, TensorView &Xz) {
        nv_detail::binary(Xx, Xy, Xz, CXM_OP_MAX, "Matrix::max");
    }
    static void min(const TensorView &Xx, const TensorView &Xy, TensorView &Xz) {
        nv_detail::binary(Xx, Xy, Xz, CXM_OP_MIN, "Matrix::min");
    }
    // Row-major Xz[M, N] = Xx[M, K] * Xy[K, N], with M, K, N implied by the
    // three element counts.
    static void matmul(const TensorView &Xx, const TensorView &Xy, TensorView &Xz) {
        std::size_t m = 0, k = 0, n = 0;
        if (!nv_detail::dims(Xx.size(), Xy.size(), Xz.size(), &m, &k, &n))
            nv_detail::fail("Matrix::matmul", "element counts are not M*K, K*N, M*N");
        matmul(Xx, Xy, Xz, m, k, n);
    }
    static void matmul(const TensorView &Xx, const TensorView &Xy, TensorView &Xz, std::size_t M, std::size_t K,
                       std::size_t N) {
        const char *what = "Matrix::matmul";
        const int dt = nv_detail::code(Xx, what);
        if (nv_detail::code(Xy, what) != dt || nv_detail::code(Xz, what) != dt)
            nv_detail::fail(what, "operands differ in dtype");
        if (Xx.size() != M * K || Xy.size() != K * N || Xz.size() != M * N)
            nv_detail::fail(what, "element counts do not match M, K, N");
        check(cxm_matmul_t(Xx.data(), Xy.data(), Xz.data(), M, K, N, dt, stream()), what);
    }
    static void add(TensorView &Xx, const TensorView &Xy) { nv_detail::binary(Xx, Xy, Xx, CXM_OP_ADD, "Matrix::add"); }
    static void sub(TensorView &Xx, const TensorView &Xy) { nv_detail::binary(Xx, Xy, Xx, CXM_OP_SUB, "Matrix::sub"); }
    static void mul(TensorView &Xx, const TensorView &Xy) { nv_detail::binary(Xx, Xy, Xx, CXM_OP_MUL, "Matrix::mul"); }
    static void div(TensorView &Xx, const TensorView &Xy) { nv_detail::binary(Xx, Xy, Xx, CXM_OP_DIV, "Matrix::div"); }
};

// nv::ScalarKernel (scalar.cuh:25-99, scalar.cu:16-134).
struct ScalarKernel {
    static void add(const TensorView &Xx, float value, TensorView &Xz) {
        nv_detail::scalar(Xx, value, Xz, CXM_OP_ADD, "ScalarKernel::add");
    }
    static void sub(const TensorView &Xx, float value, TensorView &Xz) {
        nv_detail::scalar(Xx, value, Xz, CXM_OP_SUB, "ScalarKernel::sub");
    }
    static void mul(const TensorView &Xx, float value, TensorView &Xz) {
        nv_detail::scalar(Xx, value, Xz, CXM_OP_MUL, "ScalarKernel::mul");
    }
    static void div(const TensorView &Xx, float value, TensorView &Xz) {
        nv_detail::scalar(Xx, value, Xz, CXM_OP_DIV, "ScalarKernel::div");
    }
    static void add(TensorView &Xx, float value) { nv_detail::scalar(Xx, value, Xx, CXM_OP_ADD, "ScalarKernel::add"); }
    static void sub(TensorView &Xx, float value) { nv_detail::scalar(Xx, value, Xx, CXM_OP_SUB, "ScalarKernel::sub"); }
    static void mul(TensorView &Xx, float value) { nv_detail::scalar(Xx, value, Xx, CXM_OP_MUL, "ScalarKernel::mul"); }
    static void div(TensorView &Xx, float value) { nv_detail::scalar(Xx, value, Xx, CXM_OP_DIV, "ScalarKernel::div"); }
};

}  // namespace cortex::_fw::hip

#endif  // CORTEX_HIP_NV_HPP
