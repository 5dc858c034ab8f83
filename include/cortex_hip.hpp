// cortex_hip.hpp -- C++ host layer of the gfx950 backend, mirroring the
// reference engine's static operator structs over the C ABI (cxm_hip.h).
//
// Names, argument order and meaning follow the reference's CPU engine
// (source/CortexMind/framework/Engine/AVX2/reduce.hpp:35-330,
// broadcast.hpp:20-80, matrix.hpp:30-160, scalar.hpp) with inputs Xx/Xy,
// output Xz and sizes last; pointers here are device pointers and every
// call is queued on hip::stream() (the null stream unless set).  Errors
// follow the reference's convention (CXM_ASSERT, Tools/Error/errors.cpp:
// 14-23: print a message and exit(1)) instead of returning a code.
// Header-only; link with -lcxm_hip.
#ifndef CORTEX_HIP_HPP
#define CORTEX_HIP_HPP

#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <type_traits>
#include <utility>
#include <vector>

#include "cxm_hip.h"

namespace cortex::_fw::hip {

// The stream every operator below is queued on (per thread).
inline cxm_stream_t &stream() {
    thread_local cxm_stream_t s = nullptr;
    return s;
}

// Exit on failure, as the reference's CXM_ASSERT / CXM_DEVICE_ASSERT do.
inline void check(int status, const char *what) {
    if (status != CXM_OK) {
        std::fprintf(stderr, "[ERROR] %s: %s\n", what, cxm_error_string(status));
        std::exit(1);
    }
}

// The reference's DeviceType (Memory/type.hpp:22-26) with the HIP device
// this backend adds.
enum class DeviceType : std::uint8_t { Unknown = 0, HOST = 1, CUDA = 2, HIP = 3 };

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

// Type/size.cpp:8-34: bytes per element (0 for Unknown).
inline std::size_t size_of(DType t) noexcept {
    switch (t) {
        case DType::Int32:
        case DType::Float32: return 4;
        case DType::Int64:
        case DType::Float64: return 8;
        case DType::BFloat16:
        case DType::Float16:
        case DType::QInt16:
        case DType::QUInt16: return 2;
        case DType::QInt8:
        case DType::QUInt8: return 1;
        default: return 0;
    }
}

// avx2::reduce (reduce.hpp:49-296): flat (Xx, Xz, N) and axis
// (Xx, Xz, outer_size, dim_size, inner_size) forms.
struct reduce {
    static void sum(const float *Xx, float *Xz, std::size_t N) {
        check(cxm_reduce_sum_flat_f32(Xx, Xz, N, stream()), "reduce::sum");
    }
    static void sum(const float *Xx, float *Xz, std::size_t outer, std::size_t dim, std::size_t inner) {
        check(cxm_reduce_sum_f32(Xx, Xz, outer, dim, inner, stream()), "reduce::sum");
    }
    static void mean(const float *Xx, float *Xz, std::size_t N) {
        check(cxm_reduce_mean_flat_f32(Xx, Xz, N, stream()), "reduce::mean");
    }
    static void mean(const float *Xx, float *Xz, std::size_t outer, std::size_t dim, std::size_t inner) {
        check(cxm_reduce_mean_f32(Xx, Xz, outer, dim, inner, stream()), "reduce::mean");
    }
    static void max(const float *Xx, float *Xz, std::size_t N) {
        check(cxm_reduce_max_flat_f32(Xx, Xz, N, stream()), "reduce::max");
    }
    static void max(const float *Xx, float *Xz, std::size_t outer, std::size_t dim, std::size_t inner) {
        check(cxm_reduce_max_f32(Xx, Xz, outer, dim, inner, stream()), "reduce::max");
    }
    static void argmax(const float *Xx, std::int32_t *Xz, std::size_t N) {
        check(cxm_reduce_argmax_flat_f32(Xx, Xz, N, stream()), "reduce::argmax");
    }
    static void argmax(const float *Xx, std::int32_t *Xz, std::size_t outer, std::size_t dim,
                       std::size_t inner) {
        check(cxm_reduce_argmax_f32(Xx, Xz, outer, dim, inner, stream()), "reduce::argmax");
    }
    static void argmin(const float *Xx, std::int32_t *Xz, std::size_t N) {
        check(cxm_reduce_argmin_flat_f32(Xx, Xz, N, stream()), "reduce::argmin");
    }
    static void argmin(const float *Xx, std::int32_t *Xz, std::size_t outer, std::size_t dim,
                       std::size_t inner) {
        check(cxm_reduce_argmin_f32(Xx, Xz, outer, dim, inner, stream()), "reduce::argmin");
    }
#define CXM_HIP_REDUCE(NAME)                                                                        \
    static void NAME(const float *Xx, float *Xz, std::size_t N) {                                   \
        check(cxm_reduce_##NAME##_flat_f32(Xx, Xz, N, stream()), "reduce::" #NAME);                 \
    }                                                                                               \
    static void NAME(const float *Xx, float *Xz, std::size_t outer, std::size_t dim, std::size_t inner) { \
        check(cxm_reduce_##NAME##_f32(Xx, Xz, outer, dim, inner, stream()), "reduce::" #NAME);      \
    }
    // reduce.hpp:96-263: var, stdv, min, norm1, norm2
    CXM_HIP_REDUCE(var)
    CXM_HIP_REDUCE(stdv)
    CXM_HIP_REDUCE(min)
    CXM_HIP_REDUCE(norm1)
    CXM_HIP_REDUCE(norm2)
#undef CXM_HIP_REDUCE
};

// avx2::Broadcast::row / ::col (broadcast.hpp:20-57): out-of-place
// (Xx, Xy, Xz, M, N) and in-place (Xx, Xy, M, N).
struct Broadcast {
    template <int ROW>
    struct axis {
        static void run(const float *Xx, const float *Xy, float *Xz, std::size_t M, std::size_t N, int op) {
            check(ROW ? cxm_bcast_row_f32(Xx, Xy, Xz, M, N, op, stream())
                      : cxm_bcast_col_f32(Xx, Xy, Xz, M, N, op, stream()),
                  ROW ? "Broadcast::row" : "Broadcast::col");
        }
        static void add(const float *Xx, const float *Xy, float *Xz, std::size_t M, std::size_t N) { run(Xx, Xy, Xz, M, N, CXM_OP_ADD); }
        static void sub(const float *Xx, const float *Xy, float *Xz, std::size_t M, std::size_t N) { run(Xx, Xy, Xz, M, N, CXM_OP_SUB); }
        static void mul(const float *Xx, const float *Xy, float *Xz, std::size_t M, std::size_t N) { run(Xx, Xy, Xz, M, N, CXM_OP_MUL); }
        static void div(const float *Xx, const float *Xy, float *Xz, std::size_t M, std::size_t N) { run(Xx, Xy, Xz, M, N, CXM_OP_DIV); }
        static void add(float *Xx, const float *Xy, std::size_t M, std::size_t N) { run(Xx, Xy, Xx, M, N, CXM_OP_ADD); }
        static void sub(float *Xx, const float *Xy, std::size_t M, std::size_t N) { run(Xx, Xy, Xx, M, N, CXM_OP_SUB); }
        static void mul(float *Xx, const float *Xy, std::size_t M, std::size_t N) { run(Xx, Xy, Xx, M, N, CXM_OP_MUL); }
        static void div(float *Xx, const float *Xy, std::size_t M, std::size_t N) { run(Xx, Xy, Xx, M, N, CXM_OP_DIV); }
    };
    using row = axis<1>;
    using col = axis<0>;
};

// avx2::matrix_t (matrix.hpp:38-160): same-shape ops and matmul.
struct matrix_t {
    static void op(const float *Xx, const float *Xy, float *Xz, std::size_t N, int code) {
        check(cxm_binary_f32(Xx, Xy, Xz, N, code, stream()), "matrix_t");
    }
    static void add(const float *Xx, const float *Xy, float *Xz, std::size_t N) { op(Xx, Xy, Xz, N, CXM_OP_ADD); }
    static void sub(const float *Xx, const float *Xy, float *Xz, std::size_t N) { op(Xx, Xy, Xz, N, CXM_OP_SUB); }
    static void mul(const float *Xx, const float *Xy, float *Xz, std::size_t N) { op(Xx, Xy, Xz, N, CXM_OP_MUL); }
    static void div(const float *Xx, const float *Xy, float *Xz, std::size_t N) { op(Xx, Xy, Xz, N, CXM_OP_DIV); }
    static void max(const float *Xx, const float *Xy, float *Xz, std::size_t N) { op(Xx, Xy, Xz, N, CXM_OP_MAX); }
    static void min(const float *Xx, const float *Xy, float *Xz, std::size_t N) { op(Xx, Xy, Xz, N, CXM_OP_MIN); }
    static void add(float *Xx, const float *Xy, std::size_t N) { op(Xx, Xy, Xx, N, CXM_OP_ADD); }
    static void sub(float *Xx, const float *Xy, std::size_t N) { op(Xx, Xy, Xx, N, CXM_OP_SUB); }
    static void mul(float *Xx, const float *Xy, std::size_t N) { op(Xx, Xy, Xx, N, CXM_OP_MUL); }
    static void div(float *Xx, const float *Xy, std::size_t N) { op(Xx, Xy, Xx, N, CXM_OP_DIV); }
    // Row-major Xz[xN, zN] = Xx[xN, yN] * Xy[yN, zN] (matrix.hpp:119).
    static void matmul(const float *Xx, const float *Xy, float *Xz, std::size_t xN, std::size_t yN, std::size_t zN) {
        check(cxm_matmul_f32(Xx, Xy, Xz, xN, yN, zN, stream()), "matrix_t::matmul");
    }
};

// avx2::ScalarOp (Engine/AVX2/scalar.hpp:25-104, scalar.cpp:89-119):
// Xz = Xx op value over TensorViews, out of place and in place, as the
// reference declares them; views of Float32, BFloat16 or Float16 device
// memory (the 16-bit forms widen, apply the fp32 operator and round once).
// The pointer forms (Xx, value, Xz, N) are kept for fp32 callers.
struct ScalarOp {
    static void add(const TensorView &Xx, float value, TensorView &Xz) { nv_detail::scalar(Xx, value, Xz, CXM_OP_ADD, "ScalarOp::add"); }
    static void sub(const TensorView &Xx, float value, TensorView &Xz) { nv_detail::scalar(Xx, value, Xz, CXM_OP_SUB, "ScalarOp::sub"); }
    static void mul(const TensorView &Xx, float value, TensorView &Xz) { nv_detail::scalar(Xx, value, Xz, CXM_OP_MUL, "ScalarOp::mul"); }
    static void div(const TensorView &Xx, float value, TensorView &Xz) { nv_detail::scalar(Xx, value, Xz, CXM_OP_DIV, "ScalarOp::div"); }
    static void add(TensorView &Xx, float value) { nv_detail::scalar(Xx, value, Xx, CXM_OP_ADD, "ScalarOp::add"); }
    static void sub(TensorView &Xx, float value) { nv_detail::scalar(Xx, value, Xx, CXM_OP_SUB, "ScalarOp::sub"); }
    static void mul(TensorView &Xx, float value) { nv_detail::scalar(Xx, value, Xx, CXM_OP_MUL, "ScalarOp::mul"); }
    static void div(TensorView &Xx, float value) { nv_detail::scalar(Xx, value, Xx, CXM_OP_DIV, "ScalarOp::div"); }

    static void op(const float *Xx, float v, float *Xz, std::size_t N, int code) {
        check(cxm_scalar_f32(Xx, v, Xz, N, code, stream()), "ScalarOp");
    }
    static void add(const float *Xx, float v, float *Xz, std::size_t N) { op(Xx, v, Xz, N, CXM_OP_ADD); }
    static void sub(const float *Xx, float v, float *Xz, std::size_t N) { op(Xx, v, Xz, N, CXM_OP_SUB); }
    static void mul(const float *Xx, float v, float *Xz, std::size_t N) { op(Xx, v, Xz, N, CXM_OP_MUL); }
    static void div(const float *Xx, float v, float *Xz, std::size_t N) { op(Xx, v, Xz, N, CXM_OP_DIV); }
};

// avx2::wise (Engine/AVX2/wise.hpp:27-47): Xz = fn(Xx) over TensorViews, as
// the reference declares square..sign and both pow forms (Float32,
// BFloat16 or Float16 device views), plus pointer forms over N fp32
// elements; lerp, clamp and gather are pointer forms in the reference too.
struct wise {
    static void square(const TensorView &Xx, TensorView &Xz) { nv_detail::unary(Xx, Xz, CXM_FN_SQUARE, "wise::square"); }
    static void sqrt(const TensorView &Xx, TensorView &Xz) { nv_detail::unary(Xx, Xz, CXM_FN_SQRT, "wise::sqrt"); }
    static void rsqrt(const TensorView &Xx, TensorView &Xz) { nv_detail::unary(Xx, Xz, CXM_FN_RSQRT, "wise::rsqrt"); }
    static void log(const TensorView &Xx, TensorView &Xz) { nv_detail::unary(Xx, Xz, CXM_FN_LOG, "wise::log"); }
    static void exp(const TensorView &Xx, TensorView &Xz) { nv_detail::unary(Xx, Xz, CXM_FN_EXP, "wise::exp"); }
    static void erf(const TensorView &Xx, TensorView &Xz) { nv_detail::unary(Xx, Xz, CXM_FN_ERF, "wise::erf"); }
    static void sin(const TensorView &Xx, TensorView &Xz) { nv_detail::unary(Xx, Xz, CXM_FN_SIN, "wise::sin"); }
    static void cos(const TensorView &Xx, TensorView &Xz) { nv_detail::unary(Xx, Xz, CXM_FN_COS, "wise::cos"); }
    static void abs(const TensorView &Xx, TensorView &Xz) { nv_detail::unary(Xx, Xz, CXM_FN_ABS, "wise::abs"); }
    static void neg(const TensorView &Xx, TensorView &Xz) { nv_detail::unary(Xx, Xz, CXM_FN_NEG, "wise::neg"); }
    static void rcp(const TensorView &Xx, TensorView &Xz) { nv_detail::unary(Xx, Xz, CXM_FN_RCP, "wise::rcp"); }
    static void inverse(const TensorView &Xx, TensorView &Xz) { nv_detail::unary(Xx, Xz, CXM_FN_INVERSE, "wise::inverse"); }
    static void sign(const TensorView &Xx, TensorView &Xz) { nv_detail::unary(Xx, Xz, CXM_FN_SIGN, "wise::sign"); }
    static void pow(const TensorView &Xx, float value, TensorView &Xz) {
        nv_detail::scalar(Xx, value, Xz, CXM_OP_POW, "wise::pow");
    }
    static void pow(const TensorView &Xx, const TensorView &Xy, TensorView &Xz) {
        nv_detail::binary(Xx, Xy, Xz, CXM_OP_POW, "wise::pow");
    }

    static void fn(const float *Xx, float *Xz, std::size_t N, int code) {
        check(cxm_wise_f32(Xx, Xz, N, code, stream()), "wise");
    }
    static void square(const float *Xx, float *Xz, std::size_t N) { fn(Xx, Xz, N, CXM_FN_SQUARE); }
    static void sqrt(const float *Xx, float *Xz, std::size_t N) { fn(Xx, Xz, N, CXM_FN_SQRT); }
    static void rsqrt(const float *Xx, float *Xz, std::size_t N) { fn(Xx, Xz, N, CXM_FN_RSQRT); }
    static void log(const float *Xx, float *Xz, std::size_t N) { fn(Xx, Xz, N, CXM_FN_LOG); }
    static void exp(const float *Xx, float *Xz, std::size_t N) { fn(Xx, Xz, N, CXM_FN_EXP); }
    static void erf(const float *Xx, float *Xz, std::size_t N) { fn(Xx, Xz, N, CXM_FN_ERF); }
    static void sin(const float *Xx, float *Xz, std::size_t N) { fn(Xx, Xz, N, CXM_FN_SIN); }
    static void cos(const float *Xx, float *Xz, std::size_t N) { fn(Xx, Xz, N, CXM_FN_COS); }
    static void abs(const float *Xx, float *Xz, std::size_t N) { fn(Xx, Xz, N, CXM_FN_ABS); }
    static void neg(const float *Xx, float *Xz, std::size_t N) { fn(Xx, Xz, N, CXM_FN_NEG); }
    static void rcp(const float *Xx, float *Xz, std::size_t N) { fn(Xx, Xz, N, CXM_FN_RCP); }
    static void inverse(const float *Xx, float *Xz, std::size_t N) { fn(Xx, Xz, N, CXM_FN_INVERSE); }
    static void sign(const float *Xx, float *Xz, std::size_t N) { fn(Xx, Xz, N, CXM_FN_SIGN); }
    static void pow(const float *Xx, float value, float *Xz, std::size_t N) {
        check(cxm_scalar_f32(Xx, value, Xz, N, CXM_OP_POW, stream()), "wise::pow");
    }
    static void pow(const float *Xx, const float *Xy, float *Xz, std::size_t N) {
        check(cxm_binary_f32(Xx, Xy, Xz, N, CXM_OP_POW, stream()), "wise::pow");
    }
    // wise.hpp:44-47 (the gather forms take the size of Xx as well, for bounds)
    static void lerp(const float *Xx, float value1, float value2, float *Xz, std::size_t N) {
        check(cxm_lerp_f32(Xx, value1, value2, Xz, N, stream()), "wise::lerp");
    }
    static void clamp(const float *Xx, float min, float max, float *Xz, std::size_t N) {
        check(cxm_clamp_f32(Xx, min, max, Xz, N, stream()), "wise::clamp");
    }
    static void gather(const float *Xx, std::size_t Nx, const std::int32_t *Xy, float *Xz, std::size_t N) {
        check(cxm_gather_f32(Xx, Nx, Xy, Xz, N, stream()), "wise::gather");
    }
    static void gather(const std::int32_t *Xx, std::size_t Nx, const std::int32_t *Xy, std::int32_t *Xz,
                       std::size_t N) {
        check(cxm_gather_i32(Xx, Nx, Xy, Xz, N, stream()), "wise::gather");
    }
};

// Tensor-level forms of avx2::relu / sigmoid / tanh / exp (functions.hpp:
// 186-188, 372-374, 381-383, 405-411), which the reference has only as
// 8-lane register functions.
struct activation {
    static void relu(const float *Xx, float *Xz, std::size_t N) { check(cxm_unary_f32(Xx, Xz, N, CXM_ACT_RELU, stream()), "relu"); }
    static void sigmoid(const float *Xx, float *Xz, std::size_t N) { check(cxm_unary_f32(Xx, Xz, N, CXM_ACT_SIGMOID, stream()), "sigmoid"); }
    static void tanh(const float *Xx, float *Xz, std::size_t N) { check(cxm_unary_f32(Xx, Xz, N, CXM_ACT_TANH, stream()), "tanh"); }
    static void exp(const float *Xx, float *Xz, std::size_t N) { check(cxm_unary_f32(Xx, Xz, N, CXM_ACT_EXP, stream()), "exp"); }
};

// ------------------------------------------------------------ storage

// TensorStorage (Storage/storage.hpp:14-57) for the host and HIP devices:
// an owning, move-only byte buffer.  HIP memory comes from the library's
// stream-ordered caching pool (cxm_pool_alloc on hip::stream()), in place
// of the reference's fixed 128 MiB ForgeChunk; host memory is 64-byte
// aligned.  Unlike the reference's move assignment (Storage/operator.cpp:
// 25-31, which frees the buffer it just took), moving transfers ownership.
class Storage {
public:
    Storage() = default;
    Storage(std::size_t bytes, DeviceType type) : bytes_(bytes), device_(type) {
        if (bytes_ == 0) return;
        if (type == DeviceType::HIP) {
            void *p = nullptr;
            check(cxm_pool_alloc(&p, bytes_, stream()), "Storage: device allocation");
            data_ = static_cast<std::byte *>(p);
        } else if (type == DeviceType::HOST) {
            data_ = static_cast<std::byte *>(std::aligned_alloc(64, (bytes_ + 63) / 64 * 64));
            if (!data_) check(CXM_E_INVALID, "Storage: host allocation");
        } else {
            check(CXM_E_INVALID, "Storage: unsupported device");
        }
    }
    // A copy of `bytes` of host memory at `data` on device `type`.
    Storage(std::size_t bytes, const std::byte *data, DeviceType type) : Storage(bytes, type) {
        if (!bytes_) return;
        if (type == DeviceType::HIP) check(cxm_memcpy_h2d(data_, data, bytes_, stream()), "Storage: upload");
        else std::memcpy(data_, data, bytes_);
        if (type == DeviceType::HIP) check(cxm_stream_sync(stream()), "Storage: upload");
    }
    Storage(const Storage &) = delete;
    Storage &operator=(const Storage &) = delete;
    Storage(Storage &&o) noexcept { swap(o); }
    Storage &operator=(Storage &&o) noexcept {
        if (this != &o) {
            Storage t(std::move(o));
            swap(t);
        }
        return *this;
    }
    ~Storage() { reset(); }

    template <class T>
    T *as() { return reinterpret_cast<T *>(data_); }
    template <class T>
    const T *as() const { return reinterpret_cast<const T *>(data_); }
    std::byte *raw() noexcept { return data_; }
    const std::byte *raw() const noexcept { return data_; }
    std::size_t bytes() const noexcept { return bytes_; }
    bool isEmpty() const noexcept { return bytes_ == 0; }
    bool isValid() const noexcept { return data_ != nullptr || bytes_ == 0; }
    DeviceType device() const noexcept { return device_; }

    // A copy on the same device (TensorStorage::clone).
    Storage clone() const { return copy_to(device_); }
    // A copy on `type` (the data movement of Tensor::to, Tensor/tensor.cpp:151-171).
    Storage copy_to(DeviceType type) const {
        Storage out(bytes_, type);
        if (!bytes_) return out;
        if (device_ == DeviceType::HIP && type == DeviceType::HIP)
            check(cxm_memcpy_d2d(out.data_, data_, bytes_, stream()), "Storage: copy");
        else if (device_ == DeviceType::HIP)
            check(cxm_memcpy_d2h(out.data_, data_, bytes_, stream()), "Storage: download");
        else if (type == DeviceType::HIP) {
            check(cxm_memcpy_h2d(out.data_, data_, bytes_, stream()), "Storage: upload");
            check(cxm_stream_sync(stream()), "Storage: upload");
        } else
            std::memcpy(out.data_, data_, bytes_);
        return out;
    }

private:
    void swap(Storage &o) noexcept {
        std::swap(data_, o.data_);
        std::swap(bytes_, o.bytes_);
        std::swap(device_, o.device_);
    }
    void reset() noexcept {
        if (data_) {
            if (device_ == DeviceType::HIP) (void)cxm_pool_free(data_);
            else std::free(data_);
        }
        data_ = nullptr;
        bytes_ = 0;
    }
    std::byte *data_ = nullptr;
    std::size_t bytes_ = 0;
    DeviceType device_ = DeviceType::Unknown;
};

// A dense row-major tensor on the host or the HIP device: the part of the
// reference's Tensor (Tensor/tensor.hpp:26-150) the operators and the
// autograd flows need -- shape, dtype, storage, device, to(), view(), the
// gradient and the producing flow.  The constructor takes the reference's
// arguments in its order and with its defaults (Tensor/tensor.hpp:29-31:
// Float32 on the HOST, no gradient); storage is size_of(dtype) bytes per
// element.  The fp32 accessors (data(), host(), from_host) check the dtype.
struct GradientFlow;
class Tensor {
public:
    Tensor() = default;
    explicit Tensor(std::vector<std::int64_t> shape, DType type = DType::Float32, DeviceType d = DeviceType::HOST,
                    bool requires_grad = false)
        : shape_(std::move(shape)), dtype_(type), requires_grad_(requires_grad) {
        if (size_of(type) == 0) check(CXM_E_INVALID, "Tensor: unsupported DType");
        storage_ = std::make_shared<Storage>(len() * size_of(type), d);
    }
    // A HIP fp32 tensor holding a copy of host data.
    static Tensor from_host(std::vector<std::int64_t> shape, const float *data, bool requires_grad = false) {
        Tensor t;
        t.shape_ = std::move(shape);
        t.requires_grad_ = requires_grad;
        t.storage_ = std::make_shared<Storage>(t.len() * sizeof(float), reinterpret_cast<const std::byte *>(data),
                                               DeviceType::HIP);
        return t;
    }

    std::size_t len() const noexcept {
        std::size_t n = 1;
        for (auto d : shape_) n *= static_cast<std::size_t>(d);
        return n;
    }
    std::size_t ndim() const noexcept { return shape_.size(); }
    const std::vector<std::int64_t> &shape() const noexcept { return shape_; }
    std::int64_t dim(std::size_t i) const { return shape_.at(i); }
    DType dtype() const noexcept { return dtype_; }
    DeviceType device() const noexcept { return storage_ ? storage_->device() : DeviceType::Unknown; }
    bool empty() const noexcept { return !storage_ || storage_->isEmpty(); }
    float *data() { return get<float>(); }
    const float *data() const { return get<float>(); }
    std::byte *raw() noexcept { return storage_ ? storage_->raw() : nullptr; }
    const std::byte *raw() const noexcept { return storage_ ? storage_->raw() : nullptr; }

    // Tensor::get<T> (tensor.hpp:64-77): the storage as T, which must be the
    // element type of the tensor's dtype (std::uint16_t for the 16-bit types).
    template <class T>
    T *get() {
        check_type<T>();
        return storage_->as<T>();
    }
    template <class T>
    const T *get() const {
        check_type<T>();
        return storage_->as<T>();
    }

    // Tensor::view (tensor.hpp:124-125, tensor.cpp:183-185): a non-owning
    // view of the elements, what the nv:: operators and the TensorView forms
    // of ScalarOp / wise take.
    TensorView view() const noexcept { return TensorView(storage_ ? storage_->raw() : nullptr, dtype_, device(), len()); }

    // Tensor::to (Tensor/tensor.cpp:151-171): moves the data to `type`.
    Tensor &to(DeviceType type) {
        if (device() != type) storage_ = std::make_shared<Storage>(storage_->copy_to(type));
        return *this;
    }
    std::vector<float> host() const {
        std::vector<float> out(len());
        if (device() == DeviceType::HIP)
            check(cxm_memcpy_d2h(out.data(), data(), len() * sizeof(float), stream()), "Tensor: download");
        else
            std::memcpy(out.data(), data(), len() * sizeof(float));
        return out;
    }

    bool isRequired() const noexcept { return requires_grad_; }
    bool has_grad() const noexcept { return grad_ != nullptr; }
    Tensor &grad() { return *grad_; }
    std::shared_ptr<Tensor> &grad_ptr() { return grad_; }
    std::shared_ptr<GradientFlow> &flow() { return flow_; }
    // Same tensor (shared storage, gradient and flow), as a handle.
    std::shared_ptr<Storage> storage() const { return storage_; }

private:
    template <class T>
    void check_type() const {
        const bool ok = (std::is_same_v<T, float> && dtype_ == DType::Float32) ||
                        (std::is_same_v<T, double> && dtype_ == DType::Float64) ||
                        (std::is_same_v<T, std::int32_t> && dtype_ == DType::Int32) ||
                        (std::is_same_v<T, std::int64_t> && dtype_ == DType::Int64) ||
                        (std::is_same_v<T, std::uint16_t> && size_of(dtype_) == 2) ||
                        (std::is_same_v<T, std::byte>);
        if (!ok) check(CXM_E_INVALID, "Tensor::get: element type does not match the tensor's DType");
    }

    std::vector<std::int64_t> shape_;
    DType dtype_ = DType::Float32;
    std::shared_ptr<Storage> storage_;
    std::shared_ptr<Tensor> grad_;
    std::shared_ptr<GradientFlow> flow_;
    bool requires_grad_ = false;
};

}  // namespace cortex::_fw::hip

#endif  // CORTEX_HIP_HPP
