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

// avx2::ScalarOp (scalar.cpp:89-119): Xz = Xx op value.
struct ScalarOp {
    static void op(const float *Xx, float v, float *Xz, std::size_t N, int code) {
        check(cxm_scalar_f32(Xx, v, Xz, N, code, stream()), "ScalarOp");
    }
    static void add(const float *Xx, float v, float *Xz, std::size_t N) { op(Xx, v, Xz, N, CXM_OP_ADD); }
    static void sub(const float *Xx, float v, float *Xz, std::size_t N) { op(Xx, v, Xz, N, CXM_OP_SUB); }
    static void mul(const float *Xx, float v, float *Xz, std::size_t N) { op(Xx, v, Xz, N, CXM_OP_MUL); }
    static void div(const float *Xx, float v, float *Xz, std::size_t N) { op(Xx, v, Xz, N, CXM_OP_DIV); }
};

// avx2::wise / nv::ElementWise (Engine/AVX2/wise.hpp:28-42,
// Engine/CUDA/element_wise.cuh:11-27) in pointer form: Xz = fn(Xx) over N.
struct wise {
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

}  // namespace cortex::_fw::hip

#endif  // CORTEX_HIP_HPP
