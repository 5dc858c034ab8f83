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

// DType, TensorView and the dtype dispatch (nv_detail) are defined in
// cortex_hip.hpp, which the pointer-form operator structs share.


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
