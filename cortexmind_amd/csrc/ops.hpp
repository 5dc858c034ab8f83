// Scalar operators shared by the fp32 and the 16-bit elementwise kernels:
// binary ops, activations and their derivative factors, and the unary math
// functions of the elementwise surface.  Each is the per-element
// expression the reference's operators apply (cited where defined); the
// library is built with -ffp-contract=off, so no product is fused into a
// sum unless fmaf says so.
#pragma once

#include "cxm_common.hpp"

namespace cxm {

template <int OP>
__device__ __forceinline__ float bin_t(float a, float b) {
    if constexpr (OP == CXM_OP_ADD) return a + b;
    else if constexpr (OP == CXM_OP_SUB) return a - b;
    else if constexpr (OP == CXM_OP_MUL) return a * b;
    else if constexpr (OP == CXM_OP_DIV) return a / b;
    else if constexpr (OP == CXM_OP_MAX) return a > b ? a : b;
    else if constexpr (OP == CXM_OP_MIN) return a < b ? a : b;
    else return powf(a, b);
}

// tanh(t) by the classic two-range method (an odd polynomial near 0, the
// exponential form beyond; e.g. W. J. Cody and W. Waite, Software Manual
// for the Elementary Functions, 1980, ch. 13), with coefficients of our own:
//  * |t| < 0.9: t + t^3 P(t^2), P of degree 5 fitted to (tanh(x) - x) / x^3
//    for the relative error of tanh on [0, 0.9] (iteratively reweighted
//    least squares toward minimax), Horner in fp32;
//  * otherwise q = (1 - e) / (1 + e) with e = exp(-2|t|) = 2^(|t| C),
//    C = fl(-2 / ln 2); the quotient is the hardware reciprocal times
//    1 - e, refined by one Newton step on the exact residual
//    (1 - q) - e - q e ((1 - q) - e is exact by Sterbenz for e <= 0.17), so
//    only the last rounding and e's error (scaled by 2e / (1 - e^2) <= 0.42)
//    remain.  |t| is clamped to 16 on that path (tanh rounds to 1 from 9.01
//    on), so infinities give +-1 and NaN stays NaN.
// Modelled in float64 with the exp2 and reciprocal estimates off by one ulp
// either way: at most 1.38 ulp; measured on the device against float64 in
// tests/test_elementwise_gpu.py.  No branches (the math library's tanhf
// branches on |t|).
__device__ __forceinline__ float tanh_f32(float t) {
    const float ax = fabsf(t);
    const float z = ax * ax;
    float p = 0x1.56e070p-10f;
    p = fmaf(p, z, -0x1.c2429ep-8f);
    p = fmaf(p, z, 0x1.56a8d2p-6f);
    p = fmaf(p, z, -0x1.b81fd0p-5f);
    p = fmaf(p, z, 0x1.1101fap-3f);
    p = fmaf(p, z, -0x1.555508p-2f);
    const float small = fmaf(ax * z, p, ax);
    const float a = ax > 16.0f ? 16.0f : ax;  // NaN stays NaN
    const float e = __builtin_amdgcn_exp2f(a * -0x1.715476p+1f);
    const float r0 = __builtin_amdgcn_rcpf(1.0f + e);
    const float q0 = (1.0f - e) * r0;
    const float res = fmaf(-e, q0, (1.0f - q0) - e);
    const float q = fmaf(r0, res, q0);
    return __builtin_copysignf(ax < 0.9f ? small : q, t);
}

// relu: functions.hpp:372-374; sigmoid: functions.hpp:405-411 (1/(1+exp(-x)));
// tanh: functions.hpp:381-383; exp: functions.hpp:186-188.
template <int ACT>
__device__ __forceinline__ float act(float t) {
    if constexpr (ACT == CXM_ACT_RELU) return 0.0f > t ? 0.0f : t;
    else if constexpr (ACT == CXM_ACT_SIGMOID) {
        // sigmoid(t) = n / (1 + e) with e = exp(-|t|) in [0, 1], n = 1 for
        // t >= 0 and n = e for t < 0.  The divisor stays in [1, 2] for every
        // t, so nothing overflows, and results below the normal range come
        // out of e itself.  The quotient is the hardware reciprocal estimate
        // (v_rcp_f32, about 1 ulp) times n, refined by one Newton-Raphson
        // step on the residual n - q (1 + e) = (n - q) - q e, formed from the
        // unrounded 1 + e: n - q is exact (Sterbenz: q lies in [n/2, n]) and
        // the fma rounds q e once.  This replaces the IEEE division's ten
        // or so instructions with four and is never less accurate.
        const float e = expf(-fabsf(t));
        const float n = t >= 0.0f ? 1.0f : e;
        const float r0 = __builtin_amdgcn_rcpf(1.0f + e);
        const float q0 = n * r0;
        const float res = fmaf(-q0, e, n - q0);
        return fmaf(r0, res, q0);
    } else if constexpr (ACT == CXM_ACT_TANH) return tanh_f32(t);
    else if constexpr (ACT == CXM_ACT_EXP) return expf(t);
    else return t;
}

// Derivative factor from the saved output y (one rounding per operation):
// relu' = y > 0, sigmoid' = y*(1-y), tanh' = 1 - y*y.
template <int ACT>
__device__ __forceinline__ float dact(float y) {
    if constexpr (ACT == CXM_ACT_RELU) return y > 0.0f ? 1.0f : 0.0f;
    else if constexpr (ACT == CXM_ACT_SIGMOID) {
        const float t = 1.0f - y;
        return y * t;
    } else if constexpr (ACT == CXM_ACT_TANH) {
        const float t = y * y;
        return 1.0f - t;
    } else return 1.0f;
}

// ------------------------------------------------ unary math functions
// (nv::ElementWise / avx2::wise: Operations/kernel_ops.cuh:73-284)

struct FSquare { __device__ float operator()(float x) const { return x * x; } };
struct FSqrt { __device__ float operator()(float x) const { return __builtin_sqrtf(x); } };
struct FRsqrt {
    __device__ float operator()(float x) const {
        const float r = __builtin_sqrtf(x);
        return 1.0f / r;
    }
};
struct FLog { __device__ float operator()(float x) const { return logf(x); } };
struct FExp { __device__ float operator()(float x) const { return expf(x); } };
struct FErf { __device__ float operator()(float x) const { return erff(x); } };
struct FSin { __device__ float operator()(float x) const { return sinf(x); } };
struct FCos { __device__ float operator()(float x) const { return cosf(x); } };
struct FAbs { __device__ float operator()(float x) const { return fabsf(x); } };
struct FNeg { __device__ float operator()(float x) const { return -x; } };
struct FRcp { __device__ float operator()(float x) const { return 1.0f / x; } };
// (x > 0) - (x < 0): Operations/kernel_ops.cuh:268-274
struct FSign {
    __device__ float operator()(float x) const {
        return static_cast<float>(static_cast<int>(x > 0.0f) - static_cast<int>(x < 0.0f));
    }
};
// fma(t, b - a, a) with a = x, b = v1, t = v2: functions.hpp:271-274
struct FLerp {
    float v1, v2;
    __device__ float operator()(float x) const {
        const float d = v1 - x;
        return fmaf(v2, d, x);
    }
};
// min(max(x, lo), hi) with the SIMD operand rule max(a, b) = a > b ? a : b,
// min(a, b) = a < b ? a : b: functions.hpp:332-335
struct FClamp {
    float lo, hi;
    __device__ float operator()(float x) const {
        const float m = x > lo ? x : lo;
        return m < hi ? m : hi;
    }
};

}  // namespace cxm
