// Scalar operators shared by the fp32 and the 16-bit elementwise kernels:
// binary ops, activations and their derivative factors, and the unary math
// functions of the elementwise surface.  Each is the per-element
// expression the reference's operators apply (cited where defined); the
// library is built with -ffp-contract=off, so no product is fused into a
// sum unless fmaf says so.
#pragma once

#include "cxm_common.hpp"

namespace cxm {

// powf(x, y) as 2^(y log2|x|) with log2|x| in double-float arithmetic
// (a head and a tail of fp32, about 2^-45 apart), the classic scheme of
// table-free pow implementations (e.g. P. T. P. Tang, "Table-driven
// implementation of the logarithm function in IEEE floating-point
// arithmetic", ACM TOMS 16(4), 1990, for the atanh form of the logarithm):
//  * |x| = m 2^e with m in [sqrt(1/2), sqrt(2)) (v_frexp_*), u = (m-1)/(m+1)
//    as uh + ul (the division's exact fma residual), |u| <= 0.1716;
//  * log2 m = u (2/ln 2) + u^3 S(u^2), S the atanh series (2/ln 2)(1/3 +
//    w/5 + w^2/7 + ... + w^5/13), truncated at 4e-12 of log2 m; u (2/ln 2)
//    and u^3 S0 (S0 = 2/(3 ln 2)) carried as double-float products (fma
//    splits of the constants and of u^3 = uh^3 + 3 uh^2 ul), the rest of S
//    in fp32;
//  * t = y log2|x| as th + tl, k = rint(th), 2^(th - k + tl) by a degree-6
//    polynomial fitted on [-1/2, 1/2] (relative error below 2^-28), then
//    v_ldexp by k (one rounding in the subnormal range);
//  * the IEEE / C99 special cases (pow(x, +-0) = pow(1, y) = 1, NaN
//    operands, zeros, infinities, negative x with integer or other y) by
//    selects, no branches.
// Modelled in float64 with exact fp32 rounding: at most 1.06 ulp over
// x in [1e-38, 1e38] and |y| up to 1000 with finite results (the edges of
// m's interval with |y| up to 140 included); tested on the device against
// float64 in tests/test_wise_gpu.py.  About a third of the math library's
// powf instructions, which made pow ALU-bound.
__device__ __forceinline__ float pow_f32(float x, float y) {
    const float ax = fabsf(x), ay = fabsf(y);
    float m = __builtin_amdgcn_frexp_mantf(ax);  // [0.5, 1) for finite nonzero x
    int ei = __builtin_amdgcn_frexp_expf(ax);
    const bool low = m < 0x1.6a09e6p-1f;  // fl(sqrt(1/2))
    m = low ? m + m : m;
    ei = low ? ei - 1 : ei;
    const float e = static_cast<float>(ei);
    // u = (m - 1) / (m + 1) = uh + ul; m + 1 = dh + dl exactly
    const float f = m - 1.0f;
    const float dh = m + 1.0f;
    const float dl = m - (dh - 1.0f);
    const float r = __builtin_amdgcn_rcpf(dh);
    const float uh = f * r;
    const float e1 = fmaf(-uh, dl, fmaf(-uh, dh, f));
    const float ul = e1 * r;
    // u^3 = ch + cl
    const float wh = uh * uh;
    const float wl = fmaf(uh, uh, -wh);
    const float ch = uh * wh;
    const float cl = fmaf(3.0f * wh, ul, fmaf(uh, wl, fmaf(uh, wh, -ch)));
    // S - S0 = w (2/ln 2)(1/5 + w/7 + w^2/9 + w^3/11 + w^4/13)
    float rr = 0x1.c68f56p-3f;
    rr = fmaf(rr, wh, 0x1.0c9a84p-2f);
    rr = fmaf(rr, wh, 0x1.484b14p-2f);
    rr = fmaf(rr, wh, 0x1.a61762p-2f);
    rr = fmaf(rr, wh, 0x1.2776c6p-1f);
    const float dlt = wh * rr;
    constexpr float S0h = 0x1.ec709ep-1f, S0l = -0x1.e2fe02p-28f;  // 2/(3 ln 2)
    constexpr float Ah = 0x1.715476p+1f, Al = 0x1.4ae0c0p-25f;    // 2/ln 2
    const float th3 = ch * S0h;  // u^3 S = th3 + tl3
    const float tl3 = fmaf(cl, S0h, fmaf(ch, S0l + dlt, fmaf(ch, S0h, -th3)));
    const float ph = uh * Ah;  // u (2/ln 2) = ph + pl
    const float pl = fmaf(ul, Ah, fmaf(uh, Al, fmaf(uh, Ah, -ph)));
    const float lh = ph + th3;  // log2 m = lh + ll (|ph| >= |th3|)
    const float ll = (pl + tl3) + (th3 - (lh - ph));
    const float Lh = e + lh;  // log2|x| = Lh + Ll (e = 0 or |e| >= 1 > |lh|)
    const float Ll = (lh - (Lh - e)) + ll;
    // 2^(y log2|x|)
    const float th = y * Lh;
    const float tl = fmaf(y, Ll, fmaf(y, Lh, -th));
    // beyond +-160 the result is inf or 0 whatever the tail (which may be
    // huge there): k saturates and the fraction is 0; NaN is replaced below
    const bool in = th >= -160.0f && th <= 160.0f;
    const float tc = th > 160.0f ? 160.0f : (th < -160.0f ? -160.0f : th);
    const float k = __builtin_rintf(tc);
    const float fr = in ? (tc - k) + tl : 0.0f;
    float q = 0x1.4258f6p-13f;
    q = fmaf(q, fr, 0x1.5f44d4p-10f);
    q = fmaf(q, fr, 0x1.3b2cc4p-7f);
    q = fmaf(q, fr, 0x1.c6aed6p-5f);
    q = fmaf(q, fr, 0x1.ebfbdcp-3f);
    q = fmaf(q, fr, 0x1.62e430p-1f);
    float res = __builtin_amdgcn_ldexpf(fmaf(fr, q, 1.0f), static_cast<int>(k));
    // special cases
    const bool yint = __builtin_rintf(y) == y;  // +-inf count as (even) integers; NaN does not
    const int yi = ay < 0x1p24f ? static_cast<int>(y) : 0;
    const bool yodd = yint && (yi & 1);
    const float inf = __builtin_inff();
    res = ax == 0.0f ? (y < 0.0f ? inf : 0.0f) : res;
    res = ax == inf ? (y < 0.0f ? 0.0f : inf) : res;
    res = ay == inf ? (ax == 1.0f ? 1.0f : ((ax < 1.0f) == (y < 0.0f) ? inf : 0.0f)) : res;
    res = (__builtin_signbitf(x) && yodd) ? -res : res;
    res = (x < 0.0f && x > -inf && !yint) ? __builtin_nanf("") : res;
    res = (x != x || y != y) ? __builtin_nanf("") : res;
    return (y == 0.0f || x == 1.0f) ? 1.0f : res;
}

template <int OP>
__device__ __forceinline__ float bin_t(float a, float b) {
    if constexpr (OP == CXM_OP_ADD) return a + b;
    else if constexpr (OP == CXM_OP_SUB) return a - b;
    else if constexpr (OP == CXM_OP_MUL) return a * b;
    else if constexpr (OP == CXM_OP_DIV) return a / b;
    else if constexpr (OP == CXM_OP_MAX) return a > b ? a : b;
    else if constexpr (OP == CXM_OP_MIN) return a < b ? a : b;
    else return pow_f32(a, b);
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
