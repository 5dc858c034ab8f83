// Elementwise math surface: z = fn(x) for the unary functions of the
// reference's GPU and CPU engines, plus lerp, clamp and gather.
//
// Replaces kernels::Unary<Op> (source/CortexMind/framework/Engine/Kernels/
// unary.cuh:16-40) as instantiated by nv::ElementWise (Engine/CUDA/
// element_wise.cu:17-181), and the fp32 branch of avx2::wise (Engine/AVX2/
// wise.cpp:56-194).  pow lives with the binary/scalar operator kernels.
//
// Each function is the correctly rounded IEEE operation where one exists
// (x*x, sqrt, 1/x, |x|, -x); rsqrt is 1/sqrt(x), two correctly rounded
// steps; log/exp/erf/sin/cos are the device math library's functions.  The
// reference's AVX2 body uses 12-bit approximations for rcp and rsqrt
// (_mm256_rcp_ps / _mm256_rsqrt_ps, functions.hpp:168-170, 240-242) and its
// CUDA build compiles with --use_fast_math; the results here are at least as
// accurate as either.
#include "cxm_common.hpp"
#include "ops.hpp"

namespace cxm {
namespace {

template <class F>
__global__ __launch_bounds__(kBlock) void k_map_any(F f, const float *x, float *z, size_t n) {
    const size_t stride = static_cast<size_t>(gridDim.x) * kBlock;
    for (size_t i = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride)
        z[i] = f(x[i]);
}

// Grid-stride launch for the unaligned and gather kernels: at most 16
// workgroups per CU, each thread striding through the rest.
inline unsigned map_grid(size_t units) {
    size_t b = (units + kBlock - 1) / kBlock;
    const size_t cap = 256 * 16;
    return static_cast<unsigned>(b < 1 ? 1 : (b > cap ? cap : b));
}

inline hipStream_t hs(cxm_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// 16-byte aligned: the one-float4-per-thread streaming map; otherwise a
// scalar grid-stride loop.
template <class F>
int map(F f, const float *x, float *z, size_t n, cxm_stream_t s) {
    if (aligned16(x) && aligned16(z)) {
        const unsigned g = map4_grid(n);
        if (!g) return CXM_E_TOO_LARGE;
        hipLaunchKernelGGL(k_map4<F>, dim3(g), dim3(kBlock), 0, hs(s), f, x, z, n);
    } else {
        hipLaunchKernelGGL(k_map_any<F>, dim3(map_grid(n)), dim3(kBlock), 0, hs(s), f, x, z, n);
    }
    return launch_status();
}

// z[i] = x[idx[i]]; an index outside [0, xn) gives `bad` and reads nothing.
template <class T>
__global__ __launch_bounds__(kBlock) void k_gather(const T *__restrict__ x, size_t xn,
                                                   const int32_t *__restrict__ idx, T *z, size_t n,
                                                   T bad) {
    const size_t stride = static_cast<size_t>(gridDim.x) * kBlock;
    for (size_t i = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
        const int32_t k = idx[i];
        z[i] = (k >= 0 && static_cast<size_t>(k) < xn) ? x[k] : bad;
    }
}

}  // namespace
}  // namespace cxm

using namespace cxm;

extern "C" {

int cxm_wise_f32(const float *x, float *z, size_t n, int fn, cxm_stream_t s) {
    if (!x || !z || fn < CXM_FN_SQUARE || fn > CXM_FN_SIGN) return CXM_E_INVALID;
    if (n == 0) return CXM_OK;
    switch (fn) {
        case CXM_FN_SQUARE: return map(FSquare{}, x, z, n, s);
        case CXM_FN_SQRT: return map(FSqrt{}, x, z, n, s);
        case CXM_FN_RSQRT: return map(FRsqrt{}, x, z, n, s);
        case CXM_FN_LOG: return map(FLog{}, x, z, n, s);
        case CXM_FN_EXP: return map(FExp{}, x, z, n, s);
        case CXM_FN_ERF: return map(FErf{}, x, z, n, s);
        case CXM_FN_SIN: return map(FSin{}, x, z, n, s);
        case CXM_FN_COS: return map(FCos{}, x, z, n, s);
        case CXM_FN_ABS: return map(FAbs{}, x, z, n, s);
        case CXM_FN_NEG: return map(FNeg{}, x, z, n, s);
        case CXM_FN_RCP:
        case CXM_FN_INVERSE: return map(FRcp{}, x, z, n, s);
        default: return map(FSign{}, x, z, n, s);
    }
}

int cxm_lerp_f32(const float *x, float v1, float v2, float *z, size_t n, cxm_stream_t s) {
    if (!x || !z) return CXM_E_INVALID;
    if (n == 0) return CXM_OK;
    return map(FLerp{v1, v2}, x, z, n, s);
}

int cxm_clamp_f32(const float *x, float lo, float hi, float *z, size_t n, cxm_stream_t s) {
    if (!x || !z) return CXM_E_INVALID;
    if (n == 0) return CXM_OK;
    return map(FClamp{lo, hi}, x, z, n, s);
}

int cxm_gather_f32(const float *x, size_t x_n, const int32_t *idx, float *z, size_t n,
                   cxm_stream_t s) {
    if (!x || !idx || !z) return CXM_E_INVALID;
    if (n == 0) return CXM_OK;
    hipLaunchKernelGGL(k_gather<float>, dim3(map_grid(n)), dim3(kBlock), 0, hs(s), x, x_n, idx, z, n,
                       __builtin_nanf(""));
    return launch_status();
}

int cxm_gather_i32(const int32_t *x, size_t x_n, const int32_t *idx, int32_t *z, size_t n,
                   cxm_stream_t s) {
    if (!x || !idx || !z) return CXM_E_INVALID;
    if (n == 0) return CXM_OK;
    hipLaunchKernelGGL(k_gather<int32_t>, dim3(map_grid(n)), dim3(kBlock), 0, hs(s), x, x_n, idx, z, n,
                       INT32_MIN);
    return launch_status();
}

}  // extern "C"
