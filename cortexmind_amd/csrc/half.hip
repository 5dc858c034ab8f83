// bf16 / fp16 forms of the elementwise surface, and the dtype conversions.
//
// Replaces the 16-bit paths of the reference: the CPU engine converts to
// fp32, computes in fp32 and converts back (avx2::wise kernel_t,
// source/CortexMind/framework/Engine/AVX2/wise.cpp:17-52, with convert()
// of Tools/cast.cpp:7-90); the CUDA kernels take __nv_bfloat162 / __half2
// pairs (Engine/Kernels/unary.cuh:42-90, binary.cuh:41-89, scalar.cuh:
// 69-130).  Here every 16-bit element is widened to fp32 exactly, the fp32
// operator of ops.hpp is applied, and the result is rounded to nearest-even
// once.  For + - * / and sqrt that equals the correctly rounded 16-bit
// result (fp32 carries more than twice the 16-bit precision plus two bits);
// scalar operands are first rounded to the 16-bit type, as the CUDA path
// passes them.
//
// Conversions (cast.cpp:7-90): see half.hpp.
//
// Vector path: 16-byte aligned pointers, eight 16-bit elements (one
// 128-bit load) per thread, one 256-thread workgroup per 2048 elements,
// non-temporal loads and stores; otherwise a scalar grid-stride loop.
#include <cstring>

#include "cxm_common.hpp"
#include "half.hpp"
#include "ops.hpp"

namespace cxm {
namespace {

__device__ __forceinline__ u32x4 ld16(const uint16_t *p) { return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p)); }
__device__ __forceinline__ void st16(uint16_t *p, u32x4 v) { __builtin_nontemporal_store(v, reinterpret_cast<u32x4 *>(p)); }

template <int DT>
__device__ __forceinline__ void unpack8(u32x4 v, float (&f)[8]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        f[2 * k] = H<DT>::load(static_cast<uint16_t>(v[k] & 0xffffu));
        f[2 * k + 1] = H<DT>::load(static_cast<uint16_t>(v[k] >> 16));
    }
}
template <int DT>
__device__ __forceinline__ u32x4 pack8(const float (&f)[8]) {
    u32x4 v;
#pragma unroll
    for (int k = 0; k < 4; ++k)
        v[k] = static_cast<unsigned>(H<DT>::store(f[2 * k])) | (static_cast<unsigned>(H<DT>::store(f[2 * k + 1])) << 16);
    return v;
}

template <int DT, class F>
__global__ __launch_bounds__(kBlock) void k_map8(F f, const uint16_t *x, uint16_t *z, size_t n) {
    const size_t i = stream_vec();
    const size_t n8 = n / 8;
    if (i < n8) {
        float v[8];
        unpack8<DT>(ld16(x + 8 * i), v);
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = f(v[k]);
        st16(z + 8 * i, pack8<DT>(v));
    } else if (i == n8) {
        for (size_t j = 8 * n8; j < n; ++j) z[j] = H<DT>::store(f(H<DT>::load(x[j])));
    }
}

template <int DT, class F>
__global__ __launch_bounds__(kBlock) void k_zip8(F f, const uint16_t *x, const uint16_t *y, uint16_t *z, size_t n) {
    const size_t i = stream_vec();
    const size_t n8 = n / 8;
    if (i < n8) {
        float a[8], b[8];
        unpack8<DT>(ld16(x + 8 * i), a);
        unpack8<DT>(ld16(y + 8 * i), b);
#pragma unroll
        for (int k = 0; k < 8; ++k) a[k] = f(a[k], b[k]);
        st16(z + 8 * i, pack8<DT>(a));
    } else if (i == n8) {
        for (size_t j = 8 * n8; j < n; ++j) z[j] = H<DT>::store(f(H<DT>::load(x[j]), H<DT>::load(y[j])));
    }
}

template <int DT, class F>
__global__ __launch_bounds__(kBlock) void k_map16_any(F f, const uint16_t *x, uint16_t *z, size_t n) {
    const size_t stride = static_cast<size_t>(gridDim.x) * kBlock;
    for (size_t i = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride)
        z[i] = H<DT>::store(f(H<DT>::load(x[i])));
}

template <int DT, class F>
__global__ __launch_bounds__(kBlock) void k_zip16_any(F f, const uint16_t *x, const uint16_t *y, uint16_t *z,
                                                      size_t n) {
    const size_t stride = static_cast<size_t>(gridDim.x) * kBlock;
    for (size_t i = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride)
        z[i] = H<DT>::store(f(H<DT>::load(x[i]), H<DT>::load(y[i])));
}

// f32 -> 16-bit and 16-bit -> f32, eight elements per thread.
template <int DT>
__global__ __launch_bounds__(kBlock) void k_to16(const float *x, uint16_t *z, size_t n) {
    const size_t i = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;
    const size_t n8 = n / 8;
    if (i < n8) {
        const float4 a = ld4_stream(x + 8 * i), b = ld4_stream(x + 8 * i + 4);
        const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        st16(z + 8 * i, pack8<DT>(v));
    } else if (i == n8) {
        for (size_t j = 8 * n8; j < n; ++j) z[j] = H<DT>::store(x[j]);
    }
}
template <int DT>
__global__ __launch_bounds__(kBlock) void k_from16(const uint16_t *x, float *z, size_t n) {
    const size_t i = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;
    const size_t n8 = n / 8;
    if (i < n8) {
        float v[8];
        unpack8<DT>(ld16(x + 8 * i), v);
        st4_stream(z + 8 * i, make_float4(v[0], v[1], v[2], v[3]));
        st4_stream(z + 8 * i + 4, make_float4(v[4], v[5], v[6], v[7]));
    } else if (i == n8) {
        for (size_t j = 8 * n8; j < n; ++j) z[j] = H<DT>::load(x[j]);
    }
}
template <int SDT, int DDT>
__global__ __launch_bounds__(kBlock) void k_conv_any(const void *x, void *z, size_t n) {
    const size_t stride = static_cast<size_t>(gridDim.x) * kBlock;
    for (size_t i = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
        float v;
        if constexpr (SDT == CXM_DT_F32) v = static_cast<const float *>(x)[i];
        else v = H<SDT>::load(static_cast<const uint16_t *>(x)[i]);
        if constexpr (DDT == CXM_DT_F32) static_cast<float *>(z)[i] = v;
        else static_cast<uint16_t *>(z)[i] = H<DDT>::store(v);
    }
}

inline hipStream_t hs(cxm_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// k_map8 / k_zip8 over n 16-bit elements: 8 per thread, the streaming
// maps' layout (stream_vec)
inline unsigned grid8(size_t n) { return stream_grid_for(n / 8); }
inline unsigned grid_any(size_t n) {
    size_t b = (n + kBlock - 1) / kBlock;
    const size_t cap = 256 * 16;
    return static_cast<unsigned>(b < 1 ? 1 : (b > cap ? cap : b));
}

template <int DT, class F>
int map16(F f, const void *x, void *z, size_t n, cxm_stream_t s) {
    const auto *xs = static_cast<const uint16_t *>(x);
    auto *zs = static_cast<uint16_t *>(z);
    if (aligned16(x) && aligned16(z)) {
        const unsigned g = grid8(n);
        if (!g) return CXM_E_TOO_LARGE;
        hipLaunchKernelGGL((k_map8<DT, F>), dim3(g), dim3(kBlock), 0, hs(s), f, xs, zs, n);
    } else {
        hipLaunchKernelGGL((k_map16_any<DT, F>), dim3(grid_any(n)), dim3(kBlock), 0, hs(s), f, xs, zs, n);
    }
    return launch_status();
}

template <int DT, class F>
int zip16(F f, const void *x, const void *y, void *z, size_t n, cxm_stream_t s) {
    const auto *xs = static_cast<const uint16_t *>(x);
    const auto *ys = static_cast<const uint16_t *>(y);
    auto *zs = static_cast<uint16_t *>(z);
    if (aligned16(x) && aligned16(y) && aligned16(z)) {
        const unsigned g = grid8(n);
        if (!g) return CXM_E_TOO_LARGE;
        hipLaunchKernelGGL((k_zip8<DT, F>), dim3(g), dim3(kBlock), 0, hs(s), f, xs, ys, zs, n);
    } else {
        hipLaunchKernelGGL((k_zip16_any<DT, F>), dim3(grid_any(n)), dim3(kBlock), 0, hs(s), f, xs, ys, zs, n);
    }
    return launch_status();
}

template <int OP>
struct Bin16 {
    __device__ float operator()(float a, float b) const { return bin_t<OP>(a, b); }
};
template <int OP>
struct Scal16 {
    float v;
    __device__ float operator()(float a) const { return bin_t<OP>(a, v); }
};
template <int ACT>
struct Act16 {
    __device__ float operator()(float t) const { return act<ACT>(t); }
};

// The host-side rounding of a scalar operand to the 16-bit type (the same
// rounding as H<DT>::store).
float round16(float v, int dt) {
    uint32_t u;
    std::memcpy(&u, &v, 4);
    if (dt == CXM_DT_BF16) {
        if ((u & 0x7fffffffu) > 0x7f800000u) return v;
        u += 0x7fffu + ((u >> 16) & 1u);
        u &= 0xffff0000u;
        float r;
        std::memcpy(&r, &u, 4);
        return r;
    }
    return static_cast<float>(static_cast<_Float16>(v));
}

template <int DT>
int binary16(const void *x, const void *y, void *z, size_t n, int op, cxm_stream_t s) {
    switch (op) {
        case CXM_OP_ADD: return zip16<DT>(Bin16<CXM_OP_ADD>{}, x, y, z, n, s);
        case CXM_OP_SUB: return zip16<DT>(Bin16<CXM_OP_SUB>{}, x, y, z, n, s);
        case CXM_OP_MUL: return zip16<DT>(Bin16<CXM_OP_MUL>{}, x, y, z, n, s);
        case CXM_OP_DIV: return zip16<DT>(Bin16<CXM_OP_DIV>{}, x, y, z, n, s);
        case CXM_OP_MAX: return zip16<DT>(Bin16<CXM_OP_MAX>{}, x, y, z, n, s);
        case CXM_OP_MIN: return zip16<DT>(Bin16<CXM_OP_MIN>{}, x, y, z, n, s);
        default: return zip16<DT>(Bin16<CXM_OP_POW>{}, x, y, z, n, s);
    }
}

template <int DT>
int scalar16(const void *x, float v, void *z, size_t n, int op, cxm_stream_t s) {
    switch (op) {
        case CXM_OP_ADD: return map16<DT>(Scal16<CXM_OP_ADD>{v}, x, z, n, s);
        case CXM_OP_SUB: return map16<DT>(Scal16<CXM_OP_SUB>{v}, x, z, n, s);
        case CXM_OP_MUL: return map16<DT>(Scal16<CXM_OP_MUL>{v}, x, z, n, s);
        case CXM_OP_DIV: return map16<DT>(Scal16<CXM_OP_DIV>{v}, x, z, n, s);
        case CXM_OP_MAX: return map16<DT>(Scal16<CXM_OP_MAX>{v}, x, z, n, s);
        case CXM_OP_MIN: return map16<DT>(Scal16<CXM_OP_MIN>{v}, x, z, n, s);
        default: return map16<DT>(Scal16<CXM_OP_POW>{v}, x, z, n, s);
    }
}

template <int DT>
int unary16(const void *x, void *z, size_t n, int act_code, cxm_stream_t s) {
    switch (act_code) {
        case CXM_ACT_RELU: return map16<DT>(Act16<CXM_ACT_RELU>{}, x, z, n, s);
        case CXM_ACT_SIGMOID: return map16<DT>(Act16<CXM_ACT_SIGMOID>{}, x, z, n, s);
        case CXM_ACT_TANH: return map16<DT>(Act16<CXM_ACT_TANH>{}, x, z, n, s);
        default: return map16<DT>(Act16<CXM_ACT_EXP>{}, x, z, n, s);
    }
}

template <int DT>
int wise16(const void *x, void *z, size_t n, int fn, cxm_stream_t s) {
    switch (fn) {
        case CXM_FN_SQUARE: return map16<DT>(FSquare{}, x, z, n, s);
        case CXM_FN_SQRT: return map16<DT>(FSqrt{}, x, z, n, s);
        case CXM_FN_RSQRT: return map16<DT>(FRsqrt{}, x, z, n, s);
        case CXM_FN_LOG: return map16<DT>(FLog{}, x, z, n, s);
        case CXM_FN_EXP: return map16<DT>(FExp{}, x, z, n, s);
        case CXM_FN_ERF: return map16<DT>(FErf{}, x, z, n, s);
        case CXM_FN_SIN: return map16<DT>(FSin{}, x, z, n, s);
        case CXM_FN_COS: return map16<DT>(FCos{}, x, z, n, s);
        case CXM_FN_ABS: return map16<DT>(FAbs{}, x, z, n, s);
        case CXM_FN_NEG: return map16<DT>(FNeg{}, x, z, n, s);
        case CXM_FN_RCP:
        case CXM_FN_INVERSE: return map16<DT>(FRcp{}, x, z, n, s);
        default: return map16<DT>(FSign{}, x, z, n, s);
    }
}

bool dt_ok(int dt) { return dt == CXM_DT_F32 || dt == CXM_DT_BF16 || dt == CXM_DT_F16; }

}  // namespace
}  // namespace cxm

using namespace cxm;

extern "C" {

int cxm_convert(void *dst, int dst_dtype, const void *src, int src_dtype, size_t n, cxm_stream_t s) {
    if (!dst || !src || !dt_ok(dst_dtype) || !dt_ok(src_dtype)) return CXM_E_INVALID;
    if (n == 0) return CXM_OK;
    if (dst_dtype == src_dtype) {
        const size_t w = dst_dtype == CXM_DT_F32 ? 4 : 2;
        return cxm_memcpy_d2d(dst, src, n * w, s);
    }
    const bool al = aligned16(dst) && aligned16(src);
    const unsigned g8 = grid8(n);
    if (al && g8 && src_dtype == CXM_DT_F32) {
        if (dst_dtype == CXM_DT_BF16)
            hipLaunchKernelGGL(k_to16<CXM_DT_BF16>, dim3(g8), dim3(kBlock), 0, hs(s), static_cast<const float *>(src),
                               static_cast<uint16_t *>(dst), n);
        else
            hipLaunchKernelGGL(k_to16<CXM_DT_F16>, dim3(g8), dim3(kBlock), 0, hs(s), static_cast<const float *>(src),
                               static_cast<uint16_t *>(dst), n);
        return launch_status();
    }
    if (al && g8 && dst_dtype == CXM_DT_F32) {
        if (src_dtype == CXM_DT_BF16)
            hipLaunchKernelGGL(k_from16<CXM_DT_BF16>, dim3(g8), dim3(kBlock), 0, hs(s),
                               static_cast<const uint16_t *>(src), static_cast<float *>(dst), n);
        else
            hipLaunchKernelGGL(k_from16<CXM_DT_F16>, dim3(g8), dim3(kBlock), 0, hs(s),
                               static_cast<const uint16_t *>(src), static_cast<float *>(dst), n);
        return launch_status();
    }
    const dim3 g(grid_any(n));
#define CXM_CONV(S, D) \
    if (src_dtype == S && dst_dtype == D) hipLaunchKernelGGL((k_conv_any<S, D>), g, dim3(kBlock), 0, hs(s), src, dst, n)
    CXM_CONV(CXM_DT_F32, CXM_DT_BF16);
    CXM_CONV(CXM_DT_F32, CXM_DT_F16);
    CXM_CONV(CXM_DT_BF16, CXM_DT_F32);
    CXM_CONV(CXM_DT_F16, CXM_DT_F32);
    CXM_CONV(CXM_DT_BF16, CXM_DT_F16);
    CXM_CONV(CXM_DT_F16, CXM_DT_BF16);
#undef CXM_CONV
    return launch_status();
}

int cxm_binary_t(const void *x, const void *y, void *z, size_t n, int op, int dtype, cxm_stream_t s) {
    if (dtype == CXM_DT_F32)
        return cxm_binary_f32(static_cast<const float *>(x), static_cast<const float *>(y), static_cast<float *>(z), n,
                              op, s);
    if (!x || !y || !z || op < CXM_OP_ADD || op > CXM_OP_POW || !dt_ok(dtype)) return CXM_E_INVALID;
    if (n == 0) return CXM_OK;
    return dtype == CXM_DT_BF16 ? binary16<CXM_DT_BF16>(x, y, z, n, op, s) : binary16<CXM_DT_F16>(x, y, z, n, op, s);
}

int cxm_scalar_t(const void *x, float value, void *z, size_t n, int op, int dtype, cxm_stream_t s) {
    if (dtype == CXM_DT_F32)
        return cxm_scalar_f32(static_cast<const float *>(x), value, static_cast<float *>(z), n, op, s);
    if (!x || !z || op < CXM_OP_ADD || op > CXM_OP_POW || !dt_ok(dtype)) return CXM_E_INVALID;
    if (n == 0) return CXM_OK;
    const float v = round16(value, dtype);
    return dtype == CXM_DT_BF16 ? scalar16<CXM_DT_BF16>(x, v, z, n, op, s) : scalar16<CXM_DT_F16>(x, v, z, n, op, s);
}

int cxm_unary_t(const void *x, void *z, size_t n, int act, int dtype, cxm_stream_t s) {
    if (dtype == CXM_DT_F32) return cxm_unary_f32(static_cast<const float *>(x), static_cast<float *>(z), n, act, s);
    if (!x || !z || act < CXM_ACT_RELU || act > CXM_ACT_EXP || !dt_ok(dtype)) return CXM_E_INVALID;
    if (n == 0) return CXM_OK;
    return dtype == CXM_DT_BF16 ? unary16<CXM_DT_BF16>(x, z, n, act, s) : unary16<CXM_DT_F16>(x, z, n, act, s);
}

int cxm_wise_t(const void *x, void *z, size_t n, int fn, int dtype, cxm_stream_t s) {
    if (dtype == CXM_DT_F32) return cxm_wise_f32(static_cast<const float *>(x), static_cast<float *>(z), n, fn, s);
    if (!x || !z || fn < CXM_FN_SQUARE || fn > CXM_FN_SIGN || !dt_ok(dtype)) return CXM_E_INVALID;
    if (n == 0) return CXM_OK;
    return dtype == CXM_DT_BF16 ? wise16<CXM_DT_BF16>(x, z, n, fn, s) : wise16<CXM_DT_F16>(x, z, n, fn, s);
}

}  // extern "C"
