// bf16 / fp16 element conversions shared by the 16-bit kernels.
//
// bf16 -> f32 is a 16-bit shift; f32 -> bf16 rounds to nearest-even by
// adding 0x7FFF + lsb, as the reference's SIMD body
// (source/CortexMind/framework/Tools/cast.cpp:55-68), except that NaN stays
// a quiet NaN (the reference's formula turns a NaN with a small payload
// into infinity); f16 <-> f32 is the IEEE conversion (v_cvt_f16_f32 /
// v_cvt_f32_f16, round to nearest-even), as _mm256_cvtps_ph /
// _mm256_cvtph_ps.
#pragma once

#include "cxm_common.hpp"

namespace cxm {
namespace {

template <int DT>
struct H;
template <>
struct H<CXM_DT_BF16> {
    __device__ static float load(uint16_t h) { return __builtin_bit_cast(float, static_cast<uint32_t>(h) << 16); }
    __device__ static uint16_t store(float f) {
        uint32_t u = __builtin_bit_cast(uint32_t, f);
        if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
        u += 0x7fffu + ((u >> 16) & 1u);
        return static_cast<uint16_t>(u >> 16);
    }
};
template <>
struct H<CXM_DT_F16> {
    __device__ static float load(uint16_t h) { return static_cast<float>(__builtin_bit_cast(_Float16, h)); }
    __device__ static uint16_t store(float f) { return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f)); }
};

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

}  // namespace
}  // namespace cxm
