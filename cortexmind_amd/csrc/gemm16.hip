// bf16 / fp16 GEMM on the CDNA4 matrix cores (v_mfma_f32_32x32x16_bf16 /
// _f16): 16-bit operands, fp32 accumulation, one rounding to the 16-bit
// output type.
//
// Replaces the 16-bit branches of nv::Matrix::matmul
// (source/CortexMind/framework/Engine/CUDA/matrix.cu:112-159, cublasGemmEx
// with the per-dtype BlasTraits of matrix.cu:18-37: bf16 computes in fp32,
// fp16 in fp16).  Here both accumulate in fp32, so the fp16 form is the more
// accurate of the two; results differ from the exact product of the 16-bit
// inputs by the fp32 accumulation error plus the final rounding.
//
// Tiling: a 256-thread workgroup (four waves, one per SIMD) computes a
// 128x128 tile of C; each wave owns 64x64 = 2x2 MFMA tiles of 32x32
// (64 accumulator registers per lane).  K advances in steps of 64 through
// double-buffered LDS tiles stored with k contiguous (As[m][k], Bs[n][k],
// row stride 72 elements = 144 bytes), so one ds_read_b128 is one MFMA
// operand: lane l supplies A[l%32][8*(l/32) .. +7] and B[8*(l/32) .. +7][l%32]
// of a 32x32x16 block; accumulator register r of lane l holds
// C[8*(r/4) + 4*(l/32) + r%4][l%32].
//
// Staging through registers:
//  * operand stored with k contiguous (A [m,k], or B^T stored [n,k]): one
//    128-bit load of 8 k and one 128-bit LDS write per chunk;
//  * operand stored with the tile row contiguous (B [k,n], or A^T stored
//    [k,m]): a thread loads an 8-row x 4-k block (four 128-bit loads, one
//    per k), transposes it in registers (16 byte permutes) and writes eight
//    64-bit LDS rows.
// The next k step's tiles, loaded into registers at the top of the step,
// are written to the other LDS buffer three quarters of the way through the
// step's MFMAs, so one barrier separates two steps.
#include "cxm_common.hpp"
#include "half.hpp"

namespace cxm {
namespace {

constexpr int kH_BM = 128, kH_BN = 128, kH_BK = 64;
constexpr int kH_KP = kH_BK + 8;  // LDS row stride in 16-bit elements
constexpr int kHThreads = 256;

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

template <int DT>
__device__ __forceinline__ f32x16 mfma16(u32x4 a, u32x4 b, f32x16 c) {
    if constexpr (DT == CXM_DT_BF16)
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                       0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                      0, 0);
}

__device__ __forceinline__ unsigned xcd_remap16(unsigned b, unsigned g) {
    if (g % 8 != 0) return b;
    return (b % 8) * (g / 8) + b / 8;
}

// Eight 16-bit elements at p[0..7] with p[i] valid for i < n (the rest 0).
__device__ __forceinline__ u32x4 ld8_part(const uint16_t *p, size_t n) {
    u32x4 v = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const unsigned e = static_cast<size_t>(i) < n ? p[i] : 0u;
        v[i / 2] |= (i & 1) ? (e << 16) : e;
    }
    return v;
}

// One operand tile: 128 tile rows (m or n) x 64 k, into Xs[row][k].
//  KC: stored X[R][Kd] (k contiguous); 4 chunks of 8 k per thread.
//  !KC: stored X[Kd][R] (rows contiguous); one 8-row x 4-k block per thread.
template <bool KC>
struct Stage16 {
    static constexpr int kRegs = 4;  // u32x4 registers held between load and store
    int r, k;
    __device__ __forceinline__ void init(int tid) {
        if constexpr (KC) {
            r = tid / 8;  // chunk s adds 32 rows
            k = (tid % 8) * 8;
        } else {
            r = (tid % 16) * 8;
            k = (tid / 16) * 4;
        }
    }
    template <bool V>
    __device__ __forceinline__ void load(const uint16_t *__restrict__ X, size_t r0, size_t k0, size_t R, size_t Kd,
                                         u32x4 (&v)[kRegs]) const {
        const u32x4 zero = {0u, 0u, 0u, 0u};
        if constexpr (KC) {
#pragma unroll
            for (int s = 0; s < kRegs; ++s) {
                const size_t rg = r0 + r + 32 * s, kg = k0 + k;
                if (rg >= R || kg >= Kd) {
                    v[s] = zero;
                } else {
                    const uint16_t *p = X + rg * Kd + kg;
                    v[s] = V ? *reinterpret_cast<const u32x4 *>(p) : ld8_part(p, Kd - kg);
                }
            }
        } else {
#pragma unroll
            for (int s = 0; s < kRegs; ++s) {
                const size_t rg = r0 + r, kg = k0 + k + s;
                if (rg >= R || kg >= Kd) {
                    v[s] = zero;
                } else {
                    const uint16_t *p = X + kg * R + rg;
                    v[s] = V ? *reinterpret_cast<const u32x4 *>(p) : ld8_part(p, R - rg);
                }
            }
        }
    }
    __device__ __forceinline__ void store(uint16_t (*Xs)[kH_KP], const u32x4 (&v)[kRegs]) const {
        if constexpr (KC) {
#pragma unroll
            for (int s = 0; s < kRegs; ++s) *reinterpret_cast<u32x4 *>(&Xs[r + 32 * s][k]) = v[s];
        } else {
            // v[s] holds rows r..r+7 at k + s; row r+2w+h takes half h of
            // word w of each v[s]
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const u32x2 lo = {(v[0][w] & 0xffffu) | (v[1][w] << 16), (v[2][w] & 0xffffu) | (v[3][w] << 16)};
                const u32x2 hi = {(v[0][w] >> 16) | (v[1][w] & 0xffff0000u), (v[2][w] >> 16) | (v[3][w] & 0xffff0000u)};
                *reinterpret_cast<u32x2 *>(&Xs[r + 2 * w][k]) = lo;
                *reinterpret_cast<u32x2 *>(&Xs[r + 2 * w + 1][k]) = hi;
            }
        }
    }
};

template <int DT, bool TA, bool TB, bool VA, bool VB>
__global__ __launch_bounds__(kHThreads) void k_gemm16(const uint16_t *__restrict__ A, const uint16_t *__restrict__ B,
                                                      uint16_t *__restrict__ C, size_t M, size_t N, size_t K,
                                                      unsigned tiles_n) {
    constexpr int NB = kH_BK / 16;  // MFMA k blocks per step
    constexpr int WAT = 3;          // LDS writes after this many blocks
    constexpr int WI = 2, WJ = 2;
    __shared__ uint16_t As[2][kH_BM][kH_KP];
    __shared__ uint16_t Bs[2][kH_BN][kH_KP];
    constexpr bool KCA = !TA, KCB = TB;

    const unsigned wg = xcd_remap16(blockIdx.x, gridDim.x);
    const size_t m0 = static_cast<size_t>(wg / tiles_n) * kH_BM;
    const size_t n0 = static_cast<size_t>(wg % tiles_n) * kH_BN;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int wm = wave >> 1, wn = wave & 1;
    const int l32 = lane & 31, lhi = lane >> 5;

    f32x16 acc[WI][WJ];
#pragma unroll
    for (int i = 0; i < WI; ++i)
#pragma unroll
        for (int j = 0; j < WJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    Stage16<KCA> sa;
    Stage16<KCB> sb;
    sa.init(tid);
    sb.init(tid);
    u32x4 ra[4], rb[4];
    sa.template load<VA>(A, m0, 0, M, K, ra);
    sb.template load<VB>(B, n0, 0, N, K, rb);
    sa.store(As[0], ra);
    sb.store(Bs[0], rb);
    __syncthreads();

    int buf = 0;
    for (size_t k0 = 0; k0 < K; k0 += kH_BK) {
        const bool more = k0 + kH_BK < K;
        if (more) {
            sa.template load<VA>(A, m0, k0 + kH_BK, M, K, ra);
            sb.template load<VB>(B, n0, k0 + kH_BK, N, K, rb);
        }
        u32x4 fa[WI], fb[WJ];
#pragma unroll
        for (int i = 0; i < WI; ++i) fa[i] = *reinterpret_cast<const u32x4 *>(&As[buf][wm * 64 + i * 32 + l32][8 * lhi]);
#pragma unroll
        for (int j = 0; j < WJ; ++j) fb[j] = *reinterpret_cast<const u32x4 *>(&Bs[buf][wn * 64 + j * 32 + l32][8 * lhi]);
#pragma unroll
        for (int kb = 0; kb < NB; ++kb) {
            u32x4 na[WI], nb[WJ];
            if (kb + 1 < NB) {
#pragma unroll
                for (int i = 0; i < WI; ++i)
                    na[i] = *reinterpret_cast<const u32x4 *>(&As[buf][wm * 64 + i * 32 + l32][16 * (kb + 1) + 8 * lhi]);
#pragma unroll
                for (int j = 0; j < WJ; ++j)
                    nb[j] = *reinterpret_cast<const u32x4 *>(&Bs[buf][wn * 64 + j * 32 + l32][16 * (kb + 1) + 8 * lhi]);
            }
#pragma unroll
            for (int i = 0; i < WI; ++i)
#pragma unroll
                for (int j = 0; j < WJ; ++j) acc[i][j] = mfma16<DT>(fa[i], fb[j], acc[i][j]);
            if (kb + 1 == WAT && more) {
                // the other buffer was last read before the previous barrier
                sa.store(As[buf ^ 1], ra);
                sb.store(Bs[buf ^ 1], rb);
            }
            if (kb + 1 < NB) {
#pragma unroll
                for (int i = 0; i < WI; ++i) fa[i] = na[i];
#pragma unroll
                for (int j = 0; j < WJ; ++j) fb[j] = nb[j];
            }
        }
        __syncthreads();
        buf ^= 1;
    }

    // C tile: register r of lane l -> row 8*(r/4) + 4*lhi + r%4, column l32;
    // lanes 0-31 of one register write 64 contiguous bytes of a row.
#pragma unroll
    for (int i = 0; i < WI; ++i)
#pragma unroll
        for (int j = 0; j < WJ; ++j) {
            const size_t col = n0 + wn * 64 + j * 32 + l32;
            if (col >= N) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const size_t row = m0 + wm * 64 + i * 32 + 8 * (r / 4) + 4 * lhi + (r % 4);
                if (row < M) C[row * N + col] = H<DT>::store(acc[i][j][r]);
            }
        }
}

inline hipStream_t hs(cxm_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

template <int DT, bool TA, bool TB>
int launch16(const uint16_t *A, const uint16_t *B, uint16_t *C, size_t M, size_t N, size_t K, bool va, bool vb,
             dim3 grid, unsigned tn, hipStream_t s) {
    if (va && vb) hipLaunchKernelGGL((k_gemm16<DT, TA, TB, true, true>), grid, dim3(kHThreads), 0, s, A, B, C, M, N, K, tn);
    else if (va) hipLaunchKernelGGL((k_gemm16<DT, TA, TB, true, false>), grid, dim3(kHThreads), 0, s, A, B, C, M, N, K, tn);
    else if (vb) hipLaunchKernelGGL((k_gemm16<DT, TA, TB, false, true>), grid, dim3(kHThreads), 0, s, A, B, C, M, N, K, tn);
    else hipLaunchKernelGGL((k_gemm16<DT, TA, TB, false, false>), grid, dim3(kHThreads), 0, s, A, B, C, M, N, K, tn);
    return launch_status();
}

template <int DT>
int gemm16(const uint16_t *A, const uint16_t *B, uint16_t *C, size_t M, size_t K, size_t N, bool ta, bool tb,
           cxm_stream_t st) {
    const size_t tiles_m = (M + kH_BM - 1) / kH_BM, tiles_n = (N + kH_BN - 1) / kH_BN;
    if (tiles_m * tiles_n > 0x7fffffffu) return CXM_E_TOO_LARGE;
    // 128-bit loads need 16-byte aligned bases and stored rows of a multiple of 8
    const bool va = aligned16(A) && (ta ? M % 8 == 0 : K % 8 == 0);
    const bool vb = aligned16(B) && (tb ? K % 8 == 0 : N % 8 == 0);
    const dim3 grid(static_cast<unsigned>(tiles_m * tiles_n));
    const unsigned tn = static_cast<unsigned>(tiles_n);
    hipStream_t s = hs(st);
    if (!ta && !tb) return launch16<DT, false, false>(A, B, C, M, N, K, va, vb, grid, tn, s);
    if (ta && !tb) return launch16<DT, true, false>(A, B, C, M, N, K, va, vb, grid, tn, s);
    if (!ta && tb) return launch16<DT, false, true>(A, B, C, M, N, K, va, vb, grid, tn, s);
    return launch16<DT, true, true>(A, B, C, M, N, K, va, vb, grid, tn, s);
}

}  // namespace
}  // namespace cxm

extern "C" {

int cxm_gemm_t(const void *a, const void *b, void *c, size_t m, size_t k, size_t n, int trans_a, int trans_b,
               int dtype, cxm_stream_t s) {
    if (!a || !b || !c) return CXM_E_INVALID;
    if (dtype == CXM_DT_F32)
        return cxm_gemm_f32(static_cast<const float *>(a), static_cast<const float *>(b), static_cast<float *>(c), m,
                            k, n, trans_a, trans_b, nullptr, CXM_ACT_NONE, nullptr, s);
    if (dtype != CXM_DT_BF16 && dtype != CXM_DT_F16) return CXM_E_INVALID;
    if (m == 0 || n == 0) return CXM_OK;
    if (k == 0) return CXM_E_INVALID;
    const auto *A = static_cast<const uint16_t *>(a);
    const auto *B = static_cast<const uint16_t *>(b);
    auto *C = static_cast<uint16_t *>(c);
    if (dtype == CXM_DT_BF16) return cxm::gemm16<CXM_DT_BF16>(A, B, C, m, k, n, trans_a != 0, trans_b != 0, s);
    return cxm::gemm16<CXM_DT_F16>(A, B, C, m, k, n, trans_a != 0, trans_b != 0, s);
}

int cxm_matmul_t(const void *a, const void *b, void *c, size_t xN, size_t yN, size_t zN, int dtype,
                 cxm_stream_t s) {
    return cxm_gemm_t(a, b, c, xN, yN, zN, 0, 0, dtype, s);
}

}  // extern "C"
