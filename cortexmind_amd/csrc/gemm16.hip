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
// Four kernels, chosen by shape (gemm16() below), all accumulating each
// output over k in the same order (32x32x16 blocks in k order), so they
// give the same bits:
//  * k_gemm16_ring<TM = 256 or 128>: TMxTM tiles, four LDS stages filled by
//    direct global-to-LDS loads, for M, N multiples of TM and K of 128; B
//    is read as stored ([K,N] through the LDS transpose reads of gfx950,
//    or B^T [N,K]), A stored [K,M] is transposed into the workspace first;
//  * k_gemm16_big: 256x256 tiles with register staging, any shape;
//  * k_gemm16: 128x128 tiles with register staging, any shape.
// MFMA operand layout (32x32x16): lane l supplies A[l%32][8*(l/32) .. +7]
// and B[8*(l/32) .. +7][l%32]; accumulator register r of lane l holds
// C[8*(r/4) + 4*(l/32) + r%4][l%32].
//
// k_gemm16: a 256-thread workgroup (four waves, one per SIMD) computes a
// 128x128 tile of C; each wave owns 64x64 = 2x2 MFMA tiles of 32x32
// (64 accumulator registers per lane).  K advances in steps of 64 through
// double-buffered LDS tiles stored with k contiguous (As[m][k], Bs[n][k],
// row stride 72 elements = 144 bytes), so one ds_read_b128 is one MFMA
// operand.
//
// Staging through registers (k_gemm16, k_gemm16_big):
//  * operand stored with k contiguous (A [m,k], or B^T stored [n,k]): one
//    128-bit load of 8 k and one 128-bit LDS write per chunk;
//  * operand stored with the tile row contiguous (B [k,n], or A^T stored
//    [k,m]): a thread loads an 8-row x 4-k block (four 128-bit loads, one
//    per k), transposes it in registers (16 byte permutes) and writes eight
//    64-bit LDS rows.
// The next k step's tiles, loaded into registers at the top of the step,
// are written to the other LDS buffer three quarters of the way through the
// step's MFMAs, so one barrier separates two steps.
#include <atomic>

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

// ------------------------------------------------ 256x256 workgroup tiles
//
// Four waves, each 128x128 of C = 4x4 MFMA tiles of 32x32 (256 fp32
// accumulators per lane, in the accumulation registers), so a k block of 16
// costs 8 fragment reads for 16 MFMAs, half the LDS traffic per MFMA of the
// 64x64 waves above.  BK = 64; the 16-byte k groups of an LDS row are
// XOR-swizzled with the row's 8-row index (group g of row r sits at
// g ^ ((r / 8) % 8)): fragment reads stay single ds_read_b128s, and the
// 64-bit writes of the transposed staging, whose lanes walk along rows,
// spread over the banks instead of all landing on the same 16 bytes.
constexpr int kG_BM = 256, kG_BN = 256, kG_BK = 64, kG_KP = kG_BK + 8;

__device__ __forceinline__ int swz(int r, int g) { return g ^ ((r >> 3) & 7); }

template <bool KC>
struct StageBig {
    static constexpr int kRegs = 8;
    int r, k;  // KC: first row (chunk s adds 32 rows), k group * 8; else: r8 block base row, first k of block 0
    __device__ __forceinline__ void init(int tid) {
        if constexpr (KC) {
            r = tid / 8;
            k = (tid % 8) * 8;
        } else {
            r = (tid % 32) * 8;  // block s: k = 4 * (tid / 32 + 8 * s)
            k = (tid / 32) * 4;
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
            for (int s = 0; s < kRegs; ++s) {  // block s / 4, k row s % 4
                const size_t rg = r0 + r, kg = k0 + k + 32 * (s / 4) + (s % 4);
                if (rg >= R || kg >= Kd) {
                    v[s] = zero;
                } else {
                    const uint16_t *p = X + kg * R + rg;
                    v[s] = V ? *reinterpret_cast<const u32x4 *>(p) : ld8_part(p, R - rg);
                }
            }
        }
    }
    __device__ __forceinline__ void store(uint16_t (*Xs)[kG_KP], const u32x4 (&v)[kRegs]) const {
        if constexpr (KC) {
#pragma unroll
            for (int s = 0; s < kRegs; ++s) {
                const int row = r + 32 * s;
                *reinterpret_cast<u32x4 *>(&Xs[row][8 * swz(row, k / 8)]) = v[s];
            }
        } else {
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const int kk = k + 32 * b;  // 4 k of this block: group kk / 8, half (kk / 4) % 2
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const u32x4 *q = v + 4 * b;
                    const u32x2 lo = {(q[0][w] & 0xffffu) | (q[1][w] << 16), (q[2][w] & 0xffffu) | (q[3][w] << 16)};
                    const u32x2 hi = {(q[0][w] >> 16) | (q[1][w] & 0xffff0000u), (q[2][w] >> 16) | (q[3][w] & 0xffff0000u)};
                    const int r0 = r + 2 * w, r1 = r0 + 1;
                    *reinterpret_cast<u32x2 *>(&Xs[r0][8 * swz(r0, kk / 8) + (kk & 4)]) = lo;
                    *reinterpret_cast<u32x2 *>(&Xs[r1][8 * swz(r1, kk / 8) + (kk & 4)]) = hi;
                }
            }
        }
    }
};

// Loads of one staged tile.  CHECKED: rows and k beyond the matrix read as
// zero (edge tiles, the last partial k step); otherwise every access is in
// range and the loads are unconditional, so the main loop stays one basic
// block that the scheduling barriers below can order.
template <bool KC, bool V, bool CHECKED>
__device__ __forceinline__ void big_load(const StageBig<KC> &st, const uint16_t *__restrict__ X, size_t r0, size_t k0,
                                         size_t R, size_t Kd, u32x4 (&v)[8]) {
    if constexpr (CHECKED) {
        st.template load<V>(X, r0, k0, R, Kd, v);
    } else if constexpr (KC) {
#pragma unroll
        for (int s = 0; s < 8; ++s)
            v[s] = *reinterpret_cast<const u32x4 *>(X + (r0 + st.r + 32 * s) * Kd + k0 + st.k);
    } else {
#pragma unroll
        for (int s = 0; s < 8; ++s)
            v[s] = *reinterpret_cast<const u32x4 *>(X + (k0 + st.k + 32 * (s / 4) + (s % 4)) * R + r0 + st.r);
    }
}

// One k step: MFMAs on LDS buffer `buf` with the next block's fragments
// read during the current block's MFMAs; after block WAT-1 the staged
// registers `st_a/st_b` go to the other buffer.
template <int DT, bool TA, bool TB, int WAT>
__device__ __forceinline__ void big_step(const StageBig<!TA> &sa, const StageBig<TB> &sb, uint16_t (*As)[kG_BM][kG_KP],
                                         uint16_t (*Bs)[kG_BN][kG_KP], int buf, const u32x4 (&st_a)[8],
                                         const u32x4 (&st_b)[8], f32x16 (&acc)[4][4], int wm, int wn, int l32,
                                         int lhi) {
    constexpr int NB = kG_BK / 16;
    constexpr int WI = 4, WJ = 4;
    u32x4 fa[WI], fb[WJ];
#pragma unroll
    for (int i = 0; i < WI; ++i) {
        const int row = wm * 128 + i * 32 + l32;
        fa[i] = *reinterpret_cast<const u32x4 *>(&As[buf][row][8 * swz(row, lhi)]);
    }
#pragma unroll
    for (int j = 0; j < WJ; ++j) {
        const int row = wn * 128 + j * 32 + l32;
        fb[j] = *reinterpret_cast<const u32x4 *>(&Bs[buf][row][8 * swz(row, lhi)]);
    }
#pragma unroll
    for (int kb = 0; kb < NB; ++kb) {
        u32x4 na[WI], nb[WJ];
        if (kb + 1 < NB) {
#pragma unroll
            for (int i = 0; i < WI; ++i) {
                const int row = wm * 128 + i * 32 + l32;
                na[i] = *reinterpret_cast<const u32x4 *>(&As[buf][row][8 * swz(row, 2 * (kb + 1) + lhi)]);
            }
#pragma unroll
            for (int j = 0; j < WJ; ++j) {
                const int row = wn * 128 + j * 32 + l32;
                nb[j] = *reinterpret_cast<const u32x4 *>(&Bs[buf][row][8 * swz(row, 2 * (kb + 1) + lhi)]);
            }
        }
#pragma unroll
        for (int i = 0; i < WI; ++i)
#pragma unroll
            for (int j = 0; j < WJ; ++j) acc[i][j] = mfma16<DT>(fa[i], fb[j], acc[i][j]);
        if (kb + 1 == WAT) {
            // the other buffer was last read before the previous barrier
            sa.store(As[buf ^ 1], st_a);
            sb.store(Bs[buf ^ 1], st_b);
        }
        if (kb + 1 < NB) {
#pragma unroll
            for (int i = 0; i < WI; ++i) fa[i] = na[i];
#pragma unroll
            for (int j = 0; j < WJ; ++j) fb[j] = nb[j];
        }
    }
}

// Scheduling of an unchecked step: the next-but-one tile's global loads
// first, then per k block its MFMAs with the next block's fragment reads
// between them and, after block WAT-1, the LDS stores of the staged tile
// (loaded a whole step earlier, so neither the stores nor the register
// transposes before them wait on memory).
template <bool TB, int WAT>
__device__ __forceinline__ void big_schedule() {
    constexpr int NB = kG_BK / 16;
    constexpr int kWrites = 8 + (TB ? 8 : 16);
    __builtin_amdgcn_sched_group_barrier(0x020, 16, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
    for (int kb = 0; kb < NB; ++kb) {
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
            if (kb + 1 < NB) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        if (kb + 1 == WAT) __builtin_amdgcn_sched_group_barrier(0x200, kWrites, 0);
    }
}

// Interior tiles, K a multiple of 2*BK.  A's next tile loads at the top of
// each step and is stored after block WAT-1 (a plain copy, no arithmetic).
// B's tiles, which are transposed in registers when B is row-contiguous,
// load one step earlier: tile t+1 sits in register set (t % 2) during step t
// while tile t+2 loads into the other set.
template <int DT, bool TA, bool TB, int WAT>
__device__ __forceinline__ void big_loop_fast(const uint16_t *__restrict__ A, const uint16_t *__restrict__ B, size_t M,
                                              size_t N, size_t K, size_t m0, size_t n0, const StageBig<!TA> &sa,
                                              const StageBig<TB> &sb, uint16_t (*As)[kG_BM][kG_KP],
                                              uint16_t (*Bs)[kG_BN][kG_KP], f32x16 (&acc)[4][4], int wm, int wn,
                                              int l32, int lhi) {
    u32x4 ra[8], rb0[8], rb1[8];
    big_load<TB, true, false>(sb, B, n0, kG_BK, N, K, rb0);  // tile 1 (K >= 2*BK here)
    for (size_t k0 = 0; k0 < K; k0 += 2 * kG_BK) {
        {  // even step: tile k0 in buffer 0
            const size_t ka = k0 + kG_BK;  // < K
            const size_t kb2 = k0 + 2 * kG_BK < K ? k0 + 2 * kG_BK : k0;
            big_load<!TA, true, false>(sa, A, m0, ka, M, K, ra);
            big_load<TB, true, false>(sb, B, n0, kb2, N, K, rb1);
            big_step<DT, TA, TB, WAT>(sa, sb, As, Bs, 0, ra, rb0, acc, wm, wn, l32, lhi);
            big_schedule<TB, WAT>();
            __syncthreads();
        }
        {  // odd step: tile k0+BK in buffer 1
            const size_t ka = k0 + 2 * kG_BK < K ? k0 + 2 * kG_BK : k0;
            const size_t kb3 = k0 + 3 * kG_BK < K ? k0 + 3 * kG_BK : k0;
            big_load<!TA, true, false>(sa, A, m0, ka, M, K, ra);
            big_load<TB, true, false>(sb, B, n0, kb3, N, K, rb0);
            big_step<DT, TA, TB, WAT>(sa, sb, As, Bs, 1, ra, rb1, acc, wm, wn, l32, lhi);
            big_schedule<TB, WAT>();
            __syncthreads();
        }
    }
}

// Edge tiles and any K: checked loads, one register set.
template <int DT, bool TA, bool TB, bool VA, bool VB, int WAT>
__device__ __forceinline__ void big_loop_checked(const uint16_t *__restrict__ A, const uint16_t *__restrict__ B,
                                                 size_t M, size_t N, size_t K, size_t m0, size_t n0,
                                                 const StageBig<!TA> &sa, const StageBig<TB> &sb,
                                                 uint16_t (*As)[kG_BM][kG_KP], uint16_t (*Bs)[kG_BN][kG_KP],
                                                 f32x16 (&acc)[4][4], int wm, int wn, int l32, int lhi) {
    u32x4 ra[8], rb[8];
    int buf = 0;
    for (size_t k0 = 0; k0 < K; k0 += kG_BK) {
        // the last step reloads its own tile and stores it to the idle buffer
        const size_t kn = k0 + kG_BK < K ? k0 + kG_BK : k0;
        big_load<!TA, VA, true>(sa, A, m0, kn, M, K, ra);
        big_load<TB, VB, true>(sb, B, n0, kn, N, K, rb);
        big_step<DT, TA, TB, WAT>(sa, sb, As, Bs, buf, ra, rb, acc, wm, wn, l32, lhi);
        __syncthreads();
        buf ^= 1;
    }
}

template <int DT, bool TA, bool TB, bool VA, bool VB, int WAT>
__global__ __launch_bounds__(kHThreads) void k_gemm16_big(const uint16_t *__restrict__ A,
                                                          const uint16_t *__restrict__ B, uint16_t *__restrict__ C,
                                                          size_t M, size_t N, size_t K, unsigned tiles_n) {
    constexpr int WI = 4, WJ = 4;
    __shared__ uint16_t As[2][kG_BM][kG_KP];
    __shared__ uint16_t Bs[2][kG_BN][kG_KP];

    const unsigned wg = xcd_remap16(blockIdx.x, gridDim.x);
    const size_t m0 = static_cast<size_t>(wg / tiles_n) * kG_BM;
    const size_t n0 = static_cast<size_t>(wg % tiles_n) * kG_BN;
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

    StageBig<!TA> sa;
    StageBig<TB> sb;
    sa.init(tid);
    sb.init(tid);
    {
        u32x4 ra[8], rb[8];
        sa.template load<VA>(A, m0, 0, M, K, ra);
        sb.template load<VB>(B, n0, 0, N, K, rb);
        sa.store(As[0], ra);
        sb.store(Bs[0], rb);
    }
    __syncthreads();
    // interior tiles with 128-bit loads and K a multiple of 2*BK take the
    // unchecked, double-staged loop
    const bool full = VA && VB && m0 + kG_BM <= M && n0 + kG_BN <= N && K % (2 * kG_BK) == 0;
    if (full)
        big_loop_fast<DT, TA, TB, WAT>(A, B, M, N, K, m0, n0, sa, sb, As, Bs, acc, wm, wn, l32, lhi);
    else
        big_loop_checked<DT, TA, TB, VA, VB, WAT>(A, B, M, N, K, m0, n0, sa, sb, As, Bs, acc, wm, wn, l32, lhi);

#pragma unroll
    for (int i = 0; i < WI; ++i)
#pragma unroll
        for (int j = 0; j < WJ; ++j) {
            const size_t col = n0 + wn * 128 + j * 32 + l32;
            if (col >= N) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const size_t row = m0 + wm * 128 + i * 32 + 8 * (r / 4) + 4 * lhi + (r % 4);
                if (row < M) C[row * N + col] = H<DT>::store(acc[i][j][r]);
            }
        }
}

// ----------------------------------------------- ring: four LDS stages of BK 32
//
// A TM x TM workgroup tile (TM = 256 or 128), four waves of TM/2 x TM/2
// (NB x NB MFMA blocks of 32x32, NB = TM/64), interior tiles only (M, N
// multiples of TM, K a multiple of 128).  The k loop runs over a ring of
// four LDS stages of 32 k, filled by direct global-to-LDS loads
// (lds_load16) four steps ahead (three tiles in flight); the loop is
// unrolled over the ring so that stage addresses are constants.
// A step on stage t: MFMAs of k block 0 with block 1's fragments read
// between them; the ring barrier (this wave's loads of stage t+1 landed,
// every wave done reading stage t); the next stage's block-0 fragments;
// loads of tile t+4 into stage t; MFMAs of k block 1.
//
// A is stored [M,K] (k contiguous).  Its stage holds TM rows of 64 bytes,
// the four 16-byte groups of row r XOR-keyed by (r / 4) % 4: 16
// consecutive rows, one group each, land on 16 distinct 16-byte slots of
// the 64 banks, so a ds_read_b128 fragment read is conflict-free.
// B is either stored as B^T [N,K] (KB, same stage layout as A) or as
// [K,N] (n contiguous).  The [K,N] stage holds 32 k rows of TM columns as
// loaded, 16-byte chunk c of row r at c ^ 4*(r % 4), and fragments come
// from ds_read_b64_tr_b16: in each 16-lane group, result lane i element e
// is element i % 4 of the 64 bits addressed by lane i / 4 + 4 e.  Lane j
// of a group addresses row k0 + j / 4, columns n0 + 4 (j % 4) .. +3, so
// lane i receives B[k0 .. k0+3][n0 + i]: four consecutive k of one column,
// half of a 32x32x16 operand; two reads give the eight.  The chunk key puts
// the four rows one read touches (64 bytes each) on distinct banks.
constexpr int kR_BK = 32;

template <int TM>
struct Ring {
    static constexpr int NB = TM / 64;            // 32x32 blocks per wave side
    static constexpr int TILE = TM * kR_BK;       // elements per operand stage
    static constexpr int ISSUES = TM / 64;        // load instructions per wave per operand per stage
    static constexpr int PER_STAGE = 2 * ISSUES;  // loads a wave has in flight per stage
};

__device__ __forceinline__ int rkey(int r) { return (r >> 2) & 3; }
__device__ __forceinline__ int roff(int row, int g) { return row * kR_BK + 8 * (g ^ rkey(row)); }
// element offset of (k row r, column n) in a [K,N] stage of TM columns
template <int TM>
__device__ __forceinline__ int noff(int r, int n) {
    return r * TM + ((((n >> 3) ^ (4 * (r & 3)))) << 3) + (n & 7);
}

// Stage fills.  A TM x 32 stage of X k-contiguous (row stride Kd) at rows
// r0.., k0..: each wave fills TM/4 rows, 16 per instruction (lane L: row
// L/4, LDS group L%4, global group (L%4) ^ key).  A 32 x TM stage of B
// stored [K,N] (row stride N) at k rows k0.., columns n0..: each wave
// fills 8 rows; an instruction covers 1 KiB, i.e. 64 / (TM/8) rows (lane
// L: row L / (TM/8), LDS chunk L % (TM/8), global chunk
// (L % (TM/8)) ^ 4*(row % 4)).  Each load reads from a base uniform across
// the workgroup (X + r0 Kd + k0, or B + k0 N + n0) plus a 32-bit lane
// offset fixed for the whole K loop (RingOffs16), into an LDS destination
// computed on the scalar unit: no 64-bit vector address arithmetic per load.
template <int TM>
struct RingOffs16 {
    unsigned o[Ring<TM>::ISSUES];
};
template <int TM>
__device__ __forceinline__ RingOffs16<TM> ring_offs_k(size_t Kd) {
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
    const int rr = lane >> 2, p = lane & 3;
    RingOffs16<TM> f;
#pragma unroll
    for (int s = 0; s < Ring<TM>::ISSUES; ++s) {
        const int row = w * (TM / 4) + s * 16 + rr;
        f.o[s] = static_cast<unsigned>((row * Kd + 8 * (p ^ rkey(row))) * sizeof(uint16_t));
    }
    return f;
}
template <int TM>
__device__ __forceinline__ RingOffs16<TM> ring_offs_n(size_t N) {
    constexpr int CPR = TM / 8, RPI = kWave / CPR;
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
    const int rr = lane / CPR, p = lane % CPR;
    RingOffs16<TM> f;
#pragma unroll
    for (int s = 0; s < Ring<TM>::ISSUES; ++s) {
        const int row = w * 8 + s * RPI + rr;
        f.o[s] = static_cast<unsigned>((row * N + 8 * (p ^ (4 * (row & 3)))) * sizeof(uint16_t));
    }
    return f;
}
// k-contiguous stage (KC) at rows r0.., k0..; else a [K,N] stage at k rows
// k0.., columns r0..
template <int TM, bool KC>
__device__ __forceinline__ void ring_issue_at(const uint16_t *__restrict__ X, size_t r0, size_t k0, size_t ld,
                                              const RingOffs16<TM> &f, uint16_t *stage) {
    const unsigned w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const uint16_t *base = KC ? X + r0 * ld + k0 : X + k0 * ld + r0;
    const unsigned l0 = lds_addr(stage) + (KC ? w * (TM / 4) * kR_BK : w * 8 * TM) * sizeof(uint16_t);
#pragma unroll
    for (int s = 0; s < Ring<TM>::ISSUES; ++s) lds_load16_at(base, f.o[s], l0 + s * kWave * 16);
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

// Fragments of k block kb (16 k) of a stage: A rows wm*TM/2 + 32 i + l32,
// eight k at 16 kb + 8 lhi; B likewise from the k-contiguous or the [K,N]
// stage.
template <int TM, bool KB>
__device__ __forceinline__ void ring_frags(const uint16_t *sa, const uint16_t *sb, int kb, int wm, int wn, int l32,
                                           int lhi, u32x4 (&fa)[Ring<TM>::NB], u32x4 (&fb)[Ring<TM>::NB]) {
    constexpr int NB = Ring<TM>::NB;
#pragma unroll
    for (int i = 0; i < NB; ++i)
        fa[i] = *reinterpret_cast<const u32x4 *>(sa + roff(wm * (TM / 2) + i * 32 + l32, 2 * kb + lhi));
    if constexpr (KB) {
#pragma unroll
        for (int j = 0; j < NB; ++j)
            fb[j] = *reinterpret_cast<const u32x4 *>(sb + roff(wn * (TM / 2) + j * 32 + l32, 2 * kb + lhi));
    } else {
        const int lane = threadIdx.x & (kWave - 1);
        const int g = lane >> 4, jj = lane & 15;
        const int r = 16 * kb + 8 * (g >> 1) + (jj >> 2);
        const int c = 16 * (g & 1) + 4 * (jj & 3);
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int n = wn * (TM / 2) + j * 32 + c;
            const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) s16x4 *)(sb + noff<TM>(r, n)));
            const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) s16x4 *)(sb + noff<TM>(r + 4, n)));
            const u32x2 ul = __builtin_bit_cast(u32x2, lo), uh = __builtin_bit_cast(u32x2, hi);
            fb[j] = u32x4{ul.x, ul.y, uh.x, uh.y};
        }
    }
}

template <int DT, int NB>
__device__ __forceinline__ void ring_mfma(const u32x4 (&fa)[NB], const u32x4 (&fb)[NB], f32x16 (&acc)[NB][NB]) {
#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[i][j] = mfma16<DT>(fa[i], fb[j], acc[i][j]);
}

// Interleaves a k block's MFMAs with the fragment reads of the next block:
// two MFMAs per read for the 256 tile with k-contiguous B (eight reads),
// otherwise one MFMA per read until either runs out.
template <int TM, bool KB>
__device__ __forceinline__ void ring_interleave() {
    constexpr int NM = Ring<TM>::NB * Ring<TM>::NB;
    constexpr int ND = Ring<TM>::NB * (KB ? 2 : 3);
    if constexpr (TM == 256 && KB) {
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
    } else {
        constexpr int P = NM < ND ? NM : ND;
#pragma unroll
        for (int t = 0; t < P; ++t) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        if constexpr (NM > P) __builtin_amdgcn_sched_group_barrier(0x008, NM - P, 0);
        if constexpr (ND > P) __builtin_amdgcn_sched_group_barrier(0x100, ND - P, 0);
    }
}

// Fills a B stage: k-contiguous (B^T [N,K], rows n0..) or [K,N] (k rows k0..).
template <int TM, bool KB>
__device__ __forceinline__ void ring_issue_b(const uint16_t *__restrict__ B, size_t n0, size_t kf, size_t K, size_t N,
                                             const RingOffs16<TM> &ob, uint16_t *stage) {
    if constexpr (KB) ring_issue_at<TM, true>(B, n0, kf, K, ob, stage);
    else ring_issue_at<TM, false>(B, n0, kf, N, ob, stage);
}

// Step t on stage cur (A tile at +0, B tile at +TILE, tile t); nxt holds
// tile t+1.  After the barrier every wave has read all of cur, which is
// refilled at once with tile t+4 (k offset kf): three tiles stay in flight.
template <int DT, int TM, bool KB>
__device__ __forceinline__ void ring_step(const uint16_t *__restrict__ A, const uint16_t *__restrict__ B, size_t K,
                                          size_t N, size_t m0, size_t n0, size_t kf, uint16_t *cur,
                                          const uint16_t *nxt, u32x4 (&fa)[Ring<TM>::NB], u32x4 (&fb)[Ring<TM>::NB],
                                          f32x16 (&acc)[Ring<TM>::NB][Ring<TM>::NB], int wm, int wn, int l32,
                                          int lhi, const RingOffs16<TM> &oa, const RingOffs16<TM> &ob) {
    constexpr int NB = Ring<TM>::NB, TILE = Ring<TM>::TILE;
    u32x4 ga[NB], gb[NB];
    ring_frags<TM, KB>(cur, cur + TILE, 1, wm, wn, l32, lhi, ga, gb);  // block 1, during block 0's MFMAs
    ring_mfma<DT, NB>(fa, fb, acc);
    ring_interleave<TM, KB>();
    ring_barrier<2 * Ring<TM>::PER_STAGE>();  // tile t+1 has landed; tiles t+2, t+3 may be in flight
    ring_frags<TM, KB>(nxt, nxt + TILE, 0, wm, wn, l32, lhi, fa, fb);  // next step's block 0
    ring_issue_at<TM, true>(A, m0, kf, K, oa, cur);
    ring_issue_b<TM, KB>(B, n0, kf, K, N, ob, cur + TILE);
    ring_mfma<DT, NB>(ga, gb, acc);
    ring_interleave<TM, KB>();
    __builtin_amdgcn_sched_group_barrier(0x020, Ring<TM>::PER_STAGE, 0);
}

// Tile order: the XCD remap gives each XCD a contiguous range of tile ids;
// inside it, ids walk down GM tile rows before moving one tile column, so
// the tiles an XCD runs at once share GM row blocks of A and a few column
// blocks of B in its L2 (one tile row would share 1 and all of them).
__device__ __forceinline__ void group_tile(unsigned id, unsigned tiles_m, unsigned tiles_n, unsigned gm, unsigned *tm,
                                           unsigned *tn) {
    const unsigned per_group = gm * tiles_n;
    const unsigned group = id / per_group;
    const unsigned first = group * gm;
    const unsigned rows = tiles_m - first < gm ? tiles_m - first : gm;
    const unsigned in = id - group * per_group;
    *tm = first + in % rows;
    *tn = in / rows;
}

// C = A B with A [M,K]; B as B^T [N,K] (KB) or [K,N].
template <int DT, int TM, bool KB>
__global__ __launch_bounds__(kHThreads) void k_gemm16_ring(const uint16_t *__restrict__ A,
                                                           const uint16_t *__restrict__ B, uint16_t *__restrict__ C,
                                                           size_t M, size_t N, size_t K, unsigned tiles_n,
                                                           unsigned gm) {
    constexpr int NB = Ring<TM>::NB, TILE = Ring<TM>::TILE, PS = Ring<TM>::PER_STAGE;
    // one array per stage: A tile, then B tile
    __shared__ __attribute__((aligned(16))) uint16_t s0[2 * TILE], s1[2 * TILE], s2[2 * TILE], s3[2 * TILE];
    unsigned tm, tn;
    group_tile(xcd_remap16(blockIdx.x, gridDim.x), static_cast<unsigned>(M / TM), tiles_n, gm, &tm, &tn);
    const size_t m0 = static_cast<size_t>(tm) * TM;
    const size_t n0 = static_cast<size_t>(tn) * TM;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int wm = wave >> 1, wn = wave & 1;
    const int l32 = lane & 31, lhi = lane >> 5;

    f32x16 acc[NB][NB];
#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // K % 128 == 0: tiles 0..T-1, T >= 4.  Tiles beyond T-1 reload tile T-1
    // into stages whose fragments are not used.
    const size_t T = K / kR_BK;
    auto kt = [&](size_t t) { return (t < T ? t : T - 1) * kR_BK; };
    const RingOffs16<TM> oa = ring_offs_k<TM>(K), ob = KB ? ring_offs_k<TM>(K) : ring_offs_n<TM>(N);
    ring_issue_at<TM, true>(A, m0, kt(0), K, oa, s0);
    ring_issue_b<TM, KB>(B, n0, kt(0), K, N, ob, s0 + TILE);
    ring_issue_at<TM, true>(A, m0, kt(1), K, oa, s1);
    ring_issue_b<TM, KB>(B, n0, kt(1), K, N, ob, s1 + TILE);
    ring_issue_at<TM, true>(A, m0, kt(2), K, oa, s2);
    ring_issue_b<TM, KB>(B, n0, kt(2), K, N, ob, s2 + TILE);
    ring_issue_at<TM, true>(A, m0, kt(3), K, oa, s3);
    ring_issue_b<TM, KB>(B, n0, kt(3), K, N, ob, s3 + TILE);
    ring_barrier<3 * PS>();
    u32x4 fa[NB], fb[NB];
    ring_frags<TM, KB>(s0, s0 + TILE, 0, wm, wn, l32, lhi, fa, fb);
    for (size_t t = 0; t < T; t += 4) {
        ring_step<DT, TM, KB>(A, B, K, N, m0, n0, kt(t + 4), s0, s1, fa, fb, acc, wm, wn, l32, lhi, oa, ob);
        ring_step<DT, TM, KB>(A, B, K, N, m0, n0, kt(t + 5), s1, s2, fa, fb, acc, wm, wn, l32, lhi, oa, ob);
        ring_step<DT, TM, KB>(A, B, K, N, m0, n0, kt(t + 6), s2, s3, fa, fb, acc, wm, wn, l32, lhi, oa, ob);
        ring_step<DT, TM, KB>(A, B, K, N, m0, n0, kt(t + 7), s3, s0, fa, fb, acc, wm, wn, l32, lhi, oa, ob);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no load into LDS outlives the workgroup

    // the tile origin again, from the workgroup index: kept live across the
    // K loop it was spilled to scratch (all 512 registers hold the
    // accumulators and the ring's fragments there)
    group_tile(xcd_remap16(blockIdx.x, gridDim.x), static_cast<unsigned>(M / TM), tiles_n, gm, &tm, &tn);
    const size_t em0 = static_cast<size_t>(__builtin_amdgcn_readfirstlane(tm)) * TM;
    const size_t en0 = static_cast<size_t>(__builtin_amdgcn_readfirstlane(tn)) * TM;
#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const size_t col = en0 + wn * (TM / 2) + j * 32 + l32;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const size_t row = em0 + wm * (TM / 2) + i * 32 + 8 * (r / 4) + 4 * lhi + (r % 4);
                C[row * N + col] = H<DT>::store(acc[i][j][r]);
            }
        }
}

inline hipStream_t hs(cxm_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// 16-bit transpose of a row-major [R, Cn] matrix into [Cn, R], R and Cn
// multiples of 128: a 256-thread workgroup per 128x128 tile.  The tile
// goes through LDS so that both global sides are coalesced: loads with 16
// lanes along a row (256 contiguous bytes), then each thread takes an 8x8
// block from LDS (eight 128-bit reads), transposes it in registers and
// stores it with 16 lanes along an output row.
constexpr int kT16 = 128, kT16P = kT16 + 8;

__global__ __launch_bounds__(kHThreads) void k_t16(const uint16_t *__restrict__ X, uint16_t *__restrict__ Y, size_t R,
                                                  size_t Cn, unsigned tiles_c) {
    __shared__ __attribute__((aligned(16))) uint16_t t[kT16][kT16P];
    const size_t r0 = static_cast<size_t>(blockIdx.x / tiles_c) * kT16;
    const size_t c0 = static_cast<size_t>(blockIdx.x % tiles_c) * kT16;
    {
        const int cc = threadIdx.x % 16, rr = threadIdx.x / 16;  // 16 lanes per 256-byte row piece
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int row = rr + 16 * i;
            *reinterpret_cast<u32x4 *>(&t[row][8 * cc]) =
                *reinterpret_cast<const u32x4 *>(X + (r0 + row) * Cn + c0 + 8 * cc);
        }
    }
    __syncthreads();
    const int br = threadIdx.x % 16, bc = threadIdx.x / 16;  // block (br, bc); lanes walk br
    u32x4 v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = *reinterpret_cast<const u32x4 *>(&t[8 * br + i][8 * bc]);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        u32x4 o;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const unsigned a = v[2 * w][j / 2], b = v[2 * w + 1][j / 2];
            o[w] = (j & 1) ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16));
        }
        *reinterpret_cast<u32x4 *>(Y + (c0 + 8 * bc + j) * R + r0 + 8 * br) = o;
    }
}

// Launches k_t16 after checking the shape it assumes.
int transpose16(const uint16_t *X, uint16_t *Y, size_t R, size_t Cn, hipStream_t s) {
    if (R % kT16 != 0 || Cn % kT16 != 0 || !aligned16(X) || !aligned16(Y)) return CXM_E_INVALID;
    const size_t tiles = (R / kT16) * (Cn / kT16);
    if (tiles > 0x7fffffffu) return CXM_E_TOO_LARGE;
    hipLaunchKernelGGL(k_t16, dim3(static_cast<unsigned>(tiles)), dim3(kHThreads), 0, s, X, Y, R, Cn,
                       static_cast<unsigned>(Cn / kT16));
    return launch_status();
}

template <int DT, bool TA, bool TB>
int launch16(const uint16_t *A, const uint16_t *B, uint16_t *C, size_t M, size_t N, size_t K, bool va, bool vb,
             dim3 grid, unsigned tn, hipStream_t s) {
    if (va && vb) hipLaunchKernelGGL((k_gemm16<DT, TA, TB, true, true>), grid, dim3(kHThreads), 0, s, A, B, C, M, N, K, tn);
    else if (va) hipLaunchKernelGGL((k_gemm16<DT, TA, TB, true, false>), grid, dim3(kHThreads), 0, s, A, B, C, M, N, K, tn);
    else if (vb) hipLaunchKernelGGL((k_gemm16<DT, TA, TB, false, true>), grid, dim3(kHThreads), 0, s, A, B, C, M, N, K, tn);
    else hipLaunchKernelGGL((k_gemm16<DT, TA, TB, false, false>), grid, dim3(kHThreads), 0, s, A, B, C, M, N, K, tn);
    return launch_status();
}

template <int DT, bool TA, bool TB>
int launch_big(const uint16_t *A, const uint16_t *B, uint16_t *C, size_t M, size_t N, size_t K, bool va, bool vb,
               dim3 grid, unsigned tn, hipStream_t s) {
    constexpr int W = 3;
    if (va && vb) hipLaunchKernelGGL((k_gemm16_big<DT, TA, TB, true, true, W>), grid, dim3(kHThreads), 0, s, A, B, C, M, N, K, tn);
    else if (va) hipLaunchKernelGGL((k_gemm16_big<DT, TA, TB, true, false, W>), grid, dim3(kHThreads), 0, s, A, B, C, M, N, K, tn);
    else if (vb) hipLaunchKernelGGL((k_gemm16_big<DT, TA, TB, false, true, W>), grid, dim3(kHThreads), 0, s, A, B, C, M, N, K, tn);
    else hipLaunchKernelGGL((k_gemm16_big<DT, TA, TB, false, false, W>), grid, dim3(kHThreads), 0, s, A, B, C, M, N, K, tn);
    return launch_status();
}

template <int DT, bool TA, bool TB>
int dispatch16(const uint16_t *A, const uint16_t *B, uint16_t *C, size_t M, size_t N, size_t K, bool va, bool vb,
               hipStream_t s, int kernel) {
    if (kernel == 0) {
        const size_t tn = (N + kH_BN - 1) / kH_BN;
        return launch16<DT, TA, TB>(A, B, C, M, N, K, va, vb, dim3(static_cast<unsigned>((M + kH_BM - 1) / kH_BM * tn)),
                                    static_cast<unsigned>(tn), s);
    }
    const size_t tn = (N + kG_BN - 1) / kG_BN;
    return launch_big<DT, TA, TB>(A, B, C, M, N, K, va, vb, dim3(static_cast<unsigned>((M + kG_BM - 1) / kG_BM * tn)),
                                  static_cast<unsigned>(tn), s);
}

// Kernel choice, where the ring's conditions hold (M, N multiples of the
// tile, K of 128, 16-byte aligned bases; A stored [K,M] is first transposed
// into the stream's workspace, B is read as stored):
//  * at least 128 tiles of 256x256: the 256 ring, else the 256x256
//    register-staged kernel (any shape);
//  * smaller grids: the 128 ring, else the 128x128 register-staged kernel.
// g_gemm16_kernel (tests) forces 0 = 128x128 staged, 1 = 256x256 staged,
// 2 = 256 ring, 3 = 128 ring; a ring whose conditions fail falls back to
// the staged kernel of its tile size.
std::atomic<int> g_gemm16_kernel{-1};
constexpr unsigned kRingGroup = 4;

template <int DT, int TM>
int launch_ring(const uint16_t *A, const uint16_t *B, uint16_t *C, size_t M, size_t N, size_t K, bool ta, bool tb,
                cxm_stream_t st) {
    hipStream_t s = hs(st);
    const uint16_t *Ak = A;
    if (ta) {  // A stored [K, M]
        Workspace ws;
        const int rc = get_workspace(st, 0, M * K * sizeof(uint16_t), &ws);
        if (rc) return rc;
        uint16_t *w = static_cast<uint16_t *>(ws.scratch);
        const int r = transpose16(A, w, K, M, s);
        if (r) return r;
        Ak = w;
    }
    const unsigned tn = static_cast<unsigned>(N / TM);
    const dim3 grid(static_cast<unsigned>((M / TM) * (N / TM)));
    if (tb)
        hipLaunchKernelGGL((k_gemm16_ring<DT, TM, true>), grid, dim3(kHThreads), 0, s, Ak, B, C, M, N, K, tn,
                           kRingGroup);
    else
        hipLaunchKernelGGL((k_gemm16_ring<DT, TM, false>), grid, dim3(kHThreads), 0, s, Ak, B, C, M, N, K, tn,
                           kRingGroup);
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
    hipStream_t s = hs(st);
    const size_t big_tiles = ((M + kG_BM - 1) / kG_BM) * ((N + kG_BN - 1) / kG_BN);
    // (the ring's lane offsets within a stage are 32-bit: K, N < 2^23)
    const bool al = aligned16(A) && aligned16(B) && aligned16(C) && K % (4 * kR_BK) == 0 &&
                    K < (size_t(1) << 23) && N < (size_t(1) << 23);
    const bool ring256 = al && M % 256 == 0 && N % 256 == 0;
    const bool ring128 = al && M % 128 == 0 && N % 128 == 0;
    int kernel = big_tiles >= 128 ? (ring256 ? 2 : 1) : (ring128 ? 3 : 0);
    const int pinned = g_gemm16_kernel.load(std::memory_order_relaxed);
    if (pinned >= 0) {
        kernel = pinned;
        if (kernel == 2 && !ring256) kernel = 1;
        if (kernel == 3 && !ring128) kernel = 0;
    }
    if (kernel == 2) return launch_ring<DT, 256>(A, B, C, M, N, K, ta, tb, st);
    if (kernel == 3) return launch_ring<DT, 128>(A, B, C, M, N, K, ta, tb, st);
    if (!ta && !tb) return dispatch16<DT, false, false>(A, B, C, M, N, K, va, vb, s, kernel);
    if (ta && !tb) return dispatch16<DT, true, false>(A, B, C, M, N, K, va, vb, s, kernel);
    if (!ta && tb) return dispatch16<DT, false, true>(A, B, C, M, N, K, va, vb, s, kernel);
    return dispatch16<DT, true, true>(A, B, C, M, N, K, va, vb, s, kernel);
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

int cxm_gemm16_kernel(int kernel) {
    if (kernel < -1 || kernel > 3) return CXM_E_INVALID;
    cxm::g_gemm16_kernel.store(kernel);
    return CXM_OK;
}

}  // extern "C"
