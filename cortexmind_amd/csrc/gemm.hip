// fp32 GEMM on the CDNA4 matrix cores (v_mfma_f32_32x32x2_f32), with the
// transposed forms the MLP backward needs and a fused epilogue.
//
// Replaces matrix_t::matmul (source/CortexMind/framework/Engine/AVX2/
// matrix.cpp:75-147, row-major NN only) and nv::Matrix::matmul
// (Engine/CUDA/matrix.cu:112-159, cuBLAS with TF32 compute).  This kernel is
// true fp32: every product and sum is an fp32 operation of the MFMA unit.
//
// Tiling: a 256-thread workgroup computes a 128x128 tile of C; its four
// waves each own 64x64 = 2x2 MFMA tiles of 32x32 (64 accumulator
// registers per lane).  K advances in steps of 16 through double-buffered
// LDS tiles stored k-major (As[k][m], Bs[k][n]), so every fragment read is
// one ds_read_b32 with consecutive lanes on consecutive addresses whatever
// the global layout; global->LDS loads are 128-bit when the leading
// dimension allows.  When the grid would be too small to fill 256 CUs
// (tall-K products such as X^T * dZ), K is split across workgroups: each
// writes its partial tile to the workspace and the last workgroup of the
// tile adds the partials in split order, so results are deterministic.
//
// MFMA operand layout (32x32x2, one block): lane l supplies A[l%32][l/32]
// and B[l/32][l%32]; accumulator register r of lane l holds
// C[8*(r/4) + 4*(l/32) + r%4][l%32].
#include "cxm_common.hpp"

namespace cxm {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 128, BK = 16, PAD = 4;

struct Epilogue {
    const float *bias;  // [N] or null
    const float *gate;  // [M, N] or null: multiply by (gate > 0 ? 1 : 0)
    int act;            // CXM_ACT_NONE or CXM_ACT_RELU
};

__device__ __forceinline__ float apply_epi(const Epilogue &e, float v, size_t row, size_t col, size_t N) {
    if (e.bias) v = v + e.bias[col];
    if (e.act == CXM_ACT_RELU) v = 0.0f > v ? 0.0f : v;
    if (e.gate) v = v * (e.gate[row * N + col] > 0.0f ? 1.0f : 0.0f);
    return v;
}

// Loads one 4-element group of the A tile (slot 0..511) into registers.
// Non-transposed A [M,K]: group = 4 consecutive k of one row.
// Transposed A (stored [K,M]): group = 4 consecutive m of one k.
template <bool TA, bool VA>
__device__ __forceinline__ float4 load_a(const float *__restrict__ A, int slot, size_t m0, size_t k0,
                                         size_t M, size_t K) {
    size_t r, c;  // index in the stored matrix of the group's first element
    size_t lim_r, lim_c;
    if constexpr (!TA) {
        r = m0 + slot / 4;
        c = k0 + (slot % 4) * 4;
        lim_r = M;
        lim_c = K;
    } else {
        r = k0 + slot / 32;
        c = m0 + (slot % 32) * 4;
        lim_r = K;
        lim_c = M;
    }
    if (r >= lim_r) return make_float4(0.f, 0.f, 0.f, 0.f);
    const float *p = A + r * lim_c + c;
    if constexpr (VA) {
        if (c < lim_c) return ld4(p);  // lim_c % 4 == 0: the group is all in or all out
        return make_float4(0.f, 0.f, 0.f, 0.f);
    } else {
        return make_float4(c < lim_c ? p[0] : 0.f, c + 1 < lim_c ? p[1] : 0.f,
                           c + 2 < lim_c ? p[2] : 0.f, c + 3 < lim_c ? p[3] : 0.f);
    }
}

// Non-transposed B [K,N]: group = 4 consecutive n of one k.
// Transposed B (stored [N,K]): group = 4 consecutive k of one n.
template <bool TB, bool VB>
__device__ __forceinline__ float4 load_b(const float *__restrict__ B, int slot, size_t n0, size_t k0,
                                         size_t N, size_t K) {
    size_t r, c, lim_r, lim_c;
    if constexpr (!TB) {
        r = k0 + slot / 32;
        c = n0 + (slot % 32) * 4;
        lim_r = K;
        lim_c = N;
    } else {
        r = n0 + slot / 4;
        c = k0 + (slot % 4) * 4;
        lim_r = N;
        lim_c = K;
    }
    if (r >= lim_r) return make_float4(0.f, 0.f, 0.f, 0.f);
    const float *p = B + r * lim_c + c;
    if constexpr (VB) {
        if (c < lim_c) return ld4(p);
        return make_float4(0.f, 0.f, 0.f, 0.f);
    } else {
        return make_float4(c < lim_c ? p[0] : 0.f, c + 1 < lim_c ? p[1] : 0.f,
                           c + 2 < lim_c ? p[2] : 0.f, c + 3 < lim_c ? p[3] : 0.f);
    }
}

template <bool TA>
__device__ __forceinline__ void store_a(float (*As)[BM + PAD], int slot, float4 v) {
    if constexpr (!TA) {
        const int m = slot / 4, k = (slot % 4) * 4;
        As[k + 0][m] = v.x;
        As[k + 1][m] = v.y;
        As[k + 2][m] = v.z;
        As[k + 3][m] = v.w;
    } else {
        const int k = slot / 32, m = (slot % 32) * 4;
        *reinterpret_cast<float4 *>(&As[k][m]) = v;
    }
}

template <bool TB>
__device__ __forceinline__ void store_b(float (*Bs)[BN + PAD], int slot, float4 v) {
    if constexpr (!TB) {
        const int k = slot / 32, n = (slot % 32) * 4;
        *reinterpret_cast<float4 *>(&Bs[k][n]) = v;
    } else {
        const int n = slot / 4, k = (slot % 4) * 4;
        Bs[k + 0][n] = v.x;
        Bs[k + 1][n] = v.y;
        Bs[k + 2][n] = v.z;
        Bs[k + 3][n] = v.w;
    }
}

template <bool TA, bool TB, bool VA, bool VB>
__global__ __launch_bounds__(kBlock) void k_gemm(const float *__restrict__ A, const float *__restrict__ B,
                                                 float *__restrict__ C, size_t M, size_t N, size_t K,
                                                 unsigned tiles_n, unsigned splits, size_t kper,
                                                 Epilogue epi, float *__restrict__ part,
                                                 unsigned *__restrict__ counters) {
    __shared__ float As[2][BK][BM + PAD];
    __shared__ float Bs[2][BK][BN + PAD];
    __shared__ int flag;

    const unsigned tile = blockIdx.x / splits;
    const unsigned split = blockIdx.x - tile * splits;
    const size_t m0 = static_cast<size_t>(tile / tiles_n) * BM;
    const size_t n0 = static_cast<size_t>(tile % tiles_n) * BN;
    const size_t kbeg = static_cast<size_t>(split) * kper;
    const size_t kend = kbeg + kper < K ? kbeg + kper : K;

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int wm = wave >> 1, wn = wave & 1;
    const int l32 = lane & 31, lhi = lane >> 5;

    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    float4 ra[2], rb[2];
    int buf = 0;
    if (kbeg < kend) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            ra[s] = load_a<TA, VA>(A, tid + s * kBlock, m0, kbeg, M, K);
            rb[s] = load_b<TB, VB>(B, tid + s * kBlock, n0, kbeg, N, K);
        }
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            store_a<TA>(As[0], tid + s * kBlock, ra[s]);
            store_b<TB>(Bs[0], tid + s * kBlock, rb[s]);
        }
    }
    __syncthreads();

    for (size_t k0 = kbeg; k0 < kend; k0 += BK) {
        const bool more = k0 + BK < kend;
        if (more) {
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                ra[s] = load_a<TA, VA>(A, tid + s * kBlock, m0, k0 + BK, M, K);
                rb[s] = load_b<TB, VB>(B, tid + s * kBlock, n0, k0 + BK, N, K);
            }
        }
#pragma unroll
        for (int kk = 0; kk < BK; kk += 2) {
            float a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) a[i] = As[buf][kk + lhi][wm * 64 + i * 32 + l32];
#pragma unroll
            for (int j = 0; j < 2; ++j) b[j] = Bs[buf][kk + lhi][wn * 64 + j * 32 + l32];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        if (more) {
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                store_a<TA>(As[buf ^ 1], tid + s * kBlock, ra[s]);
                store_b<TB>(Bs[buf ^ 1], tid + s * kBlock, rb[s]);
            }
        }
        __syncthreads();
        buf ^= 1;
    }

    // Output element of accumulator (i, j, r) for this lane.
    auto out_row = [&](int i, int r) { return wm * 64 + i * 32 + 8 * (r / 4) + 4 * lhi + (r % 4); };
    auto out_col = [&](int j) { return wn * 64 + j * 32 + l32; };

    if (splits == 1) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const size_t row = m0 + out_row(i, r), col = n0 + out_col(j);
                    if (row < M && col < N) C[row * N + col] = apply_epi(epi, acc[i][j][r], row, col, N);
                }
        return;
    }

    float *my = part + (static_cast<size_t>(tile) * splits + split) * (BM * BN);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) st_dev(&my[out_row(i, r) * BN + out_col(j)], acc[i][j][r]);
    if (!last_block_ticket(ctr(counters, tile), splits, &flag)) return;
    // Sum the splits in split order; each round issues this lane's 64 loads together.
    const float *tp = part + static_cast<size_t>(tile) * splits * (BM * BN);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    for (unsigned s = 0; s < splits; ++s) {
        float v[2][2][16];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) v[i][j][r] = ld_dev(&tp[s * (BM * BN) + out_row(i, r) * BN + out_col(j)]);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = acc[i][j][r] + v[i][j][r];
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const size_t row = m0 + out_row(i, r), col = n0 + out_col(j);
                if (row < M && col < N) C[row * N + col] = apply_epi(epi, acc[i][j][r], row, col, N);
            }
}

template <bool TA, bool TB>
int launch_t(const float *A, const float *B, float *C, size_t M, size_t N, size_t K, bool va, bool vb,
             dim3 grid, unsigned tiles_n, unsigned splits, size_t kper, Epilogue epi, float *part,
             unsigned *counters, hipStream_t s) {
#define CXM_GEMM_LAUNCH(VA_, VB_)                                                                  \
    hipLaunchKernelGGL((k_gemm<TA, TB, VA_, VB_>), grid, dim3(kBlock), 0, s, A, B, C, M, N, K, tiles_n, \
                       splits, kper, epi, part, counters)
    if (va && vb) CXM_GEMM_LAUNCH(true, true);
    else if (va) CXM_GEMM_LAUNCH(true, false);
    else if (vb) CXM_GEMM_LAUNCH(false, true);
    else CXM_GEMM_LAUNCH(false, false);
#undef CXM_GEMM_LAUNCH
    return launch_status();
}

int gemm(const float *A, const float *B, float *C, size_t M, size_t K, size_t N, int ta, int tb,
         const float *bias, int act, const float *gate, cxm_stream_t st) {
    if (!A || !B || !C || (act != CXM_ACT_NONE && act != CXM_ACT_RELU)) return CXM_E_INVALID;
    if (M == 0 || N == 0) return CXM_OK;
    if (K == 0) return CXM_E_INVALID;
    const size_t tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    const size_t tiles = tiles_m * tiles_n;
    // Split K when the tile grid alone cannot fill the chip; each split
    // keeps at least 256 of K.
    size_t splits = 1;
    if (tiles < 512 && K >= 512) {
        splits = (512 + tiles - 1) / tiles;
        const size_t max_splits = K / 256;
        if (splits > max_splits) splits = max_splits;
        if (splits < 1) splits = 1;
    }
    size_t kper = (K + splits - 1) / splits;
    kper = (kper + BK - 1) / BK * BK;
    splits = (K + kper - 1) / kper;
    if (tiles * splits > 0x7fffffffu) return CXM_E_TOO_LARGE;
    float *part = nullptr;
    unsigned *counters = nullptr;
    if (splits > 1) {
        Workspace ws;
        int rc = get_workspace(st, tiles, tiles * splits * BM * BN * sizeof(float), &ws);
        if (rc) return rc;
        part = static_cast<float *>(ws.scratch);
        counters = ws.counters;
    }
    // 128-bit global loads need the stored row length to be a multiple of 4.
    const bool va = aligned16(A) && (ta ? M % 4 == 0 : K % 4 == 0);
    const bool vb = aligned16(B) && (tb ? K % 4 == 0 : N % 4 == 0);
    const Epilogue epi{bias, gate, act};
    const dim3 grid(static_cast<unsigned>(tiles * splits));
    hipStream_t s = reinterpret_cast<hipStream_t>(st);
    const unsigned tn = static_cast<unsigned>(tiles_n), sp = static_cast<unsigned>(splits);
    if (!ta && !tb) return launch_t<false, false>(A, B, C, M, N, K, va, vb, grid, tn, sp, kper, epi, part, counters, s);
    if (ta && !tb) return launch_t<true, false>(A, B, C, M, N, K, va, vb, grid, tn, sp, kper, epi, part, counters, s);
    if (!ta && tb) return launch_t<false, true>(A, B, C, M, N, K, va, vb, grid, tn, sp, kper, epi, part, counters, s);
    return launch_t<true, true>(A, B, C, M, N, K, va, vb, grid, tn, sp, kper, epi, part, counters, s);
}

}  // namespace
}  // namespace cxm

extern "C" {

int cxm_gemm_f32(const float *a, const float *b, float *c, size_t m, size_t k, size_t n, int trans_a,
                 int trans_b, const float *bias, int act, const float *gate, cxm_stream_t s) {
    return cxm::gemm(a, b, c, m, k, n, trans_a != 0, trans_b != 0, bias, act, gate, s);
}

int cxm_matmul_f32(const float *a, const float *b, float *c, size_t xN, size_t yN, size_t zN,
                   cxm_stream_t s) {
    return cxm::gemm(a, b, c, xN, yN, zN, 0, 0, nullptr, CXM_ACT_NONE, nullptr, s);
}

}  // extern "C"
