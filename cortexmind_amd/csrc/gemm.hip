// fp32 GEMM on the CDNA4 matrix cores (v_mfma_f32_32x32x2_f32), with the
// transposed forms the MLP backward needs and a fused epilogue.
//
// Replaces matrix_t::matmul (source/CortexMind/framework/Engine/AVX2/
// matrix.cpp:75-147, row-major NN only) and nv::Matrix::matmul
// (Engine/CUDA/matrix.cu:112-159, cuBLAS with TF32 compute).  This kernel is
// true fp32: every product and sum is an fp32 operation of the MFMA unit.
//
// Tiling: a 512-thread workgroup computes a 128x128 tile of C; its eight
// waves (two per SIMD, so one hides the other's LDS and barrier waits) each
// own 64x32 = 2x1 MFMA tiles of 32x32 (32 accumulator registers per lane).  K advances in steps of 32 through double-buffered
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
#include <atomic>

#include "cxm_common.hpp"
#include "mlp_side.hpp"

// Per-workgroup timeline of the ring products, for the diagnostics build only
// (this file compiled with -DCXM_TIMELINE into libcxm_hip_timeline.so,
// read by `bench.py --timeline c5`).  Thread 0 of a workgroup writes the
// 100 MHz s_memrealtime clock to mark i of its record: 0 entry, 1 the
// first four ring stages landed (prologue done), 2 the K loop done, 3 the
// epilogue done (past a barrier, so every wave's stores are issued); marks
// 4 and 5 hold the core-clock counter s_memtime at marks 1 and 2.  Table
// by instance: 0 the K-tail instance, 1 A.B, 2 A.B^T, 3 the other forms
// (the paired weight gradients' A^T.B).  Records are indexed by blockIdx.x
// modulo kGemmTlWgs; a launch overwrites the previous records of its
// instance.  Without CXM_TIMELINE the marks compile to nothing.
#ifdef CXM_TIMELINE
constexpr unsigned kGemmTlKinds = 4, kGemmTlWgs = 1024, kGemmTlMarks = 6;
static __device__ unsigned long long gemm_timeline[kGemmTlKinds][kGemmTlWgs][kGemmTlMarks];
__device__ __forceinline__ void gemm_tl_mark(unsigned kind, unsigned i) {
    if (threadIdx.x == 0) {
        unsigned long long *rec = gemm_timeline[kind][blockIdx.x % kGemmTlWgs];
        __builtin_nontemporal_store(__builtin_amdgcn_s_memrealtime(), &rec[i]);
        if (i == 1 || i == 2) __builtin_nontemporal_store(__builtin_amdgcn_s_memtime(), &rec[3 + i]);
    }
}
#else
__device__ __forceinline__ void gemm_tl_mark(unsigned, unsigned) {}
#endif

namespace cxm {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 128, BK = 32, PAD = 4;
constexpr int KQ = BK / 4;                      // 4-element groups along k in a tile row
constexpr int kGemmThreads = 512;               // 8 waves: 2 (m) x 4 (n), each 64 x 32 of C
constexpr int WI = 2, WJ = 1;                   // 32x32 MFMA tiles per wave along m and n
constexpr int SLOTS = BM * BK / 4 / kGemmThreads;  // float4 groups per thread per tile (A and B alike)
constexpr int kColTileThin = 256;  // m columns per workgroup of the thin TN kernel


// Workgroups are dispatched to the 8 XCDs round-robin (workgroup b runs on
// XCD b % 8).  Renumbering b so that each XCD gets one contiguous eighth of
// the row-major tile order makes the tiles sharing an XCD's L2 share A rows
// (and B columns), instead of every XCD touching every row block.
__device__ __forceinline__ unsigned xcd_remap(unsigned b, unsigned g) {
    if (g % 8 != 0) return b;
    return (b % 8) * (g / 8) + b / 8;
}

__device__ __forceinline__ void store_epi(const Epilogue &e, float *C, size_t row, size_t col, size_t N,
                                          float v) {
    float *p = C + row * N + col;
    if (e.sgd) {
        const float t = v * e.lr;  // matrix_t::sub(W, ScalarOp::mul(G, lr)): two roundings
        *p = *p - t;
        return;
    }
    if (e.bias) v = v + e.bias[col];
    if (e.act == CXM_ACT_RELU) v = 0.0f > v ? 0.0f : v;
    if (e.gate) v = v * (e.gate[row * N + col] > 0.0f ? 1.0f : 0.0f);
    *p = v;
}

// Writes a lane's WI_ x WJ_ accumulator blocks through the epilogue (same
// arithmetic as store_epi).  Every memory operand the epilogue reads (the
// gate, or C's old value for the SGD update, and the bias) is loaded for
// the whole tile before any result is computed, and the epilogue's options
// are applied with selects, so a lane whose outputs are all in range runs
// one straight block: loads, then arithmetic, then stores.  Element by
// element, each store waited for its own load (a memory round trip per
// element, 11 us of a 4096 x 1024 x 1024 product with a ReLU gate).
__device__ __forceinline__ float epi_value(const Epilogue &e, float v, float bias, float pre) {
    const float t = v * e.lr;  // SGD: matrix_t::sub(W, ScalarOp::mul(G, lr)): two roundings
    const float sgd = pre - t;
    float u = e.bias ? v + bias : v;
    u = (e.act == CXM_ACT_RELU && 0.0f > u) ? 0.0f : u;
    u = e.gate ? u * (pre > 0.0f ? 1.0f : 0.0f) : u;
    return e.sgd ? sgd : u;
}

template <int WI_, int WJ_, class RowF, class ColF>
__device__ __forceinline__ void store_tile_epi(const floatx16 (&acc)[WI_][WJ_], float *__restrict__ C, size_t M,
                                               size_t N, RowF row_of, ColF col_of, const Epilogue &e) {
    const float *pre_src = e.sgd ? C : e.gate;  // both [M, N]
    bool all_in = true;
#pragma unroll
    for (int i = 0; i < WI_; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) all_in = all_in && row_of(i, r) < M;
#pragma unroll
    for (int j = 0; j < WJ_; ++j) all_in = all_in && col_of(j) < N;
    float bias[WJ_];
#pragma unroll
    for (int j = 0; j < WJ_; ++j) {
        const size_t col = col_of(j);
        bias[j] = (e.bias && !e.sgd && col < N) ? e.bias[col] : 0.0f;
    }
    if (all_in) {
        float pre[WI_][WJ_][16];
#pragma unroll
        for (int i = 0; i < WI_; ++i)
#pragma unroll
            for (int j = 0; j < WJ_; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    pre[i][j][r] = pre_src ? pre_src[row_of(i, r) * N + col_of(j)] : 0.0f;
#pragma unroll
        for (int i = 0; i < WI_; ++i)
#pragma unroll
            for (int j = 0; j < WJ_; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    C[row_of(i, r) * N + col_of(j)] = epi_value(e, acc[i][j][r], bias[j], pre[i][j][r]);
        return;
    }
#pragma unroll
    for (int i = 0; i < WI_; ++i)
#pragma unroll
        for (int j = 0; j < WJ_; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const size_t row = row_of(i, r), col = col_of(j);
                if (row < M && col < N) store_epi(e, C, row, col, N, acc[i][j][r]);
            }
}

// Loads one 4-element group of the A tile (slot 0..BM*BK/4-1) into registers.
// Non-transposed A [M,K]: group = 4 consecutive k of one row.
// Transposed A (stored [K,M]): group = 4 consecutive m of one k.
template <bool TA, bool VA>
__device__ __forceinline__ float4 load_a(const float *__restrict__ A, int slot, size_t m0, size_t k0,
                                         size_t M, size_t K) {
    size_t r, c;  // index in the stored matrix of the group's first element
    size_t lim_r, lim_c;
    if constexpr (!TA) {
        r = m0 + slot / KQ;
        c = k0 + (slot % KQ) * 4;
        lim_r = M;
        lim_c = K;
    } else {
        r = k0 + slot / (BM / 4);
        c = m0 + (slot % (BM / 4)) * 4;
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
        r = k0 + slot / (BN / 4);
        c = n0 + (slot % (BN / 4)) * 4;
        lim_r = K;
        lim_c = N;
    } else {
        r = n0 + slot / KQ;
        c = k0 + (slot % KQ) * 4;
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
        const int m = slot / KQ, k = (slot % KQ) * 4;
        As[k + 0][m] = v.x;
        As[k + 1][m] = v.y;
        As[k + 2][m] = v.z;
        As[k + 3][m] = v.w;
    } else {
        const int k = slot / (BM / 4), m = (slot % (BM / 4)) * 4;
        *reinterpret_cast<float4 *>(&As[k][m]) = v;
    }
}

template <bool TB>
__device__ __forceinline__ void store_b(float (*Bs)[BN + PAD], int slot, float4 v) {
    if constexpr (!TB) {
        const int k = slot / (BN / 4), n = (slot % (BN / 4)) * 4;
        *reinterpret_cast<float4 *>(&Bs[k][n]) = v;
    } else {
        const int n = slot / KQ, k = (slot % KQ) * 4;
        Bs[k + 0][n] = v.x;
        Bs[k + 1][n] = v.y;
        Bs[k + 2][n] = v.z;
        Bs[k + 3][n] = v.w;
    }
}

// Writes the workgroup's 128x128 tile from the accumulators: directly (with
// the epilogue) when K is not split; otherwise the split's partial goes to
// the workspace and the last workgroup of the tile adds the partials in
// split order, then applies the epilogue.
template <int WI_, int WJ_>
__device__ __forceinline__ void gemm_epilogue(floatx16 (&acc)[WI_][WJ_], float *__restrict__ C, size_t M, size_t N,
                                              size_t m0, size_t n0, unsigned tile, unsigned split, unsigned splits,
                                              int wm, int wn, int lhi, int l32, const Epilogue &epi,
                                              float *__restrict__ part, unsigned *__restrict__ counters, int *flag) {
    // Output element of accumulator (i, j, r) for this lane.
    auto out_row = [&](int i, int r) { return wm * 32 * WI_ + i * 32 + 8 * (r / 4) + 4 * lhi + (r % 4); };
    auto out_col = [&](int j) { return wn * 32 * WJ_ + j * 32 + l32; };

    auto row_of = [&](int i, int r) { return m0 + out_row(i, r); };
    auto col_of = [&](int j) { return n0 + out_col(j); };
    if (splits == 1) {
        store_tile_epi<WI_, WJ_>(acc, C, M, N, row_of, col_of, epi);
        return;
    }

    float *my = part + (static_cast<size_t>(tile) * splits + split) * (BM * BN);
#pragma unroll
    for (int i = 0; i < WI_; ++i)
#pragma unroll
        for (int j = 0; j < WJ_; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) st_dev(&my[out_row(i, r) * BN + out_col(j)], acc[i][j][r]);
    if (!last_block_ticket(ctr(counters, tile), splits, flag)) return;
    // Sum the splits in split order; each round issues this lane's 64 loads together.
    const float *tp = part + static_cast<size_t>(tile) * splits * (BM * BN);
#pragma unroll
    for (int i = 0; i < WI_; ++i)
#pragma unroll
        for (int j = 0; j < WJ_; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    for (unsigned s = 0; s < splits; ++s) {
        float v[WI_][WJ_][16];
#pragma unroll
        for (int i = 0; i < WI_; ++i)
#pragma unroll
            for (int j = 0; j < WJ_; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) v[i][j][r] = ld_dev(&tp[s * (BM * BN) + out_row(i, r) * BN + out_col(j)]);
#pragma unroll
        for (int i = 0; i < WI_; ++i)
#pragma unroll
            for (int j = 0; j < WJ_; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = acc[i][j][r] + v[i][j][r];
    }
    store_tile_epi<WI_, WJ_>(acc, C, M, N, row_of, col_of, epi);
}

template <bool TA, bool TB, bool VA, bool VB, bool XCDMAP = false>
__global__ __launch_bounds__(kGemmThreads) void k_gemm(const float *__restrict__ A, const float *__restrict__ B,
                                                 float *__restrict__ C, size_t M, size_t N, size_t K,
                                                 unsigned tiles_n, unsigned splits, size_t kper,
                                                 Epilogue epi, float *__restrict__ part,
                                                 unsigned *__restrict__ counters) {
    __shared__ float As[2][BK][BM + PAD];
    __shared__ float Bs[2][BK][BN + PAD];
    __shared__ int flag;

    const unsigned wg = XCDMAP ? xcd_remap(blockIdx.x, gridDim.x) : blockIdx.x;
    const unsigned tile = wg / splits;
    const unsigned split = wg - tile * splits;
    const size_t m0 = static_cast<size_t>(tile / tiles_n) * BM;
    const size_t n0 = static_cast<size_t>(tile % tiles_n) * BN;
    const size_t kbeg = static_cast<size_t>(split) * kper;
    const size_t kend = kbeg + kper < K ? kbeg + kper : K;

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int wm = wave >> 2, wn = wave & 3;
    const int l32 = lane & 31, lhi = lane >> 5;

    floatx16 acc[WI][WJ];
#pragma unroll
    for (int i = 0; i < WI; ++i)
#pragma unroll
        for (int j = 0; j < WJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    float4 ra[SLOTS], rb[SLOTS];
    int buf = 0;
    if (kbeg < kend) {
#pragma unroll
        for (int s = 0; s < SLOTS; ++s) {
            ra[s] = load_a<TA, VA>(A, tid + s * kGemmThreads, m0, kbeg, M, K);
            rb[s] = load_b<TB, VB>(B, tid + s * kGemmThreads, n0, kbeg, N, K);
        }
#pragma unroll
        for (int s = 0; s < SLOTS; ++s) {
            store_a<TA>(As[0], tid + s * kGemmThreads, ra[s]);
            store_b<TB>(Bs[0], tid + s * kGemmThreads, rb[s]);
        }
    }
    __syncthreads();

    for (size_t k0 = kbeg; k0 < kend; k0 += BK) {
        const bool more = k0 + BK < kend;
        if (more) {
#pragma unroll
            for (int s = 0; s < SLOTS; ++s) {
                ra[s] = load_a<TA, VA>(A, tid + s * kGemmThreads, m0, k0 + BK, M, K);
                rb[s] = load_b<TB, VB>(B, tid + s * kGemmThreads, n0, k0 + BK, N, K);
            }
        }
        // Software-pipelined over k-steps of 2: the fragments of step t+1 are
        // read from LDS before the four MFMAs of step t are issued, so the
        // LDS latency hides behind 256 cycles of matrix work instead of
        // leaving the MFMA pipe idle once per step.
        float ca[WI], cb[WJ];
#pragma unroll
        for (int i = 0; i < WI; ++i) ca[i] = As[buf][lhi][wm * 64 + i * 32 + l32];
#pragma unroll
        for (int j = 0; j < WJ; ++j) cb[j] = Bs[buf][lhi][wn * 32 + j * 32 + l32];
#pragma unroll
        for (int t = 0; t < BK / 2; ++t) {
            float na[WI], nb[WJ];
            if (t + 1 < BK / 2) {
#pragma unroll
                for (int i = 0; i < WI; ++i) na[i] = As[buf][2 * (t + 1) + lhi][wm * 64 + i * 32 + l32];
#pragma unroll
                for (int j = 0; j < WJ; ++j) nb[j] = Bs[buf][2 * (t + 1) + lhi][wn * 32 + j * 32 + l32];
            }
#pragma unroll
            for (int i = 0; i < WI; ++i)
#pragma unroll
                for (int j = 0; j < WJ; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(ca[i], cb[j], acc[i][j], 0, 0, 0);
            if (t + 1 < BK / 2) {
#pragma unroll
                for (int i = 0; i < WI; ++i) ca[i] = na[i];
#pragma unroll
                for (int j = 0; j < WJ; ++j) cb[j] = nb[j];
            }
        }
        // Scheduling groups: reads of step 0, then (reads of step t+1, MFMAs of step t).
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
        for (int t = 0; t < BK / 2; ++t) {
            if (t + 1 < BK / 2) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, WI * WJ, 0);
        }
        if (more) {
#pragma unroll
            for (int s = 0; s < SLOTS; ++s) {
                store_a<TA>(As[buf ^ 1], tid + s * kGemmThreads, ra[s]);
                store_b<TB>(Bs[buf ^ 1], tid + s * kGemmThreads, rb[s]);
            }
        }
        __syncthreads();
        buf ^= 1;
    }

    gemm_epilogue<WI, WJ>(acc, C, M, N, m0, n0, tile, split, splits, wm, wn, lhi, l32, epi, part, counters, &flag);
}

// ------------------------------------------------ k-contiguous variant
//
// Same workgroup and wave tiling, but both LDS tiles are stored with k
// contiguous (As[m][k], Bs[n][k], row stride KP = 36 floats) so that one
// ds_read_b128 gives a lane the operands of four MFMAs.  The k order inside
// an 8-wide k block is permuted identically for A and B: in MFMA j of the
// block, lanes 0-31 supply k = kb + j and lanes 32-63 k = kb + 4 + j, so the
// four MFMAs still cover each k of the block exactly once.  With the stride
// of 36 floats, the 16-lane phases of a b128 read hit 16 distinct 4-bank
// groups.  The next k step's tile, already in registers, is written to the
// other LDS buffer three quarters of the way through this step's MFMAs, so
// only the barrier separates two steps.

// Staging of one operand tile (128 rows r = m or n, BK = 32 k) through
// registers into the k-contiguous LDS tile Xs[r][k].
//  * KC (stored X[R][Kd], k contiguous): slot -> row r = slot / 8, k quad
//    q = slot % 8; one 128-bit load and one 128-bit LDS write.
//  * otherwise (stored X[Kd][R]): slot -> 4 consecutive rows 4*rq.. of one
//    k; one 128-bit load along r (8 lanes cover 128 contiguous bytes) and
//    four scalar LDS writes.  The lane bits are arranged (rq low 3 bits,
//    k low 3 bits, then the high bits) so that a write instruction meets
//    at most 2-way bank conflicts with the 36-float row stride.
template <bool KC, int BKT>
struct Stage {
    static constexpr int KPT = BKT + 4;  // LDS row stride
    int r, k;  // KC: row, first k of the quad; else: first row of the quad, k
    __device__ __forceinline__ void init(int slot) {
        if constexpr (KC) {
            r = slot / (BKT / 4);
            k = (slot % (BKT / 4)) * 4;
        } else {
            r = 4 * ((slot & 7) + 8 * ((slot >> 6) & 3));
            k = ((slot >> 3) & 7) + 8 * (slot >> 8);
        }
    }
    template <bool V>
    __device__ __forceinline__ float4 load(const float *__restrict__ X, size_t r0, size_t k0, size_t R,
                                           size_t Kd) const {
        const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
        if constexpr (KC) {
            const size_t rg = r0 + r, kg = k0 + k;
            if (rg >= R) return zero;
            const float *p = X + rg * Kd + kg;
            if constexpr (V) {
                return kg < Kd ? ld4(p) : zero;  // Kd % 4 == 0: the quad is all in or all out
            } else {
                return make_float4(kg < Kd ? p[0] : 0.f, kg + 1 < Kd ? p[1] : 0.f, kg + 2 < Kd ? p[2] : 0.f,
                                   kg + 3 < Kd ? p[3] : 0.f);
            }
        } else {
            const size_t rg = r0 + r, kg = k0 + k;
            if (kg >= Kd) return zero;
            const float *p = X + kg * R + rg;
            if constexpr (V) {
                return rg < R ? ld4(p) : zero;  // R % 4 == 0
            } else {
                return make_float4(rg < R ? p[0] : 0.f, rg + 1 < R ? p[1] : 0.f, rg + 2 < R ? p[2] : 0.f,
                                   rg + 3 < R ? p[3] : 0.f);
            }
        }
    }
    __device__ __forceinline__ void store(float (*Xs)[KPT], float4 v) const {
        if constexpr (KC) {
            *reinterpret_cast<float4 *>(&Xs[r][k]) = v;
        } else {
            Xs[r + 0][k] = v.x;
            Xs[r + 1][k] = v.y;
            Xs[r + 2][k] = v.z;
            Xs[r + 3][k] = v.w;
        }
    }
};

template <bool TA, bool TB, bool VA, bool VB, int BKT, bool XCDMAP = true>
__global__ __launch_bounds__(kGemmThreads) void k_gemm_kc(const float *__restrict__ A, const float *__restrict__ B,
                                                          float *__restrict__ C, size_t M, size_t N, size_t K,
                                                          unsigned tiles_n, unsigned splits, size_t kper,
                                                          Epilogue epi, float *__restrict__ part,
                                                          unsigned *__restrict__ counters) {
    constexpr int KPT = BKT + 4;
    constexpr int SL = BM * BKT / 4 / kGemmThreads;  // staged quads per thread per operand
    constexpr int WAT = (3 * (BKT / 8)) / 4;        // LDS writes of the next tile after this many k blocks
    __shared__ float As[2][BM][KPT];
    __shared__ float Bs[2][BN][KPT];
    __shared__ int flag;
    constexpr bool KCA = !TA, KCB = TB;

    const unsigned wg = XCDMAP ? xcd_remap(blockIdx.x, gridDim.x) : blockIdx.x;
    const unsigned tile = wg / splits;
    const unsigned split = wg - tile * splits;
    const size_t m0 = static_cast<size_t>(tile / tiles_n) * BM;
    const size_t n0 = static_cast<size_t>(tile % tiles_n) * BN;
    const size_t kbeg = static_cast<size_t>(split) * kper;
    const size_t kend = kbeg + kper < K ? kbeg + kper : K;

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int wm = wave >> 2, wn = wave & 3;
    const int l32 = lane & 31, lhi = lane >> 5;

    floatx16 acc[WI][WJ];
#pragma unroll
    for (int i = 0; i < WI; ++i)
#pragma unroll
        for (int j = 0; j < WJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    Stage<KCA, BKT> sa[SL];
    Stage<KCB, BKT> sb[SL];
#pragma unroll
    for (int s = 0; s < SL; ++s) {
        sa[s].init(tid + s * kGemmThreads);
        sb[s].init(tid + s * kGemmThreads);
    }
    float4 ra[SL], rb[SL];
    int buf = 0;
    if (kbeg < kend) {
#pragma unroll
        for (int s = 0; s < SL; ++s) {
            ra[s] = sa[s].template load<VA>(A, m0, kbeg, M, K);
            rb[s] = sb[s].template load<VB>(B, n0, kbeg, N, K);
        }
#pragma unroll
        for (int s = 0; s < SL; ++s) {
            sa[s].store(As[0], ra[s]);
            sb[s].store(Bs[0], rb[s]);
        }
    }
    __syncthreads();

    for (size_t k0 = kbeg; k0 < kend; k0 += BKT) {
        const bool more = k0 + BKT < kend;
        if (more) {
#pragma unroll
            for (int s = 0; s < SL; ++s) {
                ra[s] = sa[s].template load<VA>(A, m0, k0 + BKT, M, K);
                rb[s] = sb[s].template load<VB>(B, n0, k0 + BKT, N, K);
            }
        }
        // Blocks of 8 k: one b128 per fragment, the next block's reads in
        // flight while this block's 4*WI*WJ MFMAs issue.
        float4 fa[WI], fb[WJ];
#pragma unroll
        for (int i = 0; i < WI; ++i)
            fa[i] = *reinterpret_cast<const float4 *>(&As[buf][wm * 64 + i * 32 + l32][4 * lhi]);
#pragma unroll
        for (int j = 0; j < WJ; ++j)
            fb[j] = *reinterpret_cast<const float4 *>(&Bs[buf][wn * 32 + j * 32 + l32][4 * lhi]);
#pragma unroll
        for (int kb = 0; kb < BKT / 8; ++kb) {
            float4 na[WI], nb[WJ];
            if (kb + 1 < BKT / 8) {
#pragma unroll
                for (int i = 0; i < WI; ++i)
                    na[i] = *reinterpret_cast<const float4 *>(&As[buf][wm * 64 + i * 32 + l32][8 * (kb + 1) + 4 * lhi]);
#pragma unroll
                for (int j = 0; j < WJ; ++j)
                    nb[j] = *reinterpret_cast<const float4 *>(&Bs[buf][wn * 32 + j * 32 + l32][8 * (kb + 1) + 4 * lhi]);
            }
#pragma unroll
            for (int i = 0; i < WI; ++i)
#pragma unroll
                for (int j = 0; j < WJ; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i].x, fb[j].x, acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i].y, fb[j].y, acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i].z, fb[j].z, acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i].w, fb[j].w, acc[i][j], 0, 0, 0);
                }
            if (kb + 1 == WAT && more) {
                // the other buffer was last read before the previous barrier
#pragma unroll
                for (int s = 0; s < SL; ++s) {
                    sa[s].store(As[buf ^ 1], ra[s]);
                    sb[s].store(Bs[buf ^ 1], rb[s]);
                }
            }
            if (kb + 1 < BKT / 8) {
#pragma unroll
                for (int i = 0; i < WI; ++i) fa[i] = na[i];
#pragma unroll
                for (int j = 0; j < WJ; ++j) fb[j] = nb[j];
            }
        }
        // Scheduling groups: reads of block 0, then (reads of block b+1, MFMAs of block b).
        __builtin_amdgcn_sched_group_barrier(0x100, WI + WJ, 0);
#pragma unroll
        for (int kb = 0; kb < BKT / 8; ++kb) {
            if (kb + 1 < BKT / 8) __builtin_amdgcn_sched_group_barrier(0x100, WI + WJ, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 4 * WI * WJ, 0);
            if (kb + 1 == WAT) __builtin_amdgcn_sched_group_barrier(0x200, SL * ((KCA ? 1 : 4) + (KCB ? 1 : 4)), 0);
        }
        __syncthreads();
        buf ^= 1;
    }
    gemm_epilogue<WI, WJ>(acc, C, M, N, m0, n0, tile, split, splits, wm, wn, lhi, l32, epi, part, counters, &flag);
}

// ------------------------------------------------ four waves of 64x64
//
// The k-contiguous tiles of k_gemm_kc, but a 256-thread workgroup of four
// waves (one per SIMD), each owning 64x64 of C = 2x2 MFMA tiles of 32x32
// (64 accumulator registers).  Two b128 reads of A and two of B feed 16
// MFMAs.  The next k step's tile, already in registers, is written to the
// other LDS buffer three quarters of the way through this step's MFMAs, so
// only the barrier separates two steps.
constexpr int kW4Threads = 256;

template <bool TA, bool TB, bool VA, bool VB, int BKT, bool XCDMAP = true>
__global__ __launch_bounds__(kW4Threads) void k_gemm_w4(const float *__restrict__ A, const float *__restrict__ B,
                                                        float *__restrict__ C, size_t M, size_t N, size_t K,
                                                        unsigned tiles_n, unsigned splits, size_t kper,
                                                        Epilogue epi, float *__restrict__ part,
                                                        unsigned *__restrict__ counters) {
    constexpr int KPT = BKT + 4;
    constexpr int SL = BM * BKT / 4 / kW4Threads;  // staged quads per thread per operand
    constexpr int W4I = 2, W4J = 2;
    constexpr int NB = BKT / 8;             // k blocks of 8 per step
    constexpr int WAT = (3 * NB) / 4;       // LDS writes after this many blocks
    __shared__ float As[2][BM][KPT];
    __shared__ float Bs[2][BN][KPT];
    __shared__ int flag;
    constexpr bool KCA = !TA, KCB = TB;

    const unsigned wg = XCDMAP ? xcd_remap(blockIdx.x, gridDim.x) : blockIdx.x;
    const unsigned tile = wg / splits;
    const unsigned split = wg - tile * splits;
    const size_t m0 = static_cast<size_t>(tile / tiles_n) * BM;
    const size_t n0 = static_cast<size_t>(tile % tiles_n) * BN;
    const size_t kbeg = static_cast<size_t>(split) * kper;
    const size_t kend = kbeg + kper < K ? kbeg + kper : K;

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int wm = wave >> 1, wn = wave & 1;
    const int l32 = lane & 31, lhi = lane >> 5;

    floatx16 acc[W4I][W4J];
#pragma unroll
    for (int i = 0; i < W4I; ++i)
#pragma unroll
        for (int j = 0; j < W4J; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    Stage<KCA, BKT> sa[SL];
    Stage<KCB, BKT> sb[SL];
#pragma unroll
    for (int s = 0; s < SL; ++s) {
        sa[s].init(tid + s * kW4Threads);
        sb[s].init(tid + s * kW4Threads);
    }
    float4 ra[SL], rb[SL];
    int buf = 0;
    if (kbeg < kend) {
#pragma unroll
        for (int s = 0; s < SL; ++s) {
            ra[s] = sa[s].template load<VA>(A, m0, kbeg, M, K);
            rb[s] = sb[s].template load<VB>(B, n0, kbeg, N, K);
        }
#pragma unroll
        for (int s = 0; s < SL; ++s) {
            sa[s].store(As[0], ra[s]);
            sb[s].store(Bs[0], rb[s]);
        }
    }
    __syncthreads();

    for (size_t k0 = kbeg; k0 < kend; k0 += BKT) {
        const bool more = k0 + BKT < kend;
        if (more) {
#pragma unroll
            for (int s = 0; s < SL; ++s) {
                ra[s] = sa[s].template load<VA>(A, m0, k0 + BKT, M, K);
                rb[s] = sb[s].template load<VB>(B, n0, k0 + BKT, N, K);
            }
        }
        float4 fa[W4I], fb[W4J];
#pragma unroll
        for (int i = 0; i < W4I; ++i)
            fa[i] = *reinterpret_cast<const float4 *>(&As[buf][wm * 64 + i * 32 + l32][4 * lhi]);
#pragma unroll
        for (int j = 0; j < W4J; ++j)
            fb[j] = *reinterpret_cast<const float4 *>(&Bs[buf][wn * 64 + j * 32 + l32][4 * lhi]);
#pragma unroll
        for (int kb = 0; kb < NB; ++kb) {
            float4 na[W4I], nb[W4J];
            if (kb + 1 < NB) {
#pragma unroll
                for (int i = 0; i < W4I; ++i)
                    na[i] = *reinterpret_cast<const float4 *>(&As[buf][wm * 64 + i * 32 + l32][8 * (kb + 1) + 4 * lhi]);
#pragma unroll
                for (int j = 0; j < W4J; ++j)
                    nb[j] = *reinterpret_cast<const float4 *>(&Bs[buf][wn * 64 + j * 32 + l32][8 * (kb + 1) + 4 * lhi]);
            }
#pragma unroll
            for (int i = 0; i < W4I; ++i)
#pragma unroll
                for (int j = 0; j < W4J; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i].x, fb[j].x, acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i].y, fb[j].y, acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i].z, fb[j].z, acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i].w, fb[j].w, acc[i][j], 0, 0, 0);
                }
            if (kb + 1 == WAT && more) {
                // the other buffer was last read before the previous barrier
#pragma unroll
                for (int s = 0; s < SL; ++s) {
                    sa[s].store(As[buf ^ 1], ra[s]);
                    sb[s].store(Bs[buf ^ 1], rb[s]);
                }
            }
            if (kb + 1 < NB) {
#pragma unroll
                for (int i = 0; i < W4I; ++i) fa[i] = na[i];
#pragma unroll
                for (int j = 0; j < W4J; ++j) fb[j] = nb[j];
            }
        }
        // Scheduling groups: reads of block 0; then per block the next
        // block's reads and this block's MFMAs, with the LDS writes of the
        // next tile after block WAT-1.
        __builtin_amdgcn_sched_group_barrier(0x100, W4I + W4J, 0);
#pragma unroll
        for (int kb = 0; kb < NB; ++kb) {
            if (kb + 1 < NB) __builtin_amdgcn_sched_group_barrier(0x100, W4I + W4J, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 4 * W4I * W4J, 0);
            if (kb + 1 == WAT) __builtin_amdgcn_sched_group_barrier(0x200, SL * ((KCA ? 1 : 4) + (KCB ? 1 : 4)), 0);
        }
        __syncthreads();
        buf ^= 1;
    }
    gemm_epilogue<W4I, W4J>(acc, C, M, N, m0, n0, tile, split, splits, wm, wn, lhi, l32, epi, part, counters, &flag);
}

// ------------------------------------------------ direct-to-LDS ring
// A 256-thread workgroup (four waves of 64x64, 2x2 MFMA blocks each) per
// 128x128 tile; K runs over a ring of four LDS stages of 32 k (16 KiB per
// operand), filled by direct global-to-LDS loads (lds_load16) four steps
// ahead, so three tiles are in flight while one is multiplied.  The
// stage of step t is refilled with tile t+4 right after the ring barrier
// that follows its last fragment read.  K a multiple of 8 (a split's range
// a multiple of 128 but for the last split's; the last 32-k stage runs its
// whole 8-k blocks only); a partial last tile along M or N (the
// non-k-contiguous operand's row length a multiple of 4) loads clamped rows.
// Stage layouts (16-byte chunks XOR-keyed so that fragment reads are
// conflict-free across the 64 banks):
//  * k-contiguous operand (A [M,K], B^T [N,K]): row r of 32 floats, chunk c
//    at c ^ ((r / 2) % 8); a fragment is one ds_read_b128 of 4 k;
//  * the other (A^T [K,M], B [K,N]): k row of 128 floats, chunk c at
//    c ^ 8 ((k / 4) % 2); a fragment is four ds_read_b32, lanes 0-31 on
//    consecutive columns.
// A 4-k fragment feeds four MFMAs: MFMA e takes k = 8 kb + e on lanes 0-31
// and 8 kb + 4 + e on lanes 32-63 (kb the 8-k block of the stage).
constexpr int kRingThreads = 256;
constexpr int kRBK = 32;                    // k per stage
constexpr int kRST = BM * kRBK;             // floats per operand stage
constexpr int kRPS = 2 * (kRST / 4 / kRingThreads);  // lds_load16 per wave per stage (A and B)

// Shapes the ring takes: whole 8-k blocks; a partial last M or N tile is
// clamped, which needs the [K, M] / [K, N] storage's row length a multiple
// of 4; a lane's offset within a stage (at most 127 rows, or 31 k rows, of
// the stored operand) fits 32 bits.
inline bool ring_shape_ok(const float *A, const float *B, size_t M, size_t K, size_t N, int ta, int tb) {
    constexpr size_t kMaxLd = size_t(1) << 23;
    return K % 8 == 0 && aligned16(A) && aligned16(B) && M >= 4 && N >= 4 && (!ta || M % 4 == 0) &&
           (tb || N % 4 == 0) && M < kMaxLd && N < kMaxLd && K < kMaxLd;
}

__device__ __forceinline__ int rk_c(int r) { return (r >> 1) & 7; }
__device__ __forceinline__ int rk_m(int k) { return 8 * ((k >> 2) & 1); }

// Stage fills.  A k-contiguous operand X[r][k] (ld = K) fills eight rows
// of 32 floats per instruction; the other, X[k][r] (ld = row length), two
// k rows of 128 floats.  Each load reads from a base uniform across the
// workgroup, X + r0 ld + k0 (k-contiguous) or X + k0 ld + r0, plus a
// 32-bit per-lane offset that stays fixed for the whole K loop, into an
// LDS destination computed on the scalar unit: no 64-bit vector address
// arithmetic per load.  The offsets clamp the row (k-contiguous) or
// 4-column group start (otherwise) of a partial last tile to the
// operand's last one (rlast): rows or columns past the operand's end load
// duplicates, whose products land only in accumulator rows or columns
// that the epilogue does not store.  Offsets for a stage with kv < 32
// valid k (the last tile of a split whose k range is not a multiple of
// 32) clamp k the same way, to the last 4-k group start or the last k
// row: that stage loads duplicates into 8-k blocks that are never
// multiplied (ring_last).
struct RingOffs {
    unsigned o[4];
};
template <bool KC>
__device__ __forceinline__ RingOffs ring_offsets(size_t r0, size_t ld, size_t rlast, int kv) {
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
    RingOffs f;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        if constexpr (KC) {
            const int row = w * 32 + s * 8 + (lane >> 3), p = lane & 7;
            const size_t gr = r0 + row < rlast ? r0 + row : rlast;
            const int kk = 4 * (p ^ rk_c(row));
            f.o[s] = static_cast<unsigned>(((gr - r0) * ld + (kk < kv - 4 ? kk : kv - 4)) * sizeof(float));
        } else {
            const int kr = w * 8 + s * 2 + (lane >> 5), p = lane & 31;
            const size_t gc = r0 + 4 * (p ^ rk_m(kr));
            f.o[s] = static_cast<unsigned>(((kr < kv - 1 ? kr : kv - 1) * ld + ((gc < rlast ? gc : rlast) - r0)) *
                                           sizeof(float));
        }
    }
    return f;
}
template <bool KC>
__device__ __forceinline__ void ring_fill_at(const float *__restrict__ X, size_t r0, size_t k0, size_t ld,
                                             const RingOffs &f, float *stage) {
    const unsigned w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const float *base = KC ? X + r0 * ld + k0 : X + k0 * ld + r0;
    // this wave's first LDS destination; each load fills the next 1 KiB
    const unsigned l0 = lds_addr(stage) + (KC ? w * 32 * kRBK : w * 8 * BM) * sizeof(float);
#pragma unroll
    for (int s = 0; s < 4; ++s) lds_load16_at(base, f.o[s], l0 + s * kWave * 16);
}

// A workgroup's fill offsets: whole stages (a, b) and, with TAIL, the last
// tile of the split (at, bt; equal to a, b when it is whole).
struct RingLanes {
    RingOffs a, b, at, bt;
};

// Fills stage `st` (A at +0, B at +kRST) with the 32 k from kf; kl is the
// k of the split's last tile, the only one that may be partial.
template <bool KCA, bool KCB, bool TAIL>
__device__ __forceinline__ void ring_fill_any(const float *__restrict__ A, const float *__restrict__ B, size_t lda,
                                              size_t ldb, size_t m0, size_t n0, size_t kf, size_t kl,
                                              const RingLanes &L, float *st) {
    if (!TAIL || kf != kl) {
        ring_fill_at<KCA>(A, m0, kf, lda, L.a, st);
        ring_fill_at<KCB>(B, n0, kf, ldb, L.b, st + kRST);
    } else {
        ring_fill_at<KCA>(A, m0, kf, lda, L.at, st);
        ring_fill_at<KCB>(B, n0, kf, ldb, L.bt, st + kRST);
    }
}

// Fragment of 8-k block kb for tile row (or column) `row`: k = 8 kb + 4 lhi + 0..3.
template <bool KC>
__device__ __forceinline__ float4 ring_frag(const float *stage, int row, int kb, int lhi) {
    if constexpr (KC) {
        return *reinterpret_cast<const float4 *>(stage + row * kRBK + 4 * ((2 * kb + lhi) ^ rk_c(row)));
    } else {
        const int k = 8 * kb + 4 * lhi;
        auto at = [&](int kk) { return stage[kk * BM + 4 * ((row >> 2) ^ rk_m(kk)) + (row & 3)]; };
        return make_float4(at(k), at(k + 1), at(k + 2), at(k + 3));
    }
}

struct RingFrag {
    float4 a[2], b[2];
};

template <bool KCA, bool KCB>
__device__ __forceinline__ void ring_frags(const float *st, int kb, int wm, int wn, int l32, int lhi, RingFrag &f) {
#pragma unroll
    for (int i = 0; i < 2; ++i) f.a[i] = ring_frag<KCA>(st, wm * 64 + i * 32 + l32, kb, lhi);
#pragma unroll
    for (int j = 0; j < 2; ++j) f.b[j] = ring_frag<KCB>(st + kRST, wn * 64 + j * 32 + l32, kb, lhi);
}

__device__ __forceinline__ float comp(const float4 &v, int e) { return e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w; }

// The 16 MFMAs of one 8-k block, with the next block's fragment reads
// scheduled between them.
template <bool KCA, bool KCB>
__device__ __forceinline__ void ring_block(const RingFrag &f, floatx16 (&acc)[2][2]) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(comp(f.a[i], e), comp(f.b[j], e), acc[i][j], 0, 0, 0);
    constexpr int ND = (KCA ? 2 : 8) + (KCB ? 2 : 8);
#pragma unroll
    for (int t = 0; t < ND; ++t) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 16 - ND, 0);
}

// Step on stage cur (tile t; A at +0, B at +kRST); nxt holds tile t+1; f0
// holds block 0 of cur on entry and block 0 of nxt on return.
template <bool KCA, bool KCB, bool TAIL>
__device__ __forceinline__ void ring_step(const float *__restrict__ A, const float *__restrict__ B, size_t lda,
                                          size_t ldb, size_t m0, size_t n0, size_t kf, size_t kl, float *cur,
                                          const float *nxt, RingFrag &f0, floatx16 (&acc)[2][2], int wm, int wn,
                                          int l32, int lhi, const RingLanes &L) {
    RingFrag f1, f2;
    ring_frags<KCA, KCB>(cur, 1, wm, wn, l32, lhi, f1);
    ring_block<KCA, KCB>(f0, acc);
    ring_frags<KCA, KCB>(cur, 2, wm, wn, l32, lhi, f2);
    ring_block<KCA, KCB>(f1, acc);
    ring_frags<KCA, KCB>(cur, 3, wm, wn, l32, lhi, f1);
    ring_block<KCA, KCB>(f2, acc);
    ring_barrier<2 * kRPS>();  // tile t+1 landed; every wave done reading cur
    ring_frags<KCA, KCB>(nxt, 0, wm, wn, l32, lhi, f0);
    ring_fill_any<KCA, KCB, TAIL>(A, B, lda, ldb, m0, n0, kf, kl, L, cur);
    ring_block<KCA, KCB>(f1, acc);
}

// The last k tile, on stage cur (landed; f0 holds its block 0): its first
// nb 8-k blocks only (1 <= nb <= 4), no refill.
template <bool KCA, bool KCB>
__device__ __forceinline__ void ring_last(const float *cur, const RingFrag &f0, int nb, floatx16 (&acc)[2][2], int wm,
                                          int wn, int l32, int lhi) {
    ring_block<KCA, KCB>(f0, acc);
    for (int kb = 1; kb < nb; ++kb) {  // nb is uniform
        RingFrag f;
        ring_frags<KCA, KCB>(cur, kb, wm, wn, l32, lhi, f);
        ring_block<KCA, KCB>(f, acc);
    }
}

// Same arguments as k_gemm.  KCA: A stored [M,K] (else [K,M]); KCB: B stored
// [N,K] (else [K,N]).  TAIL: a split's k range may end in a partial 32-k
// stage (K not a multiple of 128).  A separate instance: the tail's extra
// steps and clamps, compiled into the one loop, moved the accumulators'
// neighbours into AGPRs and slowed every whole-stage product by 2-3 us.
template <bool KCA, bool KCB, bool TAIL>
__device__ __forceinline__ void ring_gemm(const float *__restrict__ A, const float *__restrict__ B,
                                          float *__restrict__ C, size_t M, size_t N, size_t K, unsigned tiles_n,
                                          unsigned splits, size_t kper, const Epilogue &epi,
                                          float *__restrict__ part, unsigned *__restrict__ counters, unsigned wg) {
    __shared__ __attribute__((aligned(16))) float s0[2 * kRST], s1[2 * kRST], s2[2 * kRST], s3[2 * kRST];
    __shared__ int flag;
    constexpr unsigned tl_kind = TAIL ? 0u : (KCA && !KCB) ? 1u : (KCA && KCB) ? 2u : 3u;
    gemm_tl_mark(tl_kind, 0);
    const unsigned tile = wg / splits;
    const unsigned split = wg - tile * splits;
    const size_t m0 = static_cast<size_t>(tile / tiles_n) * BM;
    const size_t n0 = static_cast<size_t>(tile % tiles_n) * BN;
    const size_t kbeg = static_cast<size_t>(split) * kper;
    const size_t kend = kbeg + kper < K ? kbeg + kper : K;
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int wm = wave >> 1, wn = wave & 1, l32 = lane & 31, lhi = lane >> 5;
    const size_t lda = KCA ? K : M, ldb = KCB ? K : N;
    const size_t ra = KCA ? M - 1 : M - 4, rb = KCB ? N - 1 : N - 4;  // ring_offsets' row clamps

    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // (kend - kbeg) % 8 == 0 (% 128 == 0 without TAIL): tiles 0..T-1 of 32
    // k, the last with nb 8-k blocks.  Tiles beyond T-1 reload tile T-1
    // into stages whose fragments go unused.
    const size_t len = kend - kbeg, T = (len + kRBK - 1) / kRBK;
    auto kt = [&](size_t t) { return kbeg + (t < T ? t : T - 1) * kRBK; };
    const size_t kl = kt(T - 1);
    RingLanes L;
    L.a = ring_offsets<KCA>(m0, lda, ra, kRBK);
    L.b = ring_offsets<KCB>(n0, ldb, rb, kRBK);
    if constexpr (TAIL) {
        const int kv = static_cast<int>(len - (T - 1) * kRBK);  // 8..32
        L.at = ring_offsets<KCA>(m0, lda, ra, kv);
        L.bt = ring_offsets<KCB>(n0, ldb, rb, kv);
    }
    ring_fill_any<KCA, KCB, TAIL>(A, B, lda, ldb, m0, n0, kt(0), kl, L, s0);
    ring_fill_any<KCA, KCB, TAIL>(A, B, lda, ldb, m0, n0, kt(1), kl, L, s1);
    ring_fill_any<KCA, KCB, TAIL>(A, B, lda, ldb, m0, n0, kt(2), kl, L, s2);
    ring_fill_any<KCA, KCB, TAIL>(A, B, lda, ldb, m0, n0, kt(3), kl, L, s3);
    ring_barrier<3 * kRPS>();
    gemm_tl_mark(tl_kind, 1);
    RingFrag f0;
    ring_frags<KCA, KCB>(s0, 0, wm, wn, l32, lhi, f0);
#define CXM_RING_STEP(T4, CUR, NXT) \
    ring_step<KCA, KCB, TAIL>(A, B, lda, ldb, m0, n0, kt(T4), kl, CUR, NXT, f0, acc, wm, wn, l32, lhi, L)
    if constexpr (!TAIL) {
        for (size_t t = 0; t < T; t += 4) {  // T is a multiple of 4
            CXM_RING_STEP(t + 4, s0, s1);
            CXM_RING_STEP(t + 5, s1, s2);
            CXM_RING_STEP(t + 6, s2, s3);
            CXM_RING_STEP(t + 7, s3, s0);
        }
    } else {
        const int nb = static_cast<int>((len - (T - 1) * kRBK) / 8);
        size_t t = 0;
        for (; t + 4 < T; t += 4) {
            CXM_RING_STEP(t + 4, s0, s1);
            CXM_RING_STEP(t + 5, s1, s2);
            CXM_RING_STEP(t + 6, s2, s3);
            CXM_RING_STEP(t + 7, s3, s0);
        }
        // tiles t .. T-1 remain (one to four), tile t on s0
        const size_t rem = T - t;
        if (rem == 1) {
            ring_last<KCA, KCB>(s0, f0, nb, acc, wm, wn, l32, lhi);
        } else {
            CXM_RING_STEP(t + 4, s0, s1);
            if (rem == 2) {
                ring_last<KCA, KCB>(s1, f0, nb, acc, wm, wn, l32, lhi);
            } else {
                CXM_RING_STEP(t + 5, s1, s2);
                if (rem == 3) {
                    ring_last<KCA, KCB>(s2, f0, nb, acc, wm, wn, l32, lhi);
                } else {
                    CXM_RING_STEP(t + 6, s2, s3);
                    ring_last<KCA, KCB>(s3, f0, nb, acc, wm, wn, l32, lhi);
                }
            }
        }
    }
#undef CXM_RING_STEP
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no load into LDS outlives the workgroup
    gemm_tl_mark(tl_kind, 2);
    gemm_epilogue<2, 2>(acc, C, M, N, m0, n0, tile, split, splits, wm, wn, lhi, l32, epi, part, counters, &flag);
#ifdef CXM_TIMELINE
    __syncthreads();
    gemm_tl_mark(tl_kind, 3);
#endif
}

template <bool KCA, bool KCB, bool TAIL>
__global__ __launch_bounds__(kRingThreads) void k_gemm_ring(const float *__restrict__ A, const float *__restrict__ B,
                                                            float *__restrict__ C, size_t M, size_t N, size_t K,
                                                            unsigned tiles_n, unsigned splits, size_t kper,
                                                            Epilogue epi, float *__restrict__ part,
                                                            unsigned *__restrict__ counters) {
    ring_gemm<KCA, KCB, TAIL>(A, B, C, M, N, K, tiles_n, splits, kper, epi, part, counters,
                              xcd_remap(blockIdx.x, gridDim.x));
}

// Two independent ring products in one launch (the MLP's two weight
// gradients): workgroups [0, g0.wgs) run the first, the rest the second,
// each with its own tile order, split-K partials and tickets.  The second
// product's workgroups start on the CUs the first one's release, with no
// drain and refill of the chip between them.
struct RingArgs {
    const float *A, *B;
    float *C;
    size_t M, N, K;
    unsigned tiles_n, splits;
    size_t kper;
    Epilogue epi;
    float *part;
    unsigned *counters;
    unsigned wgs;  // workgroups of this product (a multiple of 8 for the XCD order, else dispatch order)
};
template <bool KCA, bool KCB>
__global__ __launch_bounds__(kRingThreads) void k_gemm_ring_pair(RingArgs g0, RingArgs g1, StepSide side) {
    if (blockIdx.x >= g0.wgs + g1.wgs) {  // dispatched after every product workgroup: the free CUs
        __shared__ float slds[16][64];
        step_side(side, blockIdx.x - g0.wgs - g1.wgs, slds);
        return;
    }
    const bool second = blockIdx.x >= g0.wgs;
    const RingArgs &g = second ? g1 : g0;
    const unsigned b = second ? blockIdx.x - g0.wgs : blockIdx.x;
    ring_gemm<KCA, KCB, false>(g.A, g.B, g.C, g.M, g.N, g.K, g.tiles_n, g.splits, g.kper, g.epi, g.part, g.counters,
                               xcd_remap(b, g.wgs));
}

// ------------------------------------------------ skinny products
// Products with a dimension of at most 16 (the 10-class output layer of
// the MLP) leave a 128x128 MFMA tile almost empty; they are bandwidth
// work and get their own kernels (plain fp32 fma, fixed order per lane,
// then a fixed tree).

constexpr int kThin = 16;

// NN with N <= 16 and K <= 1024 (K % 4 == 0): B is staged once per
// workgroup through LDS (as B^T, [NC][K]) into registers (lane l holds
// B[k][0..NC-1] for its 16 k = 256u + 4l + j, NC = N rounded up to 4, zero
// past N), so a row costs its A loads and FMAs only; reading all of B^T from
// LDS per row moved 10x the bytes of A through LDS and ran 20 us at
// 4096 x 1024 x 10.
// A 256-thread workgroup takes 16 rows, four per wave, every row's loads
// issued before any FMA; each output is a fixed-order fma chain per lane,
// then a wave reduction per column.
constexpr int kThinNNT = 256;  // threads of the N <= 16 kernel
constexpr int kThinNT = 1024;  // threads of the K <= 16 kernel
constexpr int kThinRPW = 4;  // rows per wave

template <int NC>
__global__ __launch_bounds__(kThinNNT) void k_gemm_thin_n(const float *__restrict__ A, const float *__restrict__ B,
                                                        float *__restrict__ C, size_t M, size_t N, size_t K,
                                                        Epilogue epi) {
    extern __shared__ float Bs[];  // [NC][K]: B^T, rows past N zero
    for (size_t k = threadIdx.x; k < K; k += kThinNNT) {
        float t[NC];  // the row's loads issued before its stores
#pragma unroll
        for (int n = 0; n < NC; ++n) t[n] = n < static_cast<int>(N) ? B[k * N + n] : 0.0f;
#pragma unroll
        for (int n = 0; n < NC; ++n) Bs[n * K + k] = t[n];
    }
    __syncthreads();
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
    float4 breg[4][NC];  // [u][n]: B[256u + 4 lane + 0..3][n], one conflict-free ds_read_b128 each
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const size_t k = 256 * u + 4 * lane;
#pragma unroll
        for (int n = 0; n < NC; ++n)
            breg[u][n] = k < K ? *reinterpret_cast<const float4 *>(&Bs[n * K + k]) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const size_t i0 = (static_cast<size_t>(blockIdx.x) * (kThinNNT / kWave) + w) * kThinRPW;
    float4 a[kThinRPW][4];
#pragma unroll
    for (int r = 0; r < kThinRPW; ++r)
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const size_t k = 256 * u + 4 * lane;
            a[r][u] = (i0 + r < M && k < K) ? ld4(A + (i0 + r) * K + k) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
    for (int r = 0; r < kThinRPW; ++r) {
        if (i0 + r >= M) break;  // wave-uniform
        float acc[NC];
#pragma unroll
        for (int n = 0; n < NC; ++n) {
            float t = 0.0f;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                t = __builtin_fmaf(a[r][u].x, breg[u][n].x, t);
                t = __builtin_fmaf(a[r][u].y, breg[u][n].y, t);
                t = __builtin_fmaf(a[r][u].z, breg[u][n].z, t);
                t = __builtin_fmaf(a[r][u].w, breg[u][n].w, t);
            }
            acc[n] = wave_reduce<SumOp>(t);
        }
        if (lane < static_cast<int>(N)) {
            float v = 0.0f;
#pragma unroll
            for (int n = 0; n < NC; ++n) v = lane == n ? acc[n] : v;
            store_epi(epi, C, i0 + r, lane, N, v);
        }
    }
}

// TN with N <= 16: C[m, n] = sum_k A[k, m] * B[k, n], A stored [K, M]
// (M % 4 == 0), B stored [K, N].  Pass 1: a workgroup takes 256 columns of
// m (float4 per lane) and a chunk of k; its 4 waves take interleaved k and
// meet in LDS; the chunk's sums go to the workspace.  Pass 2: one thread
// per output adds the chunks in order and applies the epilogue.  (A
// last-workgroup combine here would make one workgroup read all
// chunks x 256 x N partials, tens of microseconds of serial latency.)
__global__ __launch_bounds__(kBlock) void k_gemm_thin_tn(const float *__restrict__ A, const float *__restrict__ B,
                                                        size_t M, size_t N, size_t K, unsigned ntiles, size_t kpc,
                                                        float *__restrict__ part) {
    __shared__ float lds[kWavesPerBlock][kThin][kColTileThin];
    const unsigned tile = blockIdx.x % ntiles, chunk = blockIdx.x / ntiles;
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave, tid = threadIdx.x;
    const size_t m = static_cast<size_t>(tile) * kColTileThin + lane * 4;
    const size_t k0 = static_cast<size_t>(chunk) * kpc, k1 = k0 + kpc < K ? k0 + kpc : K;
    float acc[4][kThin];
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int n = 0; n < kThin; ++n) acc[c][n] = 0.0f;
    if (m < M) {
        constexpr int U = 4;  // rows of loads in flight per wave
        for (size_t k = k0 + w; k < k1; k += U * kWavesPerBlock) {
            float4 a[U];
            float b[U][kThin];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const size_t kk = k + u * kWavesPerBlock;
                const bool in = kk < k1;
                a[u] = in ? ld4(A + kk * M + m) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                for (int n = 0; n < kThin; ++n) b[u][n] = (in && n < static_cast<int>(N)) ? B[kk * N + n] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int n = 0; n < kThin; ++n) {
                    acc[0][n] = __builtin_fmaf(a[u].x, b[u][n], acc[0][n]);
                    acc[1][n] = __builtin_fmaf(a[u].y, b[u][n], acc[1][n]);
                    acc[2][n] = __builtin_fmaf(a[u].z, b[u][n], acc[2][n]);
                    acc[3][n] = __builtin_fmaf(a[u].w, b[u][n], acc[3][n]);
                }
        }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int n = 0; n < kThin; ++n) lds[w][n][lane * 4 + c] = acc[c][n];
    __syncthreads();
    // part[chunk][n][m]: column tile*256 + tid, waves combined in order
    float *dst = part + static_cast<size_t>(chunk) * kThin * M + static_cast<size_t>(tile) * kColTileThin + tid;
    if (static_cast<size_t>(tile) * kColTileThin + tid < M)
#pragma unroll
        for (int n = 0; n < kThin; ++n)
            dst[static_cast<size_t>(n) * M] = (lds[0][n][tid] + lds[1][n][tid]) + (lds[2][n][tid] + lds[3][n][tid]);
}

__global__ __launch_bounds__(kBlock) void k_gemm_thin_tn_sum(const float *__restrict__ part, float *__restrict__ C,
                                                            size_t M, size_t N, unsigned chunks, Epilogue epi) {
    const size_t q = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;  // q = n * M + m
    if (q >= N * M) return;
    const size_t n = q / M, m = q - n * M;
    float v = 0.0f;
    unsigned c = 0;
    for (; c + 16 <= chunks; c += 16) {
        float t[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) t[u] = part[(static_cast<size_t>(c + u) * kThin + n) * M + m];
#pragma unroll
        for (int u = 0; u < 16; ++u) v = v + t[u];
    }
    for (; c < chunks; ++c) v = v + part[(static_cast<size_t>(c) * kThin + n) * M + m];
    store_epi(epi, C, m, n, N, v);
}

// Small K (<= 16), A [M, K] row-major: every output is a K-term dot
// product, so this streams C (and the gate).  The workgroup's K x 1024
// panel of B is staged in LDS once; thread t keeps the K x 4 fragment of
// columns j0 + 4*(t % 256) in registers and takes rows r0 + t/256 + 4i of
// the workgroup's 16, all four rows' loads issued together.
constexpr int kThinCols = 1024;
constexpr int kThinRows = 16;

template <bool TB>
__global__ __launch_bounds__(kThinNT) void k_gemm_thin_k(const float *__restrict__ A, const float *__restrict__ B,
                                                        float *__restrict__ C, size_t M, size_t N, size_t K,
                                                        Epilogue epi) {
    __shared__ float Bs[kThin][kThinCols];
    const size_t j0 = static_cast<size_t>(blockIdx.x) * kThinCols;
    {
        const size_t j = j0 + threadIdx.x;
        float t[kThin];  // all loads issued before any store
#pragma unroll
        for (int k = 0; k < kThin; ++k)
            t[k] = (k < static_cast<int>(K) && j < N) ? (TB ? B[j * K + k] : B[k * N + j]) : 0.0f;
#pragma unroll
        for (int k = 0; k < kThin; ++k) Bs[k][threadIdx.x] = t[k];
    }
    __syncthreads();
    const int ct = threadIdx.x % 256, rg = threadIdx.x / 256;
    const size_t j = j0 + 4 * ct;
    if (j >= N) return;  // no barrier follows
    float bf[kThin][4];
#pragma unroll
    for (int k = 0; k < kThin; ++k)
#pragma unroll
        for (int c = 0; c < 4; ++c) bf[k][c] = Bs[k][4 * ct + c];
    const bool vec = j + 3 < N && !epi.sgd && !epi.bias && aligned16(C) && N % 4 == 0 &&
                     (!epi.gate || aligned16(epi.gate));
    const size_t r0 = static_cast<size_t>(blockIdx.y) * kThinRows + rg;
    float4 g[4];  // the four rows' gate loads go out together
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const size_t r = r0 + 4 * i;
        g[i] = (vec && epi.gate && r < M) ? ld4(epi.gate + r * N + j) : make_float4(1.f, 1.f, 1.f, 1.f);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        // the row index is the same in the whole wave: keep A's row in scalar registers
        const int r = __builtin_amdgcn_readfirstlane(static_cast<int>(r0 + 4 * i));
        if (static_cast<size_t>(r) >= M) break;
        const float *__restrict__ ar = A + static_cast<size_t>(r) * K;
        float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < kThin; ++k) {
            const float a = k < static_cast<int>(K) ? ar[k] : 0.0f;
#pragma unroll
            for (int c = 0; c < 4; ++c) o[c] = __builtin_fmaf(a, bf[k][c], o[c]);
        }
        if (vec) {
            float4 v = make_float4(o[0], o[1], o[2], o[3]);
            if (epi.act == CXM_ACT_RELU) {
                v.x = 0.0f > v.x ? 0.0f : v.x; v.y = 0.0f > v.y ? 0.0f : v.y;
                v.z = 0.0f > v.z ? 0.0f : v.z; v.w = 0.0f > v.w ? 0.0f : v.w;
            }
            if (epi.gate) {
                v.x = v.x * (g[i].x > 0.0f ? 1.0f : 0.0f); v.y = v.y * (g[i].y > 0.0f ? 1.0f : 0.0f);
                v.z = v.z * (g[i].z > 0.0f ? 1.0f : 0.0f); v.w = v.w * (g[i].w > 0.0f ? 1.0f : 0.0f);
            }
            st4(C + static_cast<size_t>(r) * N + j, v);
        } else {
#pragma unroll
            for (int c = 0; c < 4; ++c)
                if (j + c < N) store_epi(epi, C, r, j + c, N, o[c]);
        }
    }
}

// Kernel variant per launch.  -1 (the default) chooses by shape;
// cxm_gemm_f32_kernel pins one for tests and tuning: 0 k-major, 1/2
// k-contiguous with BK 32/64, 3/4 four-wave with BK 32/64, 5 k-contiguous
// without the XCD renumbering, 6 k-major with it, 7 the direct-to-LDS ring
// (where its shape conditions hold, else 1).
std::atomic<int> g_gemm_kc{-1};

// Measured on gfx950 (TFLOP/s, best variant vs the others):
//  * grids of >= 1024 workgroups (8192^3, 4096^3): four waves of 64x64, BK 32
//    (125 / 115 against <= 116 / 113);
//  * A^T B (the MLP's weight gradients, split K): k-major tiles with the XCD
//    renumbering (97.5 and 77 against 87-89 and 70-75);
//  * A B and A B^T at 256-tile grids: k-contiguous tiles, BK 32, with the
//    renumbering (93 and 104 against 90 and 94 for the k-major kernel).
//  * the ring (M, N, K multiples of 128, 16-byte aligned bases) for A B,
//    A B^T and A^T B: 99-100 against 92-95 at 4096x1024x1024, 133 against
//    113 at 4096^3, 135 against 125 at 8192^3; A^T B with K split four ways
//    (1024x4096x1024) 3-8% faster than the k-major kernel in interleaved
//    runs.
inline int gemm_variant(bool ta, bool tb, unsigned wgs, bool ring_ok) {
    const int pinned = g_gemm_kc.load(std::memory_order_relaxed);
    if (pinned == 7) return ring_ok ? 7 : 1;
    if (pinned >= 0) return pinned;
    if (ring_ok && !(ta && tb)) return 7;
    if (wgs >= 1024) return 3;
    if (ta && !tb) return 6;
    return 1;
}

template <bool TA, bool TB>
int launch_t(const float *A, const float *B, float *C, size_t M, size_t N, size_t K, bool va, bool vb,
             dim3 grid, unsigned tiles_n, unsigned splits, size_t kper, Epilogue epi, float *part,
             unsigned *counters, hipStream_t s, int variant) {
    if (variant == 7) {
        if (K % (4 * kRBK) == 0)
            hipLaunchKernelGGL((k_gemm_ring<!TA, TB, false>), grid, dim3(kRingThreads), 0, s, A, B, C, M, N, K, tiles_n,
                               splits, kper, epi, part, counters);
        else
            hipLaunchKernelGGL((k_gemm_ring<!TA, TB, true>), grid, dim3(kRingThreads), 0, s, A, B, C, M, N, K, tiles_n,
                               splits, kper, epi, part, counters);
        return launch_status();
    }
#define CXM_GEMM_LAUNCH(VA_, VB_)                                                                  \
    if (variant == 5)                                                                              \
        hipLaunchKernelGGL((k_gemm_kc<TA, TB, VA_, VB_, 32, false>), grid, dim3(kGemmThreads), 0, s, A, B, C, M, N, \
                           K, tiles_n, splits, kper, epi, part, counters);                        \
    else if (variant == 6)                                                                         \
        hipLaunchKernelGGL((k_gemm<TA, TB, VA_, VB_, true>), grid, dim3(kGemmThreads), 0, s, A, B, C, M, N, K,     \
                           tiles_n, splits, kper, epi, part, counters);                           \
    else if (variant == 3)                                                                         \
        hipLaunchKernelGGL((k_gemm_w4<TA, TB, VA_, VB_, 32>), grid, dim3(kW4Threads), 0, s, A, B, C, M, N, K, \
                           tiles_n, splits, kper, epi, part, counters);                           \
    else if (variant == 4)                                                                         \
        hipLaunchKernelGGL((k_gemm_w4<TA, TB, VA_, VB_, 64>), grid, dim3(kW4Threads), 0, s, A, B, C, M, N, K, \
                           tiles_n, splits, kper, epi, part, counters);                           \
    else if (variant == 2)                                                                         \
        hipLaunchKernelGGL((k_gemm_kc<TA, TB, VA_, VB_, 64>), grid, dim3(kGemmThreads), 0, s, A, B, C, M, N, K, \
                           tiles_n, splits, kper, epi, part, counters);                           \
    else if (variant == 1)                                                                         \
        hipLaunchKernelGGL((k_gemm_kc<TA, TB, VA_, VB_, 32>), grid, dim3(kGemmThreads), 0, s, A, B, C, M, N, K, \
                           tiles_n, splits, kper, epi, part, counters);                           \
    else                                                                                           \
        hipLaunchKernelGGL((k_gemm<TA, TB, VA_, VB_>), grid, dim3(kGemmThreads), 0, s, A, B, C, M, N, K, tiles_n, \
                           splits, kper, epi, part, counters)
    if (va && vb) CXM_GEMM_LAUNCH(true, true);
    else if (va) CXM_GEMM_LAUNCH(true, false);
    else if (vb) CXM_GEMM_LAUNCH(false, true);
    else CXM_GEMM_LAUNCH(false, false);
#undef CXM_GEMM_LAUNCH
    return launch_status();
}

// Thin products; returns 1 when the shape has no thin kernel.
int gemm_thin(const float *A, const float *B, float *C, size_t M, size_t K, size_t N, int ta, int tb,
              const Epilogue &epi, cxm_stream_t st) {
    hipStream_t s = reinterpret_cast<hipStream_t>(st);
    if (N <= kThin && !tb && !ta && K % 4 == 0 && K <= 1024 && aligned16(A)) {
        const dim3 grid(ceil_div(M, kThinNNT / kWave * kThinRPW));
        const size_t nc = (N + 3) / 4 * 4, lds = K * nc * sizeof(float);
        if (nc == 4) hipLaunchKernelGGL(k_gemm_thin_n<4>, grid, dim3(kThinNNT), lds, s, A, B, C, M, N, K, epi);
        else if (nc == 8) hipLaunchKernelGGL(k_gemm_thin_n<8>, grid, dim3(kThinNNT), lds, s, A, B, C, M, N, K, epi);
        else if (nc == 12) hipLaunchKernelGGL(k_gemm_thin_n<12>, grid, dim3(kThinNNT), lds, s, A, B, C, M, N, K, epi);
        else hipLaunchKernelGGL(k_gemm_thin_n<16>, grid, dim3(kThinNNT), lds, s, A, B, C, M, N, K, epi);
        return launch_status();
    }
    if (N <= kThin && !tb && ta && M % 4 == 0 && aligned16(A)) {
        const size_t ntiles = (M + kColTileThin - 1) / kColTileThin;
        size_t chunks = (256 + ntiles - 1) / ntiles;
        const size_t max_chunks = (K + 15) / 16;
        if (chunks > max_chunks) chunks = max_chunks;
        if (chunks < 1) chunks = 1;
        const size_t kpc = (K + chunks - 1) / chunks;
        chunks = (K + kpc - 1) / kpc;
        if (ntiles * chunks > 0x7fffffffu || N * M > 0x7fffffffu) return 1;
        Workspace ws;
        int rc = get_workspace(st, 0, chunks * kThin * M * sizeof(float), &ws);
        if (rc) return rc;
        float *part = static_cast<float *>(ws.scratch);
        hipLaunchKernelGGL(k_gemm_thin_tn, dim3(static_cast<unsigned>(ntiles * chunks)), dim3(kBlock), 0, s, A, B, M,
                           N, K, static_cast<unsigned>(ntiles), kpc, part);
        if ((rc = launch_status())) return rc;
        hipLaunchKernelGGL(k_gemm_thin_tn_sum, dim3(ceil_div(N * M, kBlock)), dim3(kBlock), 0, s, part, C, M, N,
                           static_cast<unsigned>(chunks), epi);
        return launch_status();
    }
    if (K <= kThin && !ta && N >= 64 && M < 0x7fffffffu) {
        const size_t tiles = (N + kThinCols - 1) / kThinCols;
        const size_t chunks = (M + kThinRows - 1) / kThinRows;
        if (chunks > 0x7fffffffu || tiles > 65535) return 1;
        const dim3 grid(static_cast<unsigned>(tiles), static_cast<unsigned>(chunks));
        if (tb) hipLaunchKernelGGL(k_gemm_thin_k<true>, grid, dim3(kThinNT), 0, s, A, B, C, M, N, K, epi);
        else hipLaunchKernelGGL(k_gemm_thin_k<false>, grid, dim3(kThinNT), 0, s, A, B, C, M, N, K, epi);
        return launch_status();
    }
    return 1;
}

}  // namespace

int gemm_ex(const float *A, const float *B, float *C, size_t M, size_t K, size_t N, int ta, int tb,
            const Epilogue &epi, cxm_stream_t st) {
    if (!A || !B || !C || (epi.act != CXM_ACT_NONE && epi.act != CXM_ACT_RELU)) return CXM_E_INVALID;
    if (M == 0 || N == 0) return CXM_OK;
    if (K == 0) return CXM_E_INVALID;
    {
        const int t = gemm_thin(A, B, C, M, K, N, ta, tb, epi, st);
        if (t != 1) return t;
    }
    const size_t tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    const size_t tiles = tiles_m * tiles_n;
    // Split K when the tile grid alone cannot fill the chip's CUs (256 here);
    // each split keeps at least 256 of K.
    size_t splits = 1;
    // (at most one workgroup per CU: one 8-wave workgroup fills a CU, and
    // one more would run as a second round)
    const size_t cus = device_cus();
    if (tiles < cus * 3 / 4 && K >= 512) {
        splits = cus / tiles;
        const size_t max_splits = K / 256;
        if (splits > max_splits) splits = max_splits;
        if (splits < 1) splits = 1;
    }
    // a split's k range is a whole number of the kernel's k steps (the
    // ring's: four stages of 32)
    // the ring: whole 8-k blocks; a partial last M or N tile is clamped,
    // which needs the [K, M] / [K, N] storage's row length a multiple of 4;
    // its lanes address a stage with 32-bit byte offsets (ring_offsets)
    const bool ring_ok = ring_shape_ok(A, B, M, K, N, ta, tb);
    const int variant = gemm_variant(ta, tb, static_cast<unsigned>(tiles * splits), ring_ok);
    const size_t kstep = variant == 7 ? 4 * kRBK : (variant == 2 || variant == 4) ? 64 : BK;
    size_t kper = (K + splits - 1) / splits;
    kper = (kper + kstep - 1) / kstep * kstep;
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
    const dim3 grid(static_cast<unsigned>(tiles * splits));
    hipStream_t s = reinterpret_cast<hipStream_t>(st);
    const unsigned tn = static_cast<unsigned>(tiles_n), sp = static_cast<unsigned>(splits);
    if (!ta && !tb) return launch_t<false, false>(A, B, C, M, N, K, va, vb, grid, tn, sp, kper, epi, part, counters, s, variant);
    if (ta && !tb) return launch_t<true, false>(A, B, C, M, N, K, va, vb, grid, tn, sp, kper, epi, part, counters, s, variant);
    if (!ta && tb) return launch_t<false, true>(A, B, C, M, N, K, va, vb, grid, tn, sp, kper, epi, part, counters, s, variant);
    return launch_t<true, true>(A, B, C, M, N, K, va, vb, grid, tn, sp, kper, epi, part, counters, s, variant);
}

namespace {

// The split plan gemm_ex uses for a ring product (see above): the ring at
// its whole-stage instance, the split count and each split's k range.
// Returns false when gemm_ex would not run this shape on that instance.
bool ring_plan(const float *A, const float *B, size_t M, size_t K, size_t N, int ta, int tb, size_t *tiles,
               size_t *tiles_n, size_t *splits, size_t *kper) {
    if (M == 0 || N == 0 || K == 0 || K % (4 * kRBK) != 0 || (ta && tb)) return false;
    if (N <= kThin || K <= kThin) return false;  // thin kernels
    const bool ring_ok = ring_shape_ok(A, B, M, K, N, ta, tb);
    const size_t tm = (M + BM - 1) / BM, tn = (N + BN - 1) / BN, t = tm * tn;
    size_t sp = 1;
    const size_t cus = device_cus();
    if (t < cus * 3 / 4 && K >= 512) {
        sp = cus / t;
        const size_t max_splits = K / 256;
        if (sp > max_splits) sp = max_splits;
        if (sp < 1) sp = 1;
    }
    if (gemm_variant(ta, tb, static_cast<unsigned>(t * sp), ring_ok) != 7) return false;
    size_t kp = (K + sp - 1) / sp;
    kp = (kp + 4 * kRBK - 1) / (4 * kRBK) * (4 * kRBK);
    sp = (K + kp - 1) / kp;
    if (kp % (4 * kRBK) != 0 || t * sp > 0x7fffffffu) return false;
    *tiles = t;
    *tiles_n = tn;
    *splits = sp;
    *kper = kp;
    return true;
}

// Re-plans a ring product's K split at `sp` splits: each split's k range a
// whole number of ring stages.
bool ring_resplit(size_t K, size_t sp, size_t *splits, size_t *kper) {
    size_t kp = (K + sp - 1) / sp;
    kp = (kp + 4 * kRBK - 1) / (4 * kRBK) * (4 * kRBK);
    if (kp == 0 || kp % (4 * kRBK) != 0) return false;
    *kper = kp;
    *splits = (K + kp - 1) / kp;
    return true;
}

}  // namespace

int gemm_ex_pair(const GemmSpec &a, const GemmSpec &b, cxm_stream_t st, StepSide *side) {
    size_t ta_t, ta_n, ta_s, ta_k, tb_t, tb_n, tb_s, tb_k;
    StepSide none{};
    if (side) side->wgs = 0;
    if (!a.A || !a.B || !a.C || !b.A || !b.B || !b.C || a.ta != b.ta || a.tb != b.tb) return 1;
    if (a.epi.act != CXM_ACT_NONE && a.epi.act != CXM_ACT_RELU) return 1;
    if (b.epi.act != CXM_ACT_NONE && b.epi.act != CXM_ACT_RELU) return 1;
    if (!ring_plan(a.A, a.B, a.M, a.K, a.N, a.ta, a.tb, &ta_t, &ta_n, &ta_s, &ta_k)) return 1;
    if (!ring_plan(b.A, b.B, b.M, b.K, b.N, b.ta, b.tb, &tb_t, &tb_n, &tb_s, &tb_k)) return 1;
    // Each plan alone fills the chip; together they would run as two rounds
    // of workgroups, each paying the ring's fill and epilogue.  One split
    // count for both that keeps the pair within one round instead (one ring
    // workgroup, 128 KiB of LDS, per CU).
    const size_t cus = device_cus();
    if (ta_t * ta_s + tb_t * tb_s > cus) {
        const size_t sp = std::max<size_t>(1, cus / (ta_t + tb_t));
        if (!ring_resplit(a.K, sp, &ta_s, &ta_k) || !ring_resplit(b.K, sp, &tb_s, &tb_k)) return 1;
    }
    const size_t wa = ta_t * ta_s, wb = tb_t * tb_s;
    if (wa + wb > 0x7fffffffu) return 1;
    float *part = nullptr;
    unsigned *counters = nullptr;
    const size_t pa = ta_s > 1 ? ta_t * ta_s * BM * BN : 0, pb = tb_s > 1 ? tb_t * tb_s * BM * BN : 0;
    if (pa + pb) {
        Workspace ws;
        const int rc = get_workspace(st, ta_t + tb_t, (pa + pb) * sizeof(float), &ws);
        if (rc) return rc;
        part = static_cast<float *>(ws.scratch);
        counters = ws.counters;
    }
    const RingArgs ga{a.A, a.B, a.C, a.M, a.N, a.K, static_cast<unsigned>(ta_n), static_cast<unsigned>(ta_s), ta_k,
                      a.epi, part, counters, static_cast<unsigned>(wa)};
    const RingArgs gb{b.A, b.B, b.C, b.M, b.N, b.K, static_cast<unsigned>(tb_n), static_cast<unsigned>(tb_s), tb_k,
                      b.epi, part ? part + pa : nullptr, counters ? ctr(counters, ta_t) : nullptr,
                      static_cast<unsigned>(wb)};
    // side work only on CUs the products leave free (one ring workgroup
    // fills a CU's LDS), so that it never delays them
    const size_t nside = side && wa + wb + 8 <= cus ? cus - (wa + wb) : 0;
    StepSide &sd = nside ? *side : none;
    sd.wgs = static_cast<unsigned>(nside);
    hipStream_t s = reinterpret_cast<hipStream_t>(st);
    const dim3 grid(static_cast<unsigned>(wa + wb + nside));
    if (!a.ta && !a.tb) hipLaunchKernelGGL((k_gemm_ring_pair<true, false>), grid, dim3(kRingThreads), 0, s, ga, gb, sd);
    else if (a.ta && !a.tb) hipLaunchKernelGGL((k_gemm_ring_pair<false, false>), grid, dim3(kRingThreads), 0, s, ga, gb, sd);
    else hipLaunchKernelGGL((k_gemm_ring_pair<true, true>), grid, dim3(kRingThreads), 0, s, ga, gb, sd);
    const int rc = launch_status();
    if (rc && side) side->wgs = 0;
    return rc;
}

}  // namespace cxm

#ifdef CXM_TIMELINE
// Diagnostics build only (not declared in include/cxm_hip.h): copies the
// ring products' timeline tables (kGemmTlKinds x kGemmTlWgs x kGemmTlMarks
// 64-bit words) to host memory, after the caller's synchronisation.
extern "C" int cxm_timeline_gemm_read(unsigned long long *host, size_t words) {
    if (!host || words != static_cast<size_t>(kGemmTlKinds) * kGemmTlWgs * kGemmTlMarks) return CXM_E_INVALID;
    const hipError_t e = hipMemcpyFromSymbol(host, HIP_SYMBOL(gemm_timeline), words * sizeof(unsigned long long));
    return e == hipSuccess ? CXM_OK : static_cast<int>(e);
}
#endif

extern "C" {

int cxm_gemm_f32(const float *a, const float *b, float *c, size_t m, size_t k, size_t n, int trans_a,
                 int trans_b, const float *bias, int act, const float *gate, cxm_stream_t s) {
    return cxm::gemm_ex(a, b, c, m, k, n, trans_a != 0, trans_b != 0, cxm::Epilogue{bias, gate, act, 0, 0.0f}, s);
}

int cxm_gemm_f32_kernel(int variant) {
    if (variant < -1 || variant > 7) return CXM_E_INVALID;
    cxm::g_gemm_kc.store(variant);
    return CXM_OK;
}

int cxm_matmul_f32(const float *a, const float *b, float *c, size_t xN, size_t yN, size_t zN,
                   cxm_stream_t s) {
    return cxm::gemm_ex(a, b, c, xN, yN, zN, 0, 0, cxm::Epilogue{nullptr, nullptr, CXM_ACT_NONE, 0, 0.0f}, s);
}

}  // extern "C"
