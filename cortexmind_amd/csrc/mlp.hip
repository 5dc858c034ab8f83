// Training step of the 3-layer ReLU MLP (784 -> 1024 -> 1024 -> 10 at the
// C5 workload), composed on the host from the library's own kernels.
//
// The reference has no layers, loss, optimizer or concrete autograd flows:
// only the abstract meta::GradientFlow::backward(const Tensor&)
// (source/CortexMind/framework/Graph/flow.hpp:15-24).  The step below is
// the forward pass, the reverse-mode backward of each op in reverse order
// (the job a chain of concrete GradientFlows would do), and SGD:
//   h1 = relu(x W1 + b1), h2 = relu(h1 W2 + b2), logits = h2 W3 + b3
//   loss, dlogits = softmax cross-entropy
//   dh2 = (dl W3^T) * [h2 > 0], gW3 = h2^T dl, gb3 = colsum(dl)
//   dh1 = (dh2 W2^T) * [h1 > 0], gW2 = h1^T dh2, gb2 = colsum(dh2)
//   gW1 = x^T dh1, gb1 = colsum(dh1)
//   W -= lr * gW, b -= lr * gb
// Bias add and ReLU ride in the forward GEMM epilogue, the ReLU backward
// mask in the dX GEMM epilogue, and each SGD update in the epilogue of the
// kernel that produces its gradient (weights: the dW GEMM; biases: the
// column sum), so no gradient is ever written out.  A layer's weights are
// updated only after its dX product has read them, which gives the same
// values as taking every gradient first.  Everything is enqueued on one
// stream without host synchronisation.
//
// The output layer (d3 <= 16 classes, d2 <= 1024, d2 % 4 == 0) runs as one
// "head" kernel per 16 rows of the batch: logits = h2 W3 + b3, the softmax
// cross-entropy, its gradient dl, and dh2 = (dl W3^T) * [h2 > 0] from one read of h2, with
// per-workgroup partial sums of the loss, of dl's columns (gb3), of dh2's
// columns (gb2) and of h2^T dl (gW3); a finish kernel adds the partials in
// workgroup order and applies loss / B and the b3, b2 and W3 SGD steps.  The
// unfused chain (thin GEMMs for the logits, dh2 and gW3, the cross-entropy,
// two column sums) ran 67 us at the C5 shape, most of it launch and latency;
// the fused pair runs 21 us.
#include <cfloat>
#include <new>

#include "cxm_common.hpp"
#include "mlp_side.hpp"

struct cxm_mlp3 {
    size_t b, d0, d1, d2, d3;
    float *h1, *h2, *lg, *dl, *dh2, *dh1;
    float *part;  // head partials [blocks][head_part_width(d2, d3)] (fused head only)
    unsigned head_blocks;
    int fused_head;  // 1: the fused output layer (d3 <= 16, d2 <= 1024, d2 % 4 == 0); 0: unfused
    void *block;  // one allocation holding all of the above
    unsigned last_side;  // side workgroups of the last step's paired launch (0: separate kernels)
};

namespace cxm {
namespace {

constexpr int kHeadThreads = 1024;
constexpr int kHeadRows = 16;  // rows per workgroup: the 16 of a 16x16 MFMA tile
constexpr int kHeadMaxD2 = 1024;
// partial columns after the d2 of gb2 (kHeadExtra, mlp_side.hpp): the loss,
// then gb3[0..d3-1] (up to 17 values; 32 keeps the gW3 columns that follow
// 16-byte aligned)
// A head workgroup's partial row: gb2 [D2], the loss and gb3 [kHeadExtra], gW3 [D3][D2].
__host__ __device__ inline size_t head_part_width(size_t d2, size_t d3) { return d2 + kHeadExtra + d3 * d2; }

// One workgroup of 16 waves: rows r0 .. r0 + 15 of the batch; wave w owns
// columns k in [64 w, 64 w + 64) of h2 (and rows of W3).  Both products run
// on v_mfma_f32_16x16x4_f32 (lane l supplies A[l % 16][l / 16] and
// B[l / 16][l % 16]; register i of lane l receives D[4 (l / 16) + i][l % 16]):
//  1. logits [16 rows x 16 classes]: lane (r, q) = (l % 16, l / 16) holds
//     h2[r][64 w + 16 t + 4 q + e] (float4 t, component e); MFMA (t, e) takes
//     those as A and W3[64 w + 16 t + 4 q + e][c] as B (c = l % 16); the 16
//     waves' partial tiles are added in wave order;
//  2. the cross-entropy with one lane per (row, class) in waves 0..3: wave
//     w takes rows 4 w .. 4 w + 3, lane l row 4 w + l / 16, class l % 16;
//     max and sums over a row are DPP reductions inside 16-lane rows;
//  3. dh2^T = W3 dl^T per block of 16 k: A = W3[64 w + 16 blk + l % 16][4 q + j],
//     B = dl[l % 16][4 q + j] (MFMA j = 0..3 covers the 16 classes), so lane
//     (r, q) receives dh2[r][64 w + 16 blk + 4 q + i], the very elements of
//     h2 it holds: the ReLU gate needs no second read, and each lane stores
//     a float4.  The column sums over the 16 rows are DPP sums.
// Sixteen waves (four per SIMD) let one wave's loads overlap another's
// arithmetic; with four waves of 256 k each the kernel was a serial chain
// of loads, barrier, products and stores (14 us at the C5 shape).
// W3 arrives by coalesced loads of its [D2][D3] storage and is scattered
// in LDS to Wk[k][c] (row stride 20 floats, zero past D3 and D2), for
// which the B reads of step 1 (lanes (c, q): rows 4 q + e, column c) and
// the A reads of step 3 (lanes (kk, q): row kk, columns 4 q ..) meet no
// bank conflicts.  Writes dh2 [B, D2] and part[blockIdx] =
// (colsum dh2 [D2], nll sum, colsum dl [D3], gW3 [D3][D2]).
constexpr int kWkStride = 20;
constexpr int kHeadW3PerThread = kHeadMaxD2 * 16 / kHeadThreads;

// Per-workgroup timeline of the head, for the diagnostics build only (this
// file compiled with -DCXM_TIMELINE, read by `bench.py --timeline c5`):
// thread 0 writes the 100 MHz s_memrealtime clock to mark i of record
// blockIdx.x % kHeadTlWgs: 0 entry, 1 W3 and h2 loaded (first barrier),
// 2 W3 in LDS, 3 logits, 4 cross-entropy, 5 dh2 stored and summed, 6 the
// partials stored (past a final barrier).  Without CXM_TIMELINE the marks
// compile to nothing.
#ifdef CXM_TIMELINE
constexpr unsigned kHeadTlWgs = 256, kHeadTlMarks = 8;
static __device__ unsigned long long head_timeline[kHeadTlWgs][kHeadTlMarks];
__device__ __forceinline__ void head_tl_mark(unsigned i) {
    if (threadIdx.x == 0)
        __builtin_nontemporal_store(__builtin_amdgcn_s_memrealtime(), &head_timeline[blockIdx.x % kHeadTlWgs][i]);
}
#else
__device__ __forceinline__ void head_tl_mark(unsigned) {}
#endif

__device__ __forceinline__ float row16_sum(float v) {  // sum over the 16-lane row, in every lane of it
    v += dpp<kQuadXor1>(v);
    v += dpp<kQuadXor2>(v);
    v += dpp<kRowHalfMirror>(v);
    v += dpp<kRowMirror>(v);
    return v;
}
__device__ __forceinline__ float row16_max(float v) {
    v = vmax(v, dpp<kQuadXor1>(v));
    v = vmax(v, dpp<kQuadXor2>(v));
    v = vmax(v, dpp<kRowHalfMirror>(v));
    v = vmax(v, dpp<kRowMirror>(v));
    return v;
}

__global__ __launch_bounds__(kHeadThreads) void k_mlp_head(const float *__restrict__ h2,
                                                           const float *__restrict__ w3,
                                                           const float *__restrict__ b3,
                                                           const int32_t *__restrict__ labels,
                                                           float *__restrict__ dh2,
                                                           size_t B, size_t D2, size_t D3, float inv_b,
                                                           float *__restrict__ part) {
    constexpr int NW = kHeadThreads / kWave;
    __shared__ __attribute__((aligned(16))) float Wk[kHeadMaxD2 * kWkStride];
    __shared__ float red[NW][16][16];
    __shared__ __attribute__((aligned(16))) float dt[16][16];
    __shared__ float nl[16];
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave, tid = threadIdx.x;
    const int l16 = lane & 15, q = lane >> 4;
    head_tl_mark(0);
    const int nc = static_cast<int>(D3), d2 = static_cast<int>(D2), nw3 = d2 * nc;
    const size_t r0 = static_cast<size_t>(blockIdx.x) * kHeadRows;
    // Every load is issued as straight-line code from a clamped, in-range
    // address (loads under per-element conditions were compiled with waits
    // between them); what a clamped load brings is never used.  W3 goes
    // first, so that waiting for it does not wait for h2.
    float wt[kHeadW3PerThread];
#pragma unroll
    for (int j = 0; j < kHeadW3PerThread; ++j) {
        const int i = tid + kHeadThreads * j;
        wt[j] = w3[i < nw3 ? i : nw3 - 1];
    }
    const size_t arow = r0 + l16 < B ? r0 + l16 : B - 1;
    float4 a[4];  // h2[arow][64 w + 16 t + 4 q .. + 3]
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const size_t k = 64 * w + 16 * t + 4 * q;
        a[t] = ld4(h2 + arow * D2 + (k < D2 ? k : D2 - 4));
    }
    const int32_t lab = labels[r0 + 4 * w + q < B ? r0 + 4 * w + q : B - 1];  // the row of step 2 (waves 0..3)
    __builtin_amdgcn_sched_barrier(0);
    // Wk: zero row tid, then scatter W3 element i to Wk[i / D3][i % D3]
    {
        float4 *row = reinterpret_cast<float4 *>(&Wk[tid * kWkStride]);
#pragma unroll
        for (int c4 = 0; c4 < kWkStride / 4; ++c4) row[c4] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    __syncthreads();
    head_tl_mark(1);
    const float rnc = 1.0f / static_cast<float>(nc);
#pragma unroll
    for (int j = 0; j < kHeadW3PerThread; ++j) {
        const int i = tid + kHeadThreads * j;
        // (i + 0.5) / D3 lies at least 1/32 from an integer; the float error
        // at i < 16384 is below 0.005, so the truncation is the quotient
        const int k = static_cast<int>((static_cast<float>(i) + 0.5f) * rnc), c = i - k * nc;
        if (i < nw3) Wk[k * kWkStride + c] = wt[j];
    }
    __syncthreads();
    head_tl_mark(2);

    // 1. partial logits over this wave's 64 k (two accumulators, added at the end)
    f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const int kb = 64 * w + 16 * t + 4 * q;
        const float b0 = Wk[(kb + 0) * kWkStride + l16], b1 = Wk[(kb + 1) * kWkStride + l16];
        const float b2 = Wk[(kb + 2) * kWkStride + l16], b3v = Wk[(kb + 3) * kWkStride + l16];
        f32x4 &acc = (t & 1) ? acc1 : acc0;
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[t].x, b0, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[t].y, b1, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[t].z, b2, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[t].w, b3v, acc, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) red[w][4 * q + i][l16] = acc0[i] + acc1[i];
    __syncthreads();
    head_tl_mark(3);

    // 2. cross-entropy in waves 0..3: lane (row 4 w + q, class l16)
    if (w < 4) {
        const int row = 4 * w + q;
        const bool valid = r0 + row < B, cin = l16 < nc;
        float v = red[0][row][l16];
#pragma unroll
        for (int u = 1; u < NW; ++u) v += red[u][row][l16];
        v = v + (cin ? b3[l16] : 0.0f);
        const float m = row16_max(cin ? v : -FLT_MAX);
        const float e = cin ? expf(v - m) : 0.0f;
        const float s = row16_sum(e);
        float p = e / s;
        if (l16 == lab) p = p - 1.0f;
        const float d = (cin && valid) ? p * inv_b : 0.0f;
        dt[row][l16] = d;
        const bool ok = lab >= 0 && lab < nc;
        const float nll = row16_sum(l16 == lab ? -((v - m) - logf(s)) : 0.0f);
        if (l16 == 0) nl[row] = valid ? (ok ? nll : NAN) : 0.0f;
    }
    __syncthreads();
    head_tl_mark(4);

    // 3. dh2 = (dl W3^T) * [h2 > 0] through dh2^T = W3 dl^T, and its column sums
    const float4 bd = *reinterpret_cast<const float4 *>(&dt[l16][4 * q]);  // dl[l16][4 q .. + 3]
    f32x4 o[4];
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
        const float4 aw = *reinterpret_cast<const float4 *>(&Wk[(64 * w + 16 * blk + l16) * kWkStride + 4 * q]);
        o[blk] = f32x4{0.f, 0.f, 0.f, 0.f};
        o[blk] = __builtin_amdgcn_mfma_f32_16x16x4f32(aw.x, bd.x, o[blk], 0, 0, 0);
        o[blk] = __builtin_amdgcn_mfma_f32_16x16x4f32(aw.y, bd.y, o[blk], 0, 0, 0);
        o[blk] = __builtin_amdgcn_mfma_f32_16x16x4f32(aw.z, bd.z, o[blk], 0, 0, 0);
        o[blk] = __builtin_amdgcn_mfma_f32_16x16x4f32(aw.w, bd.w, o[blk], 0, 0, 0);
    }
    const bool rvalid = r0 + l16 < B;
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
        o[blk][0] = o[blk][0] * (a[blk].x > 0.0f ? 1.0f : 0.0f);
        o[blk][1] = o[blk][1] * (a[blk].y > 0.0f ? 1.0f : 0.0f);
        o[blk][2] = o[blk][2] * (a[blk].z > 0.0f ? 1.0f : 0.0f);
        o[blk][3] = o[blk][3] * (a[blk].w > 0.0f ? 1.0f : 0.0f);
        const size_t kk = 64 * w + 16 * blk + 4 * q;
        if (rvalid && kk < D2) st4(dh2 + (r0 + l16) * D2 + kk, make_float4(o[blk][0], o[blk][1], o[blk][2], o[blk][3]));
    }
    // column sums over the 16 rows (rows past B hold zeros: their dl is 0),
    // each DPP step applied to all 16 values before the next
#pragma unroll
    for (int blk = 0; blk < 4; ++blk)
#pragma unroll
        for (int i = 0; i < 4; ++i) o[blk][i] += dpp<kQuadXor1>(o[blk][i]);
#pragma unroll
    for (int blk = 0; blk < 4; ++blk)
#pragma unroll
        for (int i = 0; i < 4; ++i) o[blk][i] += dpp<kQuadXor2>(o[blk][i]);
#pragma unroll
    for (int blk = 0; blk < 4; ++blk)
#pragma unroll
        for (int i = 0; i < 4; ++i) o[blk][i] += dpp<kRowHalfMirror>(o[blk][i]);
#pragma unroll
    for (int blk = 0; blk < 4; ++blk)
#pragma unroll
        for (int i = 0; i < 4; ++i) o[blk][i] += dpp<kRowMirror>(o[blk][i]);
    head_tl_mark(5);
    float *__restrict__ prow = part + static_cast<size_t>(blockIdx.x) * head_part_width(D2, D3);

    // 4. gW3 over the 16 rows, G[k][c] = sum_b h2[b][k] dl[b][c], on the same MFMA with the
    //    contraction over b: MFMA j takes A[kk][q] = h2[4 j + q][k + kk] (lane (kk, q)) and
    //    B[q][c] = dl[4 j + q][c].  Lane (kk, q) fetches its A value from the lane that holds
    //    it, (4 j + q) + 16 (kk / 4), component kk % 4 of a[blk] (ds_bpermute, all four
    //    components, then a select); lane (c, q) receives G[k + 4 q + i][c], stored as a float4
    //    into the workgroup's [D3][D2] partial.
    float *__restrict__ pg = prow + D2 + kHeadExtra;
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
        f32x4 g = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int src = ((4 * j + q) + 16 * (l16 >> 2)) * 4;
            const float v0 = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src, __builtin_bit_cast(int, a[blk].x)));
            const float v1 = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src, __builtin_bit_cast(int, a[blk].y)));
            const float v2 = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src, __builtin_bit_cast(int, a[blk].z)));
            const float v3 = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src, __builtin_bit_cast(int, a[blk].w)));
            const int e = l16 & 3;
            const float av = e == 0 ? v0 : e == 1 ? v1 : e == 2 ? v2 : v3;
            g = __builtin_amdgcn_mfma_f32_16x16x4f32(av, dt[4 * j + q][l16], g, 0, 0, 0);
        }
        const size_t kk = 64 * w + 16 * blk + 4 * q;
        if (l16 < nc && kk < D2) *reinterpret_cast<float4 *>(pg + l16 * D2 + kk) = make_float4(g[0], g[1], g[2], g[3]);
    }
    if (l16 == 0) {
#pragma unroll
        for (int blk = 0; blk < 4; ++blk) {
            const size_t kk = 64 * w + 16 * blk + 4 * q;
            if (kk < D2) *reinterpret_cast<float4 *>(prow + kk) = make_float4(o[blk][0], o[blk][1], o[blk][2], o[blk][3]);
        }
    }
    if (tid < 16) {
        float cs = 0.0f;
        for (int r = 0; r < 16; ++r) cs += dt[r][tid];
        if (tid < nc) prow[D2 + 1 + tid] = cs;
    } else if (tid == 16) {
        float t = 0.0f;
        for (int r = 0; r < 16; ++r) t += nl[r];
        prow[D2] = t;
    }
#ifdef CXM_TIMELINE
    __syncthreads();
    head_tl_mark(6);
#endif
}

// Column c of the partials: the sum over workgroups p = q, q + 16, ... per
// thread (q = threadIdx.x / 64), then the 16 thread sums in q order.
// Columns < D2: b2 -= lr * sum; D2: *loss = sum / B; D2 + 1 + n: b3[n] -= lr * sum;
// D2 + 16 + c D2 + k: W3[k][c] -= lr * sum.
constexpr int kFinishThreads = 1024;
constexpr int kFinishCols = 64;
__global__ __launch_bounds__(kFinishThreads) void k_head_finish(const float *__restrict__ part, unsigned blocks,
                                                                size_t D2, size_t D3, size_t B, float lr,
                                                                float *__restrict__ loss, float *__restrict__ b2,
                                                                float *__restrict__ b3, float *__restrict__ w3) {
    constexpr int Q = kFinishThreads / kFinishCols;
    __shared__ float acc[Q][kFinishCols];
    const int c = threadIdx.x % kFinishCols, q = threadIdx.x / kFinishCols;
    const size_t col = static_cast<size_t>(blockIdx.x) * kFinishCols + c;
    const size_t pw = head_part_width(D2, D3);
    float v = 0.0f;
    if (col < pw) {
        constexpr unsigned G = 16;
        for (unsigned p0 = q; p0 < blocks; p0 += G * Q) {
            float t[G];
#pragma unroll
            for (unsigned g = 0; g < G; ++g) {
                const unsigned p = p0 + g * Q;
                t[g] = p < blocks ? part[static_cast<size_t>(p) * pw + col] : 0.0f;
            }
#pragma unroll
            for (unsigned g = 0; g < G; ++g) v += t[g];
        }
    }
    acc[q][c] = v;
    __syncthreads();
    if (q != 0 || col >= pw) return;
    float g = acc[0][c];
#pragma unroll
    for (int i = 1; i < Q; ++i) g += acc[i][c];
    if (col < D2) {
        const float t = g * lr;  // matrix_t::sub(b, ScalarOp::mul(g, lr)): two roundings
        b2[col] = b2[col] - t;
    } else if (col == D2) {
        loss[0] = g / static_cast<float>(B);
    } else if (col < D2 + kHeadExtra) {
        if (col - D2 - 1 < D3) {
            const float t = g * lr;
            b3[col - D2 - 1] = b3[col - D2 - 1] - t;
        }
    } else {
        const size_t i = col - D2 - kHeadExtra, cls = i / D2, k = i - cls * D2;
        const float t = g * lr;
        w3[k * D3 + cls] = w3[k * D3 + cls] - t;
    }
}


int run_head(const cxm_mlp3 *h, const int32_t *labels, const float *w3, const float *b3, hipStream_t s) {
    const float inv_b = 1.0f / static_cast<float>(h->b);
    hipLaunchKernelGGL(k_mlp_head, dim3(h->head_blocks), dim3(kHeadThreads), 0, s, h->h2, w3, b3, labels,
                       h->dh2, h->b, h->d2, h->d3, inv_b, h->part);
    return launch_status();
}

int run_head_finish(const cxm_mlp3 *h, float *w3, float *b3, float *b2, float lr, float *loss, hipStream_t s) {
    const size_t pw = head_part_width(h->d2, h->d3);
    hipLaunchKernelGGL(k_head_finish, dim3(ceil_div(pw, kFinishCols)), dim3(kFinishThreads), 0, s, h->part,
                       h->head_blocks, h->d2, h->d3, h->b, lr, loss, b2, b3, w3);
    return launch_status();
}

}  // namespace
}  // namespace cxm

#ifdef CXM_TIMELINE
// Diagnostics build only (not declared in include/cxm_hip.h): copies the
// head's timeline table (kHeadTlWgs x kHeadTlMarks 64-bit words) to host
// memory, after the caller's synchronisation.
extern "C" int cxm_timeline_head_read(unsigned long long *host, size_t words) {
    if (!host || words != static_cast<size_t>(cxm::kHeadTlWgs) * cxm::kHeadTlMarks) return CXM_E_INVALID;
    const hipError_t e = hipMemcpyFromSymbol(host, HIP_SYMBOL(cxm::head_timeline), words * sizeof(unsigned long long));
    return e == hipSuccess ? CXM_OK : static_cast<int>(e);
}
#endif

extern "C" {

int cxm_mlp3_create(cxm_mlp3 **handle, size_t batch, size_t d0, size_t d1, size_t d2, size_t d3) {
    if (!handle || !batch || !d0 || !d1 || !d2 || !d3) return CXM_E_INVALID;
    *handle = nullptr;
    cxm_mlp3 *h = new (std::nothrow) cxm_mlp3{};
    if (!h) return CXM_E_INVALID;
    h->b = batch;
    h->d0 = d0;
    h->d1 = d1;
    h->d2 = d2;
    h->d3 = d3;
    // the fused output layer when its shape fits the head kernel
    const size_t blocks = (batch + cxm::kHeadRows - 1) / cxm::kHeadRows;
    h->fused_head = d3 <= 16 && d2 <= static_cast<size_t>(cxm::kHeadMaxD2) && d2 % 4 == 0 && blocks <= 0x7fffffffu;
    h->head_blocks = static_cast<unsigned>(blocks);
    // sizes in floats, each rounded to 64 floats (256 B) to keep 128-bit alignment
    auto r = [](size_t n) { return (n + 63) / 64 * 64; };
    const size_t sizes[7] = {r(batch * d1), r(batch * d2), r(batch * d3), r(batch * d3),
                             r(batch * d2), r(batch * d1), h->fused_head ? r(blocks * cxm::head_part_width(d2, d3)) : 0};
    size_t total = 0;
    for (size_t s : sizes) total += s;
    void *p = nullptr;
    int rc = cxm_dev_malloc(&p, total * sizeof(float));
    if (rc) {
        delete h;
        return rc;
    }
    h->block = p;
    float *f = static_cast<float *>(p);
    float **slots[7] = {&h->h1, &h->h2, &h->lg, &h->dl, &h->dh2, &h->dh1, &h->part};
    for (int i = 0; i < 7; ++i) {
        *slots[i] = f;
        f += sizes[i];
    }
    *handle = h;
    return CXM_OK;
}

int cxm_mlp3_destroy(cxm_mlp3 *h) {
    if (!h) return CXM_E_INVALID;
    int rc = cxm_dev_free(h->block);
    delete h;
    return rc;
}

int cxm_mlp3_step_f32(cxm_mlp3 *h, const float *x, const int32_t *labels, float *w1, float *b1,
                      float *w2, float *b2, float *w3, float *b3, float lr, float *loss,
                      cxm_stream_t s) {
    if (!h || !x || !labels || !w1 || !b1 || !w2 || !b2 || !w3 || !b3 || !loss) return CXM_E_INVALID;
    const size_t B = h->b, d0 = h->d0, d1 = h->d1, d2 = h->d2, d3 = h->d3;
    int rc;
#define CXM_TRY(call)        \
    if ((rc = (call)) != 0) \
        return rc
    using cxm::Epilogue;
    const Epilogue sgd{nullptr, nullptr, CXM_ACT_NONE, 1, lr};
    // forward
    CXM_TRY(cxm::gemm_ex(x, w1, h->h1, B, d0, d1, 0, 0, Epilogue{b1, nullptr, CXM_ACT_RELU, 0, 0.0f}, s));
    CXM_TRY(cxm::gemm_ex(h->h1, w2, h->h2, B, d1, d2, 0, 0, Epilogue{b2, nullptr, CXM_ACT_RELU, 0, 0.0f}, s));
    if (h->fused_head) {
        // output layer fused: logits, loss, dl, dh2 (reads W3); the loss, b3,
        // b2 and W3 updates follow with the weight gradients (below)
        CXM_TRY(cxm::run_head(h, labels, w3, b3, reinterpret_cast<hipStream_t>(s)));
    } else {
        CXM_TRY(cxm::gemm_ex(h->h2, w3, h->lg, B, d2, d3, 0, 0, Epilogue{b3, nullptr, CXM_ACT_NONE, 0, 0.0f}, s));
        CXM_TRY(cxm_softmax_xent_f32(h->lg, labels, loss, h->dl, B, d3, s));
        // layer 3: dX first (reads W3), then W3 -= lr * h2^T dl, b3 -= lr * colsum(dl)
        CXM_TRY(cxm::gemm_ex(h->dl, w3, h->dh2, B, d3, d2, 0, 1, Epilogue{nullptr, h->h2, CXM_ACT_NONE, 0, 0.0f}, s));
        CXM_TRY(cxm::gemm_ex(h->h2, h->dl, w3, d2, B, d3, 1, 0, sgd, s));
        CXM_TRY(cxm::colsum_sgd(h->dl, b3, B, d3, lr, s));
    }
    // layer 2: dX first (reads W2)
    CXM_TRY(cxm::gemm_ex(h->dh2, w2, h->dh1, B, d2, d1, 0, 1, Epilogue{nullptr, h->h1, CXM_ACT_NONE, 0, 0.0f}, s));
    if (!h->fused_head) CXM_TRY(cxm::colsum_sgd(h->dh2, b2, B, d2, lr, s));
    // the two weight gradients with their SGD steps, W2 -= lr h1^T dH2 and
    // W1 -= lr x^T dH1: independent, so one launch where both take the ring
    // (the second's workgroups fill the CUs the first releases); else in turn
    // (the output layer's finish and the layer-1 bias step ride along on the
    // CUs the pair leaves free when there are enough; else they follow)
    cxm::StepSide side{};
    const bool side_ok = B <= 0xffffffffu && d1 <= 0xffffffffu;  // its sizes are 32-bit
    if (h->fused_head && side_ok) {
        side.part = h->part;
        side.blocks = h->head_blocks;
        side.pw = static_cast<unsigned>(cxm::head_part_width(d2, d3));
        side.d2 = static_cast<unsigned>(d2);
        side.d3 = static_cast<unsigned>(d3);
        side.b = static_cast<unsigned>(B);
        side.loss = loss;
        side.b2 = b2;
        side.b3 = b3;
        side.w3 = w3;
    }
    side.lr = lr;
    if (d1 % 4 == 0 && side_ok) {
        side.dh1 = h->dh1;
        side.b1 = b1;
        side.d1 = static_cast<unsigned>(d1);
        side.b = static_cast<unsigned>(B);
    }
    h->last_side = 0;
    {
        const cxm::GemmSpec g2{h->h1, h->dh2, w2, d1, B, d2, 1, 0, sgd};
        const cxm::GemmSpec g1{x, h->dh1, w1, d0, B, d1, 1, 0, sgd};
        rc = cxm::gemm_ex_pair(g2, g1, s, &side);
        if (rc == 1) {
            CXM_TRY(cxm::gemm_ex(h->h1, h->dh2, w2, d1, B, d2, 1, 0, sgd, s));
            CXM_TRY(cxm::gemm_ex(x, h->dh1, w1, d0, B, d1, 1, 0, sgd, s));
        } else if (rc) {
            return rc;
        }
    }
    if (side.wgs == 0 || !side.part) {
        if (h->fused_head) CXM_TRY(cxm::run_head_finish(h, w3, b3, b2, lr, loss, reinterpret_cast<hipStream_t>(s)));
    }
    // layer 1 bias
    if (side.wgs == 0 || !side.dh1) CXM_TRY(cxm::colsum_sgd(h->dh1, b1, B, d1, lr, s));
    h->last_side = side.wgs;
#undef CXM_TRY
    return CXM_OK;
}

int cxm_mlp3_last_side(const cxm_mlp3 *h, unsigned *wgs) {
    if (!h || !wgs) return CXM_E_INVALID;
    *wgs = h->last_side;
    return CXM_OK;
}

}  // extern "C"
