// Elementwise fp32 kernels: same-shape binary ops (pow included), row/column
// broadcast, tensor-op-scalar, unary activations, the fused affine +
// activation forward/backward of the C3 workload, and the SGD update.
//
// Replaces the float4 grid-stride loops of the reference's CUDA path
// (kernels::Binary / kernels::scalar / kernels::Unary,
// source/CortexMind/framework/Engine/Kernels/binary.cuh:15-39,
// scalar.cuh:30-54, unary.cuh:16-40) and the CPU Broadcast::row/col
// (Engine/AVX2/broadcast.cpp:182-388), which has no GPU form there.  The
// aligned forms run as the one-float4-per-thread streaming maps of
// cxm_common.hpp (k_map4, k_zip4, k_rowmap4) with the functors below;
// unaligned pointers take scalar grid-stride loops.
//
// Every op rounds exactly as the reference's scalar expression does: the
// library is built with -ffp-contract=off, so x*s+b is a rounded product
// followed by a rounded sum, never an fma.  ReLU is an explicit select
// (0 > t ? 0 : t), matching _mm256_max_ps(0, t) for -0.0 and NaN.
#include "cxm_common.hpp"
#include "ops.hpp"

namespace cxm {
namespace {

__device__ __forceinline__ float bin(int op, float a, float b) {
    switch (op) {
        case CXM_OP_ADD: return a + b;
        case CXM_OP_SUB: return a - b;
        case CXM_OP_MUL: return a * b;
        case CXM_OP_DIV: return a / b;
        case CXM_OP_MAX: return a > b ? a : b;
        case CXM_OP_MIN: return a < b ? a : b;
        default: return pow_f32(a, b);
    }
}

template <int OP>
__device__ __forceinline__ float4 bin4(float4 a, float4 b) {
    return make_float4(bin_t<OP>(a.x, b.x), bin_t<OP>(a.y, b.y), bin_t<OP>(a.z, b.z),
                       bin_t<OP>(a.w, b.w));
}

template <int ACT>
__device__ __forceinline__ float4 act4(float4 t) {
    return make_float4(act<ACT>(t.x), act<ACT>(t.y), act<ACT>(t.z), act<ACT>(t.w));
}

// Grid for a flat streaming kernel: enough workgroups to fill 256 CUs
// several times over, each thread then strides through the rest.
inline unsigned stream_grid(size_t n4) {
    size_t b = (n4 + kBlock - 1) / kBlock;
    const size_t cap = 256 * 16;
    return static_cast<unsigned>(b < 1 ? 1 : (b > cap ? cap : b));
}

// -------------------------------------------------------------- binary

__global__ __launch_bounds__(kBlock) void k_binary_scalar(const float *x, const float *y, float *z,
                                                          size_t n, int op) {
    const size_t stride = static_cast<size_t>(gridDim.x) * kBlock;
    for (size_t i = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride)
        z[i] = bin(op, x[i], y[i]);
}

// ------------------------------------------------------------ broadcast

__global__ __launch_bounds__(kBlock) void k_bcast_scalar(const float *x, const float *y, float *z,
                                                         size_t m, size_t n, int op, int row_mode) {
    const size_t total = m * n;
    const size_t stride = static_cast<size_t>(gridDim.x) * kBlock;
    for (size_t i = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x; i < total; i += stride) {
        const size_t r = i / n;
        const size_t c = i - r * n;
        z[i] = bin(op, x[i], row_mode ? y[c] : y[r]);
    }
}

// --------------------------------------------------------------- scalar

__global__ __launch_bounds__(kBlock) void k_scalar_scalar(const float *x, float v, float *z, size_t n,
                                                          int op) {
    const size_t stride = static_cast<size_t>(gridDim.x) * kBlock;
    for (size_t i = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride)
        z[i] = bin(op, x[i], v);
}

// ---------------------------------------------------------------- unary

template <int ACT>
__global__ __launch_bounds__(kBlock) void k_unary_scalar(const float *x, float *z, size_t n) {
    const size_t stride = static_cast<size_t>(gridDim.x) * kBlock;
    for (size_t i = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride)
        z[i] = act<ACT>(x[i]);
}

// Functors of the streaming maps (k_map4 / k_zip4 / k_rowmap4).
template <int OP>
struct BinF {
    __device__ float operator()(float a, float b) const { return bin_t<OP>(a, b); }
};
template <int OP>
struct ScalarF {
    float v;
    __device__ float operator()(float a) const { return bin_t<OP>(a, v); }
};
template <int ACT>
struct ActF {
    __device__ float operator()(float t) const { return act<ACT>(t); }
};
// z[i,j] = x[i,j] op y[j]
template <int OP>
struct RowBcastF {
    const float *y;
    __device__ float4 operator()(float4 v, unsigned, size_t j4) const { return bin4<OP>(v, ld4(y + 4 * j4)); }
};
// z[i,j] = x[i,j] op y[i]
template <int OP>
struct ColBcastF {
    const float *y;
    __device__ float4 operator()(float4 v, unsigned row, size_t) const {
        const float c = y[row];
        return bin4<OP>(v, make_float4(c, c, c, c));
    }
};
// y = act(x*scale[j] + bias[j]): product and sum rounded separately
template <int ACT>
struct AffineF {
    const float *scale, *bias;
    __device__ float4 operator()(float4 v, unsigned, size_t j4) const {
        const float4 sc = ld4(scale + 4 * j4), b = ld4(bias + 4 * j4);
        float4 t;
        t.x = v.x * sc.x; t.y = v.y * sc.y; t.z = v.z * sc.z; t.w = v.w * sc.w;
        t.x = t.x + b.x; t.y = t.y + b.y; t.z = t.z + b.z; t.w = t.w + b.w;
        return act4<ACT>(t);
    }
};
// dx = dy * act'(y), the derivative factor from the saved output
template <int ACT>
struct ActBwdF {
    __device__ float operator()(float y, float g) const { return g * dact<ACT>(y); }
};
// w - g*lr, two roundings
struct SgdF {
    float lr;
    __device__ float operator()(float w, float g) const {
        const float t = g * lr;
        return w - t;
    }
};

// ------------------------------------------------------ affine forward

template <int ACT>
__global__ __launch_bounds__(kBlock) void k_affine_fwd_scalar(const float *x, const float *scale,
                                                              const float *bias, float *y, size_t m,
                                                              size_t n) {
    const size_t total = m * n;
    const size_t stride = static_cast<size_t>(gridDim.x) * kBlock;
    for (size_t i = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x; i < total; i += stride) {
        const size_t c = i % n;
        float t = x[i] * scale[c];
        t = t + bias[c];
        y[i] = act<ACT>(t);
    }
}

// ----------------------------------------------------- affine backward

// dz = dy*act'(y); dx = dz*scale[j]; dscale[j] = sum_i dz*x; dbias[j] = sum_i dz.
// Workgroup = 256 columns (64 lanes x float4) x a chunk of rows; its NW
// waves take interleaved rows and meet in LDS; chunks are combined in
// chunk order by the last workgroup of the column tile.  With tile_major
// the chunks of a tile are adjacent in launch order, so early tiles'
// combines overlap later tiles' streaming.
constexpr int kAffTile = 256;

template <int ACT, bool VEC, int UNR, int NW>
__global__ __launch_bounds__(NW * kWave) void k_affine_bwd(const float *__restrict__ x,
                                                           const float *__restrict__ scale,
                                                           const float *__restrict__ y,
                                                           const float *__restrict__ dy,
                                                           float *__restrict__ dx,
                                                           float *__restrict__ dscale,
                                                           float *__restrict__ dbias, size_t m, size_t n,
                                                           unsigned ntiles, unsigned chunks,
                                                           size_t rows_per_chunk, int tile_major,
                                                           float *__restrict__ part,
                                                           unsigned *__restrict__ counters) {
    constexpr int NSLOT = VEC ? NW : NW / 4;
    __shared__ float lds_s[NSLOT][kAffTile];
    __shared__ float lds_b[NSLOT][kAffTile];
    __shared__ int flag;
    unsigned tile, chunk;
    if (tile_major) {
        chunk = blockIdx.x % chunks;
        tile = blockIdx.x / chunks;
    } else {
        tile = blockIdx.x % ntiles;
        chunk = blockIdx.x / ntiles;
    }
    const int tid = threadIdx.x;
    const size_t r0 = static_cast<size_t>(chunk) * rows_per_chunk;
    const size_t r1 = r0 + rows_per_chunk < m ? r0 + rows_per_chunk : m;

    if constexpr (VEC) {
        const int lane = tid & (kWave - 1);
        const int w = tid / kWave;
        const size_t col = static_cast<size_t>(tile) * kAffTile + lane * 4;
        float as[4] = {0, 0, 0, 0}, ab[4] = {0, 0, 0, 0};
        if (col < n) {
            const float4 sc = ld4(scale + col);
            size_t r = r0 + w;
            auto body = [&](size_t rr, float4 xv, float4 yv, float4 gv) {
                float4 dz;
                dz.x = gv.x * dact<ACT>(yv.x); dz.y = gv.y * dact<ACT>(yv.y);
                dz.z = gv.z * dact<ACT>(yv.z); dz.w = gv.w * dact<ACT>(yv.w);
                float4 d;
                d.x = dz.x * sc.x; d.y = dz.y * sc.y; d.z = dz.z * sc.z; d.w = dz.w * sc.w;
                st4_stream(dx + rr * n + col, d);
                const float p0 = dz.x * xv.x, p1 = dz.y * xv.y, p2 = dz.z * xv.z, p3 = dz.w * xv.w;
                as[0] = as[0] + p0; as[1] = as[1] + p1; as[2] = as[2] + p2; as[3] = as[3] + p3;
                ab[0] = ab[0] + dz.x; ab[1] = ab[1] + dz.y; ab[2] = ab[2] + dz.z; ab[3] = ab[3] + dz.w;
            };
            for (; r + (UNR - 1) * NW < r1; r += UNR * NW) {
                float4 xv[UNR], yv[UNR], gv[UNR];
#pragma unroll
                for (int u = 0; u < UNR; ++u) {
                    const size_t o = (r + u * NW) * n + col;
                    xv[u] = ld4_stream(x + o);
                    yv[u] = ld4_stream(y + o);
                    gv[u] = ld4_stream(dy + o);
                }
#pragma unroll
                for (int u = 0; u < UNR; ++u) body(r + u * NW, xv[u], yv[u], gv[u]);
            }
            for (; r < r1; r += NW) {
                const size_t o = r * n + col;
                body(r, ld4_stream(x + o), ld4_stream(y + o), ld4_stream(dy + o));
            }
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            lds_s[w][lane * 4 + c] = as[c];
            lds_b[w][lane * 4 + c] = ab[c];
        }
    } else {
        const int c = tid % kAffTile, ph = tid / kAffTile;
        const size_t col = static_cast<size_t>(tile) * kAffTile + c;
        float ms = 0.0f, mb = 0.0f;
        if (col < n) {
            const float sc = scale[col];
            for (size_t r = r0 + ph; r < r1; r += NSLOT) {
                const size_t o = r * n + col;
                const float dz = dy[o] * dact<ACT>(y[o]);
                dx[o] = dz * sc;
                const float p = dz * x[o];
                ms = ms + p;
                mb = mb + dz;
            }
        }
        lds_s[ph][c] = ms;
        lds_b[ph][c] = mb;
    }
    __syncthreads();
    const bool owner = tid < kAffTile;  // threads 0..255 own one column each from here
    float ms = 0.0f, mb = 0.0f;
    if (owner) {
#pragma unroll
        for (int k = 0; k < NSLOT; ++k) {  // slots in order
            ms = ms + lds_s[k][tid];
            mb = mb + lds_b[k][tid];
        }
    }
    const size_t col = static_cast<size_t>(tile) * kAffTile + tid;
    if (chunks == 1) {
        if (owner && col < n) {
            dscale[col] = ms;
            dbias[col] = mb;
        }
        return;
    }
    const size_t slot = static_cast<size_t>(tile) * chunks;
    if (owner) {
        st_dev(&part[((slot + chunk) * 2 + 0) * kAffTile + tid], ms);
        st_dev(&part[((slot + chunk) * 2 + 1) * kAffTile + tid], mb);
    }
    if (!last_block_ticket(ctr(counters, tile), chunks, &flag)) return;
    if (owner) {
        // both sums' loads go out together, 8 chunks at a time
        float a = 0.0f, bsum = 0.0f;
        for (unsigned c0 = 0; c0 < chunks; c0 += 8) {
            float va[8], vb[8];
#pragma unroll
            for (unsigned u = 0; u < 8; ++u) {
                const bool in = c0 + u < chunks;
                va[u] = in ? ld_dev(&part[((slot + c0 + u) * 2 + 0) * kAffTile + tid]) : 0.0f;
                vb[u] = in ? ld_dev(&part[((slot + c0 + u) * 2 + 1) * kAffTile + tid]) : 0.0f;
            }
#pragma unroll
            for (unsigned u = 0; u < 8; ++u) {
                a = a + va[u];
                bsum = bsum + vb[u];
            }
        }
        if (col < n) {
            dscale[col] = a;
            dbias[col] = bsum;
        }
    }
}

// ------------------------------------------------------------------ sgd

// w = w - g*lr, two roundings (matrix_t::sub of ScalarOp::mul).
__global__ __launch_bounds__(kBlock) void k_act_bwd_scalar(const float *y, const float *dy, float *dx, size_t n,
                                                            int act) {
    const size_t stride = static_cast<size_t>(gridDim.x) * kBlock;
    for (size_t i = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
        const float yy = y[i];
        const float d = act == CXM_ACT_RELU ? dact<CXM_ACT_RELU>(yy)
                                            : (act == CXM_ACT_SIGMOID ? dact<CXM_ACT_SIGMOID>(yy) : dact<CXM_ACT_TANH>(yy));
        dx[i] = dy[i] * d;
    }
}

__global__ __launch_bounds__(kBlock) void k_sgd_scalar(float *w, const float *g, float lr, size_t n) {
    const size_t stride = static_cast<size_t>(gridDim.x) * kBlock;
    for (size_t i = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
        const float t = g[i] * lr;
        w[i] = w[i] - t;
    }
}

// ----------------------------------------------------------------- host

inline hipStream_t hs(cxm_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

template <template <int> class L, class... A>
int dispatch_op(int op, A... a) {
    switch (op) {
        case CXM_OP_ADD: return L<CXM_OP_ADD>::run(a...);
        case CXM_OP_SUB: return L<CXM_OP_SUB>::run(a...);
        case CXM_OP_MUL: return L<CXM_OP_MUL>::run(a...);
        case CXM_OP_DIV: return L<CXM_OP_DIV>::run(a...);
        case CXM_OP_MAX: return L<CXM_OP_MAX>::run(a...);
        case CXM_OP_MIN: return L<CXM_OP_MIN>::run(a...);
        case CXM_OP_POW: return L<CXM_OP_POW>::run(a...);
        default: return CXM_E_INVALID;
    }
}

template <int OP>
struct BinaryL {
    static int run(const float *x, const float *y, float *z, size_t n, hipStream_t s) {
        const unsigned g = map4_grid(n);
        if (!g) return CXM_E_TOO_LARGE;
        hipLaunchKernelGGL(k_zip4<BinF<OP>>, dim3(g), dim3(kBlock), 0, s, BinF<OP>{}, x, y, z, n);
        return launch_status();
    }
};

template <int OP>
struct ScalarL {
    static int run(const float *x, float v, float *z, size_t n, hipStream_t s) {
        const unsigned g = map4_grid(n);
        if (!g) return CXM_E_TOO_LARGE;
        hipLaunchKernelGGL(k_map4<ScalarF<OP>>, dim3(g), dim3(kBlock), 0, s, ScalarF<OP>{v}, x, z, n);
        return launch_status();
    }
};

template <int OP>
struct BcastL {
    static int run(const float *x, const float *y, float *z, size_t m, size_t n, int row_mode,
                   hipStream_t s) {
        unsigned grid, tpr;
        if (!rowmap4_grid(m, n / 4, &grid, &tpr)) return CXM_E_TOO_LARGE;
        if (row_mode)
            hipLaunchKernelGGL(k_rowmap4<RowBcastF<OP>>, dim3(grid), dim3(kBlock), 0, s, RowBcastF<OP>{y}, x, z,
                               m, n / 4, tpr);
        else
            hipLaunchKernelGGL(k_rowmap4<ColBcastF<OP>>, dim3(grid), dim3(kBlock), 0, s, ColBcastF<OP>{y}, x, z,
                               m, n / 4, tpr);
        return launch_status();
    }
};

int bcast(const float *x, const float *y, float *z, size_t m, size_t n, int op, int row_mode,
          cxm_stream_t s) {
    if (!x || !y || !z || op < CXM_OP_ADD || op > CXM_OP_DIV) return CXM_E_INVALID;
    if (m == 0 || n == 0) return CXM_OK;
    if (n % 4 == 0 && aligned16(x) && aligned16(z) && (!row_mode || aligned16(y)))
        return dispatch_op<BcastL>(op, x, y, z, m, n, row_mode, hs(s));
    hipLaunchKernelGGL(k_bcast_scalar, dim3(stream_grid((m * n + 3) / 4)), dim3(kBlock), 0, hs(s), x,
                       y, z, m, n, op, row_mode);
    return launch_status();
}

template <int ACT>
int unary_t(const float *x, float *z, size_t n, hipStream_t s) {
    if (aligned16(x) && aligned16(z)) {
        const unsigned g = map4_grid(n);
        if (!g) return CXM_E_TOO_LARGE;
        hipLaunchKernelGGL(k_map4<ActF<ACT>>, dim3(g), dim3(kBlock), 0, s, ActF<ACT>{}, x, z, n);
    } else {
        hipLaunchKernelGGL(k_unary_scalar<ACT>, dim3(stream_grid((n + 3) / 4)), dim3(kBlock), 0, s, x, z, n);
    }
    return launch_status();
}

template <int ACT>
int affine_fwd_t(const float *x, const float *scale, const float *bias, float *y, size_t m,
                 size_t n, hipStream_t s) {
    unsigned grid, tpr;
    if (n % 4 == 0 && aligned16(x) && aligned16(scale) && aligned16(bias) && aligned16(y) &&
        rowmap4_grid(m, n / 4, &grid, &tpr)) {
        hipLaunchKernelGGL(k_rowmap4<AffineF<ACT>>, dim3(grid), dim3(kBlock), 0, s, AffineF<ACT>{scale, bias},
                           x, y, m, n / 4, tpr);
    } else {
        hipLaunchKernelGGL(k_affine_fwd_scalar<ACT>, dim3(stream_grid((m * n + 3) / 4)), dim3(kBlock), 0,
                           s, x, scale, bias, y, m, n);
    }
    return launch_status();
}

// Row chunks per column tile and launch order.  Measured on gfx950 at 256 MiB
// per operand, sigmoid: 512 workgroups of 4 waves (two per CU, each
// streaming a few hundred rows), one row of loads per wave in flight and
// the chunks of a tile adjacent in launch order reach 6.5 TB/s at
// [8192, 8192] and 6.7 TB/s at [1024, 65536].  Deeper unrolling (2 or 4
// rows of loads per wave, with or without a scheduling barrier that keeps
// them together), 2048 shorter workgroups, 384 workgroups (CUs unevenly
// loaded) and 16-wave workgroups were all slower, by 5-25%.
struct AffBwdPlan {
    size_t chunks;   // 0: enough for about 512 workgroups
    int tile_major;  // chunks of one tile adjacent in launch order
};

template <int ACT>
int affine_bwd_plan(const float *x, const float *scale, const float *y, const float *dy, float *dx,
                    float *dscale, float *dbias, size_t m, size_t n, AffBwdPlan plan, cxm_stream_t st) {
    const bool vec = n % 4 == 0 && aligned16(x) && aligned16(scale) && aligned16(y) &&
                     aligned16(dy) && aligned16(dx);
    const size_t ntiles = (n + kAffTile - 1) / kAffTile;
    size_t chunks = plan.chunks;
    if (chunks == 0) chunks = (512 + ntiles - 1) / ntiles;
    const size_t max_chunks = (m + 15) / 16;
    if (chunks > max_chunks) chunks = max_chunks;
    if (chunks < 1) chunks = 1;
    size_t rpc = (m + chunks - 1) / chunks;
    rpc = (rpc + 15) / 16 * 16;
    chunks = (m + rpc - 1) / rpc;
    if (chunks < 1) chunks = 1;
    if (ntiles * chunks > 0x7fffffffu) return CXM_E_TOO_LARGE;
    float *part = nullptr;
    unsigned *counters = nullptr;
    if (chunks > 1) {
        Workspace ws;
        int rc = get_workspace(st, ntiles, ntiles * chunks * 2 * kAffTile * sizeof(float), &ws);
        if (rc) return rc;
        part = static_cast<float *>(ws.scratch);
        counters = ws.counters;
    }
    const dim3 grid(static_cast<unsigned>(ntiles * chunks));
    const unsigned nt = static_cast<unsigned>(ntiles), nc = static_cast<unsigned>(chunks);
#define CXM_AFFB(VEC_)                                                                                  \
    hipLaunchKernelGGL((k_affine_bwd<ACT, VEC_, 1, 4>), grid, dim3(4 * kWave), 0, hs(st), x, scale, y, dy, dx,    \
                       dscale, dbias, m, n, nt, nc, rpc, plan.tile_major, part, counters)
    if (vec) CXM_AFFB(true);
    else CXM_AFFB(false);
#undef CXM_AFFB
    return launch_status();
}

template <int ACT>
int affine_bwd_t(const float *x, const float *scale, const float *y, const float *dy, float *dx,
                 float *dscale, float *dbias, size_t m, size_t n, cxm_stream_t st) {
    return affine_bwd_plan<ACT>(x, scale, y, dy, dx, dscale, dbias, m, n, AffBwdPlan{0, 1}, st);
}

// ------------------------------------------------- sum / mean backward

// dx[o, d, i] = g(dz[o, i]) over dx as row-major [outer, dim, inner], with
// g(v) = v for a sum and v / dim for a mean.  One float4 of dx per thread
// (the grid of k_map4).  MODE 0: inner == 1 and dim % 4 == 0, so a float4
// lies in one row o and repeats dz[o]; MODE 1: inner % 4 == 0, a float4 is
// four consecutive inner indices of one (o, d), read as a float4 of dz;
// MODE 2: any shape or alignment, element by element.
template <bool MEAN, int MODE>
__global__ __launch_bounds__(kBlock) void k_sum_bwd(const float *__restrict__ dz, float *__restrict__ dx, size_t dim,
                                                    size_t inner, size_t n, float dimf) {
    const size_t t = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;
    const size_t e = 4 * t;
    if (e >= n) return;
    auto g = [dimf](float v) { return MEAN ? v / dimf : v; };
    if constexpr (MODE == 0) {
        const float v = g(dz[e / dim]);
        st4_stream(dx + e, make_float4(v, v, v, v));
    } else if constexpr (MODE == 1) {
        const size_t slab = dim * inner;
        const size_t o = e / slab, i = e % inner;
        const float4 v = ld4(dz + o * inner + i);
        st4_stream(dx + e, make_float4(g(v.x), g(v.y), g(v.z), g(v.w)));
    } else {
        const size_t slab = dim * inner;
        for (size_t k = e; k < e + 4 && k < n; ++k) dx[k] = g(dz[(k / slab) * inner + k % inner]);
    }
}

template <bool MEAN>
int sum_bwd_t(const float *dz, float *dx, size_t outer, size_t dim, size_t inner, hipStream_t s) {
    const size_t n = outer * dim * inner;
    const unsigned grid = map4_grid(n + 3);
    if (!grid) return CXM_E_TOO_LARGE;
    const float dimf = static_cast<float>(dim);
    if (aligned16(dx) && inner == 1 && dim % 4 == 0)
        hipLaunchKernelGGL((k_sum_bwd<MEAN, 0>), dim3(grid), dim3(kBlock), 0, s, dz, dx, dim, inner, n, dimf);
    else if (aligned16(dx) && aligned16(dz) && inner % 4 == 0)
        hipLaunchKernelGGL((k_sum_bwd<MEAN, 1>), dim3(grid), dim3(kBlock), 0, s, dz, dx, dim, inner, n, dimf);
    else
        hipLaunchKernelGGL((k_sum_bwd<MEAN, 2>), dim3(grid), dim3(kBlock), 0, s, dz, dx, dim, inner, n, dimf);
    return launch_status();
}

}  // namespace
}  // namespace cxm

using namespace cxm;

extern "C" {

int cxm_binary_f32(const float *x, const float *y, float *z, size_t n, int op, cxm_stream_t s) {
    if (!x || !y || !z || op < CXM_OP_ADD || op > CXM_OP_POW) return CXM_E_INVALID;
    if (n == 0) return CXM_OK;
    if (aligned16(x) && aligned16(y) && aligned16(z)) return dispatch_op<BinaryL>(op, x, y, z, n, hs(s));
    hipLaunchKernelGGL(k_binary_scalar, dim3(stream_grid((n + 3) / 4)), dim3(kBlock), 0, hs(s), x, y, z,
                       n, op);
    return launch_status();
}

int cxm_bcast_row_f32(const float *x, const float *y, float *z, size_t m, size_t n, int op,
                      cxm_stream_t s) {
    return bcast(x, y, z, m, n, op, 1, s);
}

int cxm_bcast_col_f32(const float *x, const float *y, float *z, size_t m, size_t n, int op,
                      cxm_stream_t s) {
    return bcast(x, y, z, m, n, op, 0, s);
}

int cxm_scalar_f32(const float *x, float value, float *z, size_t n, int op, cxm_stream_t s) {
    if (!x || !z || op < CXM_OP_ADD || op > CXM_OP_POW) return CXM_E_INVALID;
    if (n == 0) return CXM_OK;
    if (aligned16(x) && aligned16(z)) return dispatch_op<ScalarL>(op, x, value, z, n, hs(s));
    hipLaunchKernelGGL(k_scalar_scalar, dim3(stream_grid((n + 3) / 4)), dim3(kBlock), 0, hs(s), x, value,
                       z, n, op);
    return launch_status();
}

int cxm_unary_f32(const float *x, float *z, size_t n, int act, cxm_stream_t s) {
    if (!x || !z) return CXM_E_INVALID;
    if (n == 0) return CXM_OK;
    switch (act) {
        case CXM_ACT_RELU: return unary_t<CXM_ACT_RELU>(x, z, n, hs(s));
        case CXM_ACT_SIGMOID: return unary_t<CXM_ACT_SIGMOID>(x, z, n, hs(s));
        case CXM_ACT_TANH: return unary_t<CXM_ACT_TANH>(x, z, n, hs(s));
        case CXM_ACT_EXP: return unary_t<CXM_ACT_EXP>(x, z, n, hs(s));
        default: return CXM_E_INVALID;
    }
}

int cxm_affine_act_fwd_f32(const float *x, const float *scale, const float *bias, float *y,
                           size_t m, size_t n, int act, cxm_stream_t s) {
    if (!x || !scale || !bias || !y) return CXM_E_INVALID;
    if (m == 0 || n == 0) return CXM_OK;
    switch (act) {
        case CXM_ACT_NONE: return affine_fwd_t<CXM_ACT_NONE>(x, scale, bias, y, m, n, hs(s));
        case CXM_ACT_RELU: return affine_fwd_t<CXM_ACT_RELU>(x, scale, bias, y, m, n, hs(s));
        case CXM_ACT_SIGMOID: return affine_fwd_t<CXM_ACT_SIGMOID>(x, scale, bias, y, m, n, hs(s));
        case CXM_ACT_TANH: return affine_fwd_t<CXM_ACT_TANH>(x, scale, bias, y, m, n, hs(s));
        default: return CXM_E_INVALID;
    }
}

int cxm_affine_act_bwd_f32(const float *x, const float *scale, const float *y, const float *dy,
                           float *dx, float *dscale, float *dbias, size_t m, size_t n, int act,
                           cxm_stream_t s) {
    if (!x || !scale || !y || !dy || !dx || !dscale || !dbias) return CXM_E_INVALID;
    if (n == 0) return CXM_OK;
    if (m == 0) return CXM_E_INVALID;  // column sums over zero rows are undefined in the reference
    switch (act) {
        case CXM_ACT_NONE:
            return affine_bwd_t<CXM_ACT_NONE>(x, scale, y, dy, dx, dscale, dbias, m, n, s);
        case CXM_ACT_RELU:
            return affine_bwd_t<CXM_ACT_RELU>(x, scale, y, dy, dx, dscale, dbias, m, n, s);
        case CXM_ACT_SIGMOID:
            return affine_bwd_t<CXM_ACT_SIGMOID>(x, scale, y, dy, dx, dscale, dbias, m, n, s);
        case CXM_ACT_TANH:
            return affine_bwd_t<CXM_ACT_TANH>(x, scale, y, dy, dx, dscale, dbias, m, n, s);
        default: return CXM_E_INVALID;
    }
}

int cxm_act_bwd_f32(const float *y, const float *dy, float *dx, size_t n, int act, cxm_stream_t s) {
    if (!y || !dy || !dx || act < CXM_ACT_RELU || act > CXM_ACT_TANH) return CXM_E_INVALID;
    if (n == 0) return CXM_OK;
    if (!(aligned16(y) && aligned16(dy) && aligned16(dx))) {
        hipLaunchKernelGGL(k_act_bwd_scalar, dim3(stream_grid((n + 3) / 4)), dim3(kBlock), 0, hs(s), y, dy, dx, n,
                           act);
        return launch_status();
    }
    const unsigned g = map4_grid(n);
    if (!g) return CXM_E_TOO_LARGE;
    switch (act) {
        case CXM_ACT_RELU:
            hipLaunchKernelGGL(k_zip4<ActBwdF<CXM_ACT_RELU>>, dim3(g), dim3(kBlock), 0, hs(s), ActBwdF<CXM_ACT_RELU>{},
                               y, dy, dx, n);
            break;
        case CXM_ACT_SIGMOID:
            hipLaunchKernelGGL(k_zip4<ActBwdF<CXM_ACT_SIGMOID>>, dim3(g), dim3(kBlock), 0, hs(s),
                               ActBwdF<CXM_ACT_SIGMOID>{}, y, dy, dx, n);
            break;
        default:
            hipLaunchKernelGGL(k_zip4<ActBwdF<CXM_ACT_TANH>>, dim3(g), dim3(kBlock), 0, hs(s), ActBwdF<CXM_ACT_TANH>{},
                               y, dy, dx, n);
    }
    return launch_status();
}

int cxm_reduce_sum_bwd_f32(const float *dz, float *dx, size_t outer, size_t dim, size_t inner, int mean,
                           cxm_stream_t s) {
    if (!dz || !dx || (mean != 0 && mean != 1)) return CXM_E_INVALID;
    if (outer == 0 || dim == 0 || inner == 0) return CXM_OK;
    if (outer > SIZE_MAX / dim / inner) return CXM_E_TOO_LARGE;
    return mean ? sum_bwd_t<true>(dz, dx, outer, dim, inner, hs(s)) : sum_bwd_t<false>(dz, dx, outer, dim, inner, hs(s));
}

int cxm_sgd_f32(float *w, const float *g, float lr, size_t n, cxm_stream_t s) {
    if (!w || !g) return CXM_E_INVALID;
    if (n == 0) return CXM_OK;
    if (aligned16(w) && aligned16(g)) {
        const unsigned grid = map4_grid(n);
        if (!grid) return CXM_E_TOO_LARGE;
        hipLaunchKernelGGL(k_zip4<SgdF>, dim3(grid), dim3(kBlock), 0, hs(s), SgdF{lr}, w, g, w, n);
    } else {
        hipLaunchKernelGGL(k_sgd_scalar, dim3(stream_grid((n + 3) / 4)), dim3(kBlock), 0, hs(s), w, g, lr, n);
    }
    return launch_status();
}

}  // extern "C"
