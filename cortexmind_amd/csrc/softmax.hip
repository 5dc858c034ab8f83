// Row softmax / log-softmax over the last axis, forward and backward, and
// the softmax cross-entropy of the MLP step.
//
// The reference has no softmax; its composition of reference primitives is
//   m = reduce::max (source/CortexMind/framework/Engine/AVX2/reduce.cpp:204-215,
//       lanes start at -FLT_MAX), z = Broadcast::col::sub(x, m)
//       (broadcast.cpp:292-304), e = exp(z), s = reduce::sum(e)
//       (reduce.cpp:17-28), y = Broadcast::col::div(e, s) (broadcast.cpp:320-332)
//       or y = z - log(s),
// and these kernels compute that per element (z = x - m rounded, then expf,
// then a subtraction of log(s), or a product with the correctly rounded 1/s
// in place of the division: at most one rounding apart); the order in
// which s is summed differs.
//
// Three kernel families by row length:
//  * wave per row, row in registers (cols <= 4096, cols % 4 == 0): one pass
//    over HBM, DPP wave reductions, no LDS;
//  * split rows (long rows): pass 1 reduces each 4096-element segment to
//    (max m_b, sum_b exp(x - m_b)) [forward] or to its partial dot product
//    [backward]; pass 2 combines the row's partials in segment order
//    (S = sum_b s_b * exp(m_b - M)), re-reads its segment and writes;
//  * any shape or alignment: wave per row, three sweeps over the row.
// The running max starts from -FLT_MAX, as reduce::max does, so an
// all -inf row (or segment) never forms (-inf) - (-inf).
#include "cxm_common.hpp"

namespace cxm {
namespace {

constexpr float kLowest = -FLT_MAX;

// ------------------------------------------------- wave per row, registers

// NV float4 per lane: cols <= 256 * NV.  WPB rows (one per wave) per workgroup.
template <int NV, bool LOG, int WPB = kWavesPerBlock>
__global__ __launch_bounds__(WPB * kWave) void k_sm_fwd_wave(const float *__restrict__ x,
                                                             float *__restrict__ y, size_t rows,
                                                             size_t cols) {
    const size_t row = static_cast<size_t>(blockIdx.x) * WPB + threadIdx.x / kWave;
    if (row >= rows) return;  // whole waves leave together
    const int lane = threadIdx.x & (kWave - 1);
    const float *__restrict__ xr = x + row * cols;
    float *__restrict__ yr = y + row * cols;
    const size_t c4 = cols / 4;
    float4 v[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const size_t i = static_cast<size_t>(k) * kWave + lane;
        v[k] = i < c4 ? ld4_stream(xr + 4 * i) : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
    }
    float m = kLowest;
#pragma unroll
    for (int k = 0; k < NV; ++k) m = vmax(vmax(vmax(vmax(m, v[k].x), v[k].y), v[k].z), v[k].w);
    m = wave_reduce<MaxOp>(m);
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        v[k].x = v[k].x - m; v[k].y = v[k].y - m; v[k].z = v[k].z - m; v[k].w = v[k].w - m;
        if constexpr (LOG) {
            s += (expf(v[k].x) + expf(v[k].y)) + (expf(v[k].z) + expf(v[k].w));
        } else {  // keep e = exp(z) for the output
            v[k] = make_float4(expf(v[k].x), expf(v[k].y), expf(v[k].z), expf(v[k].w));
            s += (v[k].x + v[k].y) + (v[k].z + v[k].w);
        }
    }
    s = wave_reduce<SumOp>(s);
    if constexpr (LOG) {
        const float ls = logf(s);
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const size_t i = static_cast<size_t>(k) * kWave + lane;
            if (i < c4)
                st4_stream(yr + 4 * i, make_float4(v[k].x - ls, v[k].y - ls, v[k].z - ls, v[k].w - ls));
        }
    } else {
        const float inv = 1.0f / s;  // e * rn(1/s): one rounding from e / s
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const size_t i = static_cast<size_t>(k) * kWave + lane;
            if (i < c4) st4_stream(yr + 4 * i, make_float4(v[k].x * inv, v[k].y * inv, v[k].z * inv, v[k].w * inv));
        }
    }
}

// Backward from the saved output: softmax dx = y*(dy - sum(dy*y)),
// log-softmax dx = dy - exp(y)*sum(dy).
template <int NV, bool LOG, int WPB = kWavesPerBlock>
__global__ __launch_bounds__(WPB * kWave) void k_sm_bwd_wave(const float *__restrict__ y,
                                                             const float *__restrict__ dy,
                                                             float *__restrict__ dx, size_t rows,
                                                             size_t cols) {
    const size_t row = static_cast<size_t>(blockIdx.x) * WPB + threadIdx.x / kWave;
    if (row >= rows) return;
    const int lane = threadIdx.x & (kWave - 1);
    const size_t off = row * cols;
    const size_t c4 = cols / 4;
    const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
    float4 yv[NV], gv[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const size_t i = static_cast<size_t>(k) * kWave + lane;
        yv[k] = i < c4 ? ld4_stream(y + off + 4 * i) : zero;
        gv[k] = i < c4 ? ld4_stream(dy + off + 4 * i) : zero;
    }
    float r = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        if constexpr (LOG) r += (gv[k].x + gv[k].y) + (gv[k].z + gv[k].w);
        else r += (gv[k].x * yv[k].x + gv[k].y * yv[k].y) + (gv[k].z * yv[k].z + gv[k].w * yv[k].w);
    }
    r = wave_reduce<SumOp>(r);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const size_t i = static_cast<size_t>(k) * kWave + lane;
        if (i >= c4) continue;
        float4 o;
        if constexpr (LOG) {
            o.x = gv[k].x - expf(yv[k].x) * r; o.y = gv[k].y - expf(yv[k].y) * r;
            o.z = gv[k].z - expf(yv[k].z) * r; o.w = gv[k].w - expf(yv[k].w) * r;
        } else {
            o.x = yv[k].x * (gv[k].x - r); o.y = yv[k].y * (gv[k].y - r);
            o.z = yv[k].z * (gv[k].z - r); o.w = yv[k].w * (gv[k].w - r);
        }
        st4_stream(dx + off + 4 * i, o);
    }
}

// ------------------------------------------------------------ split rows

// Segment = NV float4 per thread of a 256-thread workgroup (1024*NV floats).
constexpr int kSegNV = 4;

struct MS {
    float m, s;
};
// Pass 1 forward: per (row, segment) the segment max m_b and
// s_b = sum exp(x - m_b).  A segment is NV float4 per thread, streamed in
// chunks of 4 float4 with the next chunk's loads in flight while the
// current one is folded into the thread's running (max, sum) -- the
// online rescaling s = s*exp(m - m') + sum exp(x - m') of Milakov and
// Gimelshein (2018).  Then a block max, one rescale per thread, and a block
// sum.  grid = rows * segs.
template <int NV>
__global__ __launch_bounds__(kBlock) void k_sm_fwd_part(const float *__restrict__ x, size_t cols,
                                                        unsigned segs, MS *__restrict__ part) {
    constexpr size_t L = kBlock * 4 * NV;
    constexpr int C = NV < 4 ? NV : 4;  // float4 per thread per chunk
    static_assert(NV % C == 0, "segment = whole chunks");
    __shared__ float lds[kWavesPerBlock];
    const size_t row = blockIdx.x / segs;
    const unsigned seg = blockIdx.x - static_cast<unsigned>(row) * segs;
    const float *__restrict__ xs = x + row * cols + static_cast<size_t>(seg) * L;
    const size_t n4 = (cols - static_cast<size_t>(seg) * L) / 4;  // float4 left in the row
    const float4 ninf = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
    float4 cur[C], nxt[C];
#pragma unroll
    for (int k = 0; k < C; ++k) {
        const size_t i = static_cast<size_t>(k) * kBlock + threadIdx.x;
        cur[k] = i < n4 ? ld4(xs + 4 * i) : ninf;
    }
    float m = kLowest, s = 0.0f;
#pragma unroll
    for (int c = 0; c < NV / C; ++c) {
        if (c + 1 < NV / C) {
#pragma unroll
            for (int k = 0; k < C; ++k) {
                const size_t i = static_cast<size_t>((c + 1) * C + k) * kBlock + threadIdx.x;
                nxt[k] = i < n4 ? ld4(xs + 4 * i) : ninf;
            }
        }
        float mc = m;
#pragma unroll
        for (int k = 0; k < C; ++k) mc = vmax(vmax(vmax(vmax(mc, cur[k].x), cur[k].y), cur[k].z), cur[k].w);
        float sc = s * expf(m - mc);
#pragma unroll
        for (int k = 0; k < C; ++k)
            sc += (expf(cur[k].x - mc) + expf(cur[k].y - mc)) + (expf(cur[k].z - mc) + expf(cur[k].w - mc));
        m = mc;
        s = sc;
#pragma unroll
        for (int k = 0; k < C; ++k) cur[k] = nxt[k];
    }
    const float M = block_reduce<MaxOp, kBlock>(m, lds);
    const float S = block_reduce<SumOp, kBlock>(s * expf(m - M), lds);
    if (threadIdx.x == 0) part[blockIdx.x] = MS{M, S};
}

// Row max M and S = sum_b s_b * exp(m_b - M) from the row's partials, in a
// fixed order, so every workgroup of the row computes identical values.
__device__ __forceinline__ MS combine_row(const MS *__restrict__ p, unsigned segs, float *lds) {
    float m = kLowest;
    for (unsigned b = threadIdx.x; b < segs; b += kBlock) m = vmax(m, p[b].m);
    m = block_reduce<MaxOp, kBlock>(m, lds);
    float s = 0.0f;
    for (unsigned b = threadIdx.x; b < segs; b += kBlock) s += p[b].s * expf(p[b].m - m);
    s = block_reduce<SumOp, kBlock>(s, lds);
    return MS{m, s};
}

// Pass 2 forward: y = exp(x - M) * (1/S), or (x - M) - log(S).  The
// correctly rounded reciprocal times e differs from e / S by at most one
// rounding, and saves the per-element division.  Chunks of 4 float4 per
// thread, the next chunk's loads in flight while the current one is
// written.
template <int NV, bool LOG>
__global__ __launch_bounds__(kBlock) void k_sm_fwd_apply(const float *__restrict__ x,
                                                         float *__restrict__ y, size_t cols,
                                                         unsigned segs, const MS *__restrict__ part) {
    constexpr size_t L = kBlock * 4 * NV;
    constexpr int C = NV < 4 ? NV : 4;
    static_assert(NV % C == 0, "segment = whole chunks");
    __shared__ float lds[kWavesPerBlock];
    const size_t row = blockIdx.x / segs;
    const unsigned seg = blockIdx.x - static_cast<unsigned>(row) * segs;
    const size_t base = row * cols + static_cast<size_t>(seg) * L;
    const size_t n4 = (cols - static_cast<size_t>(seg) * L) / 4;
    float4 cur[C], nxt[C];
#pragma unroll
    for (int k = 0; k < C; ++k) {
        const size_t i = static_cast<size_t>(k) * kBlock + threadIdx.x;
        if (i < n4) cur[k] = ld4_stream(x + base + 4 * i);
    }
    const MS t = combine_row(part + row * segs, segs, lds);
    const float ls = LOG ? logf(t.s) : 0.0f;
    const float inv = LOG ? 0.0f : 1.0f / t.s;
#pragma unroll
    for (int c = 0; c < NV / C; ++c) {
        if (c + 1 < NV / C) {
#pragma unroll
            for (int k = 0; k < C; ++k) {
                const size_t i = static_cast<size_t>((c + 1) * C + k) * kBlock + threadIdx.x;
                if (i < n4) nxt[k] = ld4_stream(x + base + 4 * i);
            }
        }
#pragma unroll
        for (int k = 0; k < C; ++k) {
            const size_t i = static_cast<size_t>(c * C + k) * kBlock + threadIdx.x;
            if (i >= n4) continue;
            float4 z;
            z.x = cur[k].x - t.m; z.y = cur[k].y - t.m; z.z = cur[k].z - t.m; z.w = cur[k].w - t.m;
            float4 o;
            if constexpr (LOG) {
                o = make_float4(z.x - ls, z.y - ls, z.z - ls, z.w - ls);
            } else {
                o = make_float4(expf(z.x) * inv, expf(z.y) * inv, expf(z.z) * inv, expf(z.w) * inv);
            }
            st4_stream(y + base + 4 * i, o);
        }
#pragma unroll
        for (int k = 0; k < C; ++k) cur[k] = nxt[k];
    }
}

// Pass 1 backward: per (row, segment) partial of sum(dy*y) or sum(dy).
template <int NV, bool LOG>
__global__ __launch_bounds__(kBlock) void k_sm_bwd_part(const float *__restrict__ y,
                                                        const float *__restrict__ dy, size_t cols,
                                                        unsigned segs, float *__restrict__ part) {
    constexpr size_t L = kBlock * 4 * NV;
    __shared__ float lds[kWavesPerBlock];
    const size_t row = blockIdx.x / segs;
    const unsigned seg = blockIdx.x - static_cast<unsigned>(row) * segs;
    const size_t base = row * cols + static_cast<size_t>(seg) * L;
    const size_t n4 = (cols - static_cast<size_t>(seg) * L) / 4;
    float4 g[NV], yy[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const size_t i = static_cast<size_t>(k) * kBlock + threadIdx.x;
        const bool in = i < n4;
        g[k] = in ? ld4(dy + base + 4 * i) : make_float4(0.f, 0.f, 0.f, 0.f);
        if constexpr (!LOG) yy[k] = in ? ld4(y + base + 4 * i) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float r = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        if constexpr (LOG) r += (g[k].x + g[k].y) + (g[k].z + g[k].w);
        else r += (g[k].x * yy[k].x + g[k].y * yy[k].y) + (g[k].z * yy[k].z + g[k].w * yy[k].w);
    }
    r = block_reduce<SumOp, kBlock>(r, lds);
    if (threadIdx.x == 0) part[blockIdx.x] = r;
}

template <int NV, bool LOG>
__global__ __launch_bounds__(kBlock) void k_sm_bwd_apply(const float *__restrict__ y,
                                                         const float *__restrict__ dy,
                                                         float *__restrict__ dx, size_t cols,
                                                         unsigned segs,
                                                         const float *__restrict__ part) {
    constexpr size_t L = kBlock * 4 * NV;
    __shared__ float lds[kWavesPerBlock];
    const size_t row = blockIdx.x / segs;
    const unsigned seg = blockIdx.x - static_cast<unsigned>(row) * segs;
    float r = 0.0f;
    for (unsigned b = threadIdx.x; b < segs; b += kBlock) r += part[row * segs + b];
    r = block_reduce<SumOp, kBlock>(r, lds);
    const size_t base = row * cols + static_cast<size_t>(seg) * L;
    const size_t n4 = (cols - static_cast<size_t>(seg) * L) / 4;
    float4 yy[NV], g[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const size_t i = static_cast<size_t>(k) * kBlock + threadIdx.x;
        if (i < n4) {
            yy[k] = ld4_stream(y + base + 4 * i);
            g[k] = ld4_stream(dy + base + 4 * i);
        }
    }
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const size_t i = static_cast<size_t>(k) * kBlock + threadIdx.x;
        if (i >= n4) continue;
        float4 o;
        if constexpr (LOG) {
            o.x = g[k].x - expf(yy[k].x) * r; o.y = g[k].y - expf(yy[k].y) * r;
            o.z = g[k].z - expf(yy[k].z) * r; o.w = g[k].w - expf(yy[k].w) * r;
        } else {
            o.x = yy[k].x * (g[k].x - r); o.y = yy[k].y * (g[k].y - r);
            o.z = yy[k].z * (g[k].z - r); o.w = yy[k].w * (g[k].w - r);
        }
        st4_stream(dx + base + 4 * i, o);
    }
}

// --------------------------------------------------- generic (any shape)

// Wave per row, three sweeps; handles every column count and alignment.
template <bool LOG>
__global__ __launch_bounds__(kBlock) void k_sm_fwd_any(const float *__restrict__ x,
                                                       float *__restrict__ y, size_t rows,
                                                       size_t cols) {
    const size_t row = static_cast<size_t>(blockIdx.x) * kWavesPerBlock + threadIdx.x / kWave;
    if (row >= rows) return;
    const int lane = threadIdx.x & (kWave - 1);
    const float *__restrict__ xr = x + row * cols;
    float *__restrict__ yr = y + row * cols;
    float m = kLowest;
    for (size_t j = lane; j < cols; j += kWave) m = vmax(m, xr[j]);
    m = wave_reduce<MaxOp>(m);
    float s = 0.0f;
    for (size_t j = lane; j < cols; j += kWave) s += expf(xr[j] - m);
    s = wave_reduce<SumOp>(s);
    const float ls = LOG ? logf(s) : 0.0f;
    for (size_t j = lane; j < cols; j += kWave) {
        const float z = xr[j] - m;
        yr[j] = LOG ? z - ls : expf(z) / s;
    }
}

template <bool LOG>
__global__ __launch_bounds__(kBlock) void k_sm_bwd_any(const float *__restrict__ y,
                                                       const float *__restrict__ dy,
                                                       float *__restrict__ dx, size_t rows,
                                                       size_t cols) {
    const size_t row = static_cast<size_t>(blockIdx.x) * kWavesPerBlock + threadIdx.x / kWave;
    if (row >= rows) return;
    const int lane = threadIdx.x & (kWave - 1);
    const size_t off = row * cols;
    float r = 0.0f;
    for (size_t j = lane; j < cols; j += kWave) r += LOG ? dy[off + j] : dy[off + j] * y[off + j];
    r = wave_reduce<SumOp>(r);
    for (size_t j = lane; j < cols; j += kWave) {
        const float yy = y[off + j], g = dy[off + j];
        dx[off + j] = LOG ? g - expf(yy) * r : yy * (g - r);
    }
}

// ------------------------------------------------ softmax cross-entropy

// One thread per row of [b, c] logits: nll_r = log(s) - z_label, and
// dlogits = (softmax - onehot) * rn(1/b).  Per-workgroup nll sums go to the
// workspace; the last workgroup adds them in order and writes the mean.
// A label outside [0, c) is never used as an index: that row's nll is NaN,
// so the loss comes out NaN (no host round trip to validate labels).
__global__ __launch_bounds__(kBlock) void k_xent(const float *__restrict__ logits,
                                                 const int32_t *__restrict__ labels,
                                                 float *__restrict__ loss, float *__restrict__ dl,
                                                 size_t b, size_t c, float inv_b,
                                                 float *__restrict__ part,
                                                 unsigned *__restrict__ counter) {
    __shared__ float lds[kWavesPerBlock];
    __shared__ int flag;
    const size_t r = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;
    float nll = 0.0f;
    if (r < b) {
        const float *__restrict__ xr = logits + r * c;
        float *__restrict__ dr = dl + r * c;
        const int32_t lab = labels[r];
        const bool ok = lab >= 0 && static_cast<size_t>(lab) < c;
        float m = kLowest;
        for (size_t j = 0; j < c; ++j) m = vmax(m, xr[j]);
        float s = 0.0f;
        for (size_t j = 0; j < c; ++j) s += expf(xr[j] - m);
        for (size_t j = 0; j < c; ++j) {
            float p = expf(xr[j] - m) / s;
            if (static_cast<int32_t>(j) == lab) p = p - 1.0f;
            dr[j] = p * inv_b;
        }
        if (ok) {
            const float zl = xr[lab] - m;
            const float yl = zl - logf(s);
            nll = -yl;
        } else {
            nll = NAN;
        }
    }
    nll = block_reduce<SumOp, kBlock>(nll, lds);
    if (gridDim.x == 1) {
        if (threadIdx.x == 0) loss[0] = nll / static_cast<float>(b);
        return;
    }
    if (threadIdx.x == 0) st_dev(&part[blockIdx.x], nll);
    if (!last_block_ticket(counter, gridDim.x, &flag)) return;
    const unsigned mine = threadIdx.x < gridDim.x ? (gridDim.x - threadIdx.x + kBlock - 1) / kBlock : 0;
    float t = combine_partials<SumOp>(part + threadIdx.x, mine, kBlock, 0.0f);
    t = block_reduce<SumOp, kBlock>(t, lds);
    if (threadIdx.x == 0) loss[0] = t / static_cast<float>(b);
}

// ------------------------------------------------------------------ host

inline hipStream_t hs(cxm_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

constexpr size_t kWaveRowMax = 256 * 16;  // wave-per-row kernel holds up to 4096 columns

// Two rows (waves) per workgroup: measured on [512, 1024] as 3.35 us per
// launch against 3.5-3.8 us with four or eight rows per workgroup (more
// workgroups spread the rows over more CUs).
constexpr int kSmWpb = 2;

template <bool LOG>
int sm_fwd_wave(const float *x, float *y, size_t rows, size_t cols, hipStream_t s) {
    const dim3 grid(ceil_div(rows, kSmWpb)), block(kSmWpb * kWave);
    const size_t nv = (cols + 255) / 256;
    if (nv <= 1) hipLaunchKernelGGL((k_sm_fwd_wave<1, LOG, kSmWpb>), grid, block, 0, s, x, y, rows, cols);
    else if (nv <= 2) hipLaunchKernelGGL((k_sm_fwd_wave<2, LOG, kSmWpb>), grid, block, 0, s, x, y, rows, cols);
    else if (nv <= 4) hipLaunchKernelGGL((k_sm_fwd_wave<4, LOG, kSmWpb>), grid, block, 0, s, x, y, rows, cols);
    else if (nv <= 8) hipLaunchKernelGGL((k_sm_fwd_wave<8, LOG, kSmWpb>), grid, block, 0, s, x, y, rows, cols);
    else hipLaunchKernelGGL((k_sm_fwd_wave<16, LOG, kSmWpb>), grid, block, 0, s, x, y, rows, cols);
    return launch_status();
}

template <bool LOG>
int sm_bwd_wave(const float *y, const float *dy, float *dx, size_t rows, size_t cols, hipStream_t s) {
    const dim3 grid(ceil_div(rows, kSmWpb)), block(kSmWpb * kWave);
    const size_t nv = (cols + 255) / 256;
    if (nv <= 1) hipLaunchKernelGGL((k_sm_bwd_wave<1, LOG, kSmWpb>), grid, block, 0, s, y, dy, dx, rows, cols);
    else if (nv <= 2) hipLaunchKernelGGL((k_sm_bwd_wave<2, LOG, kSmWpb>), grid, block, 0, s, y, dy, dx, rows, cols);
    else if (nv <= 4) hipLaunchKernelGGL((k_sm_bwd_wave<4, LOG, kSmWpb>), grid, block, 0, s, y, dy, dx, rows, cols);
    else if (nv <= 8) hipLaunchKernelGGL((k_sm_bwd_wave<8, LOG, kSmWpb>), grid, block, 0, s, y, dy, dx, rows, cols);
    else hipLaunchKernelGGL((k_sm_bwd_wave<16, LOG, kSmWpb>), grid, block, 0, s, y, dy, dx, rows, cols);
    return launch_status();
}

// Long rows: split when a row exceeds the wave kernel's register capacity.
bool use_split(size_t cols) { return cols > kWaveRowMax; }

template <int NV>
int sm_fwd_split(const float *x, float *y, size_t rows, size_t cols, int log_mode, cxm_stream_t st) {
    constexpr size_t L = kBlock * 4 * NV;
    const size_t segs = (cols + L - 1) / L;
    if (rows * segs > 0x7fffffffu) return CXM_E_TOO_LARGE;
    Workspace ws;
    int rc = get_workspace(st, 0, rows * segs * sizeof(MS), &ws);
    if (rc) return rc;
    MS *part = static_cast<MS *>(ws.scratch);
    const dim3 grid(static_cast<unsigned>(rows * segs));
    hipStream_t s = hs(st);
    hipLaunchKernelGGL(k_sm_fwd_part<NV>, grid, dim3(kBlock), 0, s, x, cols, static_cast<unsigned>(segs), part);
    if ((rc = launch_status())) return rc;
    if (log_mode)
        hipLaunchKernelGGL((k_sm_fwd_apply<NV, true>), grid, dim3(kBlock), 0, s, x, y, cols,
                           static_cast<unsigned>(segs), part);
    else
        hipLaunchKernelGGL((k_sm_fwd_apply<NV, false>), grid, dim3(kBlock), 0, s, x, y, cols,
                           static_cast<unsigned>(segs), part);
    return launch_status();
}

template <int NV>
int sm_bwd_split(const float *y, const float *dy, float *dx, size_t rows, size_t cols, int log_mode,
                 cxm_stream_t st) {
    constexpr size_t L = kBlock * 4 * NV;
    const size_t segs = (cols + L - 1) / L;
    if (rows * segs > 0x7fffffffu) return CXM_E_TOO_LARGE;
    Workspace ws;
    int rc = get_workspace(st, 0, rows * segs * sizeof(float), &ws);
    if (rc) return rc;
    float *part = static_cast<float *>(ws.scratch);
    const dim3 grid(static_cast<unsigned>(rows * segs));
    hipStream_t s = hs(st);
    const unsigned sg = static_cast<unsigned>(segs);
    if (log_mode) {
        hipLaunchKernelGGL((k_sm_bwd_part<NV, true>), grid, dim3(kBlock), 0, s, y, dy, cols, sg, part);
        if ((rc = launch_status())) return rc;
        hipLaunchKernelGGL((k_sm_bwd_apply<NV, true>), grid, dim3(kBlock), 0, s, y, dy, dx, cols, sg, part);
    } else {
        hipLaunchKernelGGL((k_sm_bwd_part<NV, false>), grid, dim3(kBlock), 0, s, y, dy, cols, sg, part);
        if ((rc = launch_status())) return rc;
        hipLaunchKernelGGL((k_sm_bwd_apply<NV, false>), grid, dim3(kBlock), 0, s, y, dy, dx, cols, sg, part);
    }
    return launch_status();
}

int softmax_fwd(const float *x, float *y, size_t rows, size_t cols, int log_mode, cxm_stream_t st) {
    if (!x || !y || (log_mode != 0 && log_mode != 1)) return CXM_E_INVALID;
    if (rows == 0 || cols == 0) return CXM_OK;
    hipStream_t s = hs(st);
    const bool vec = cols % 4 == 0 && aligned16(x) && aligned16(y);
    if (!vec) {
        const dim3 grid(ceil_div(rows, kWavesPerBlock));
        if (log_mode) hipLaunchKernelGGL(k_sm_fwd_any<true>, grid, dim3(kBlock), 0, s, x, y, rows, cols);
        else hipLaunchKernelGGL(k_sm_fwd_any<false>, grid, dim3(kBlock), 0, s, x, y, rows, cols);
        return launch_status();
    }
    if (!use_split(cols))
        return log_mode ? sm_fwd_wave<true>(x, y, rows, cols, s) : sm_fwd_wave<false>(x, y, rows, cols, s);
    return sm_fwd_split<kSegNV>(x, y, rows, cols, log_mode, st);
}

int softmax_bwd(const float *y, const float *dy, float *dx, size_t rows, size_t cols, int log_mode,
                cxm_stream_t st) {
    if (!y || !dy || !dx || (log_mode != 0 && log_mode != 1)) return CXM_E_INVALID;
    if (rows == 0 || cols == 0) return CXM_OK;
    hipStream_t s = hs(st);
    const bool vec = cols % 4 == 0 && aligned16(y) && aligned16(dy) && aligned16(dx);
    if (!vec) {
        const dim3 grid(ceil_div(rows, kWavesPerBlock));
        if (log_mode) hipLaunchKernelGGL(k_sm_bwd_any<true>, grid, dim3(kBlock), 0, s, y, dy, dx, rows, cols);
        else hipLaunchKernelGGL(k_sm_bwd_any<false>, grid, dim3(kBlock), 0, s, y, dy, dx, rows, cols);
        return launch_status();
    }
    if (!use_split(cols))
        return log_mode ? sm_bwd_wave<true>(y, dy, dx, rows, cols, s)
                        : sm_bwd_wave<false>(y, dy, dx, rows, cols, s);
    return sm_bwd_split<kSegNV>(y, dy, dx, rows, cols, log_mode, st);
}

}  // namespace
}  // namespace cxm

using namespace cxm;

extern "C" {

int cxm_softmax_fwd_f32(const float *x, float *y, size_t rows, size_t cols, int log_mode,
                        cxm_stream_t s) {
    return softmax_fwd(x, y, rows, cols, log_mode, s);
}

int cxm_softmax_bwd_f32(const float *y, const float *dy, float *dx, size_t rows, size_t cols,
                        int log_mode, cxm_stream_t s) {
    return softmax_bwd(y, dy, dx, rows, cols, log_mode, s);
}

int cxm_softmax_xent_f32(const float *logits, const int32_t *labels, float *loss, float *dlogits,
                         size_t b, size_t c, cxm_stream_t st) {
    if (!logits || !labels || !loss || !dlogits || b == 0 || c == 0) return CXM_E_INVALID;
    if (c > 0x7fffffffu) return CXM_E_TOO_LARGE;
    const size_t blocks = (b + kBlock - 1) / kBlock;
    if (blocks > 0x7fffffffu) return CXM_E_TOO_LARGE;
    Workspace ws;
    int rc = get_workspace(st, 1, blocks * sizeof(float), &ws);
    if (rc) return rc;
    hipStream_t s = hs(st);
    const float inv_b = 1.0f / static_cast<float>(b);
    hipLaunchKernelGGL(k_xent, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, s, logits, labels, loss,
                       dlogits, b, c, inv_b, static_cast<float *>(ws.scratch), ws.counters);
    return launch_status();
}

}  // extern "C"
