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
// Kernel families by row length:
//  * wave per row, row in registers (cols <= 4096, cols % 4 == 0): one pass
//    over HBM, DPP wave reductions, no LDS;
//  * long rows (up to 64 segments of 8192, up to 8192 rows): one pass, each
//    workgroup holds a segment in registers and the workgroups of a row
//    exchange partials through device memory (see the single-pass section);
//  * longer rows or more rows: pass 1 reduces each 4096-element segment to
//    (max m_b, sum_b exp(x - m_b)) [forward] or to its partial dot product
//    [backward]; pass 2 combines the row's partials in segment order
//    (S = sum_b s_b * exp(m_b - M)), re-reads its segment and writes;
//  * any shape or alignment: wave per row, three sweeps over the row.
// The running max starts from -FLT_MAX, as reduce::max does, so an
// all -inf row (or segment) never forms (-inf) - (-inf).
#include <atomic>

#include "cxm_common.hpp"

// Per-workgroup timeline of the single-pass long-row kernels, for the
// diagnostics build only (this file compiled with -DCXM_TIMELINE into
// libcxm_hip_timeline.so, read by `bench.py --timeline c4`).  Thread 0 of a
// workgroup writes the 100 MHz s_memrealtime clock to mark i of its
// record: 0 entry, 1 (forward only) its staggered start over, 2 its
// partial reduced and published, 3 the row's partials in
// (past the barrier after the exchange), 4 its stores issued (past a final
// barrier).  Tables: 0 softmax forward, 1 log-softmax forward, 2 softmax
// backward, 3 log-softmax backward; records indexed by the linear
// workgroup id modulo kSmTlWgs, overwritten by the next launch of the same
// table.  Without CXM_TIMELINE the marks compile to nothing.
#ifdef CXM_TIMELINE
constexpr unsigned kSmTlKinds = 4, kSmTlWgs = 1024, kSmTlMarks = 5;
static __device__ unsigned long long sm_timeline[kSmTlKinds][kSmTlWgs][kSmTlMarks];
__device__ __forceinline__ void sm_tl_mark(unsigned kind, unsigned i) {
    if (threadIdx.x == 0)
        __builtin_nontemporal_store(__builtin_amdgcn_s_memrealtime(),
                                    &sm_timeline[kind][(blockIdx.x + gridDim.x * blockIdx.y) % kSmTlWgs][i]);
}
#else
__device__ __forceinline__ void sm_tl_mark(unsigned, unsigned) {}
#endif

namespace cxm {
namespace {

constexpr float kLowest = -FLT_MAX;

// exp(y) of a log-softmax output in the backward (dx = dy - exp(y) * sum dy),
// as exp2(y * log2 e): v_exp_f32 with the compiler's scaling for results
// below the normal range, seven instructions where expf's extended-precision
// range reduction takes about thirteen.  The rounded product costs a relative
// error of at most |y| * 2^-24 (5.2e-6 while exp(y) is normal, |y| < 87.4),
// plus about 1 ulp from v_exp_f32, inside the backward's 1e-5 bar on that term.
// Measured on the [64, 131072] backward: 18.0 -> 17.4 us.
__device__ __forceinline__ float exp_lsm(float y) { return exp2f(y * 1.44269504088896341f); }

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
            o.x = gv[k].x - exp_lsm(yv[k].x) * r; o.y = gv[k].y - exp_lsm(yv[k].y) * r;
            o.z = gv[k].z - exp_lsm(yv[k].z) * r; o.w = gv[k].w - exp_lsm(yv[k].w) * r;
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
            o.x = g[k].x - exp_lsm(yy[k].x) * r; o.y = g[k].y - exp_lsm(yy[k].y) * r;
            o.z = g[k].z - exp_lsm(yy[k].z) * r; o.w = g[k].w - exp_lsm(yy[k].w) * r;
        } else {
            o.x = yy[k].x * (g[k].x - r); o.y = yy[k].y * (g[k].y - r);
            o.z = yy[k].z * (g[k].z - r); o.w = yy[k].w * (g[k].w - r);
        }
        st4_stream(dx + base + 4 * i, o);
    }
}

// ------------------------------------------- single pass, long rows
//
// A row of up to kXMaxSegs segments of kXNV float4 per thread (8192 floats)
// is read once: workgroup (row, b) keeps its segment in registers, reduces
// it to a partial, publishes the partial in its slot of the row's exchange
// record, reads the partials of the other segments of its row, combines all
// of them in segment order (so every workgroup of the row gets the same
// row statistic, bit for bit), and writes its segment.  HBM traffic is one
// read and one write, where the two-pass form reads the input twice.
//
// No cooperative launch and no grid-wide barrier: a slot is valid when its
// tag equals the row's epoch + 1.  Every workgroup reads the epoch first
// (before its data loads, so the read is off the critical path) and takes
// an arrival ticket right after it publishes its partial; the workgroup
// that took the row's last ticket advances the epoch (and resets the
// ticket) after its stores, which is after every workgroup of the row has
// read the epoch, so a slot written by any earlier call never carries the
// current tag.  Measured at [64, 131072] on gfx950 (forward / backward):
// ticket at the start, before the partial, 13.4 / 18.0 us; after the
// stores 13.0 / 18.1; after the publish 11.5 / 16.8.  The
// wait for a peer's slot is bounded (exchange_wait_limit() polls, each a
// device round trip plus a short sleep); a peer not seen by then is not
// waited for: its partial is recomputed from the input with the same
// arithmetic as the owner's, so the result is the same bit for bit, only
// slower.  Every workgroup therefore finishes whatever the dispatch order
// or residency of its peers.

constexpr int kXNV = 8;
constexpr size_t kXSeg = static_cast<size_t>(kBlock) * 4 * kXNV;  // floats per segment
constexpr size_t kXRowsMax = 8192;

// Staggered start of row groups.  Left alone, every workgroup loads at
// once, every row then waits for its exchange with HBM idle, and every
// workgroup stores at once.  Workgroups of row group g (of `groups`) sleep
// g * quanta times 128 cycles before their first load, so the later groups'
// loads fill the earlier groups' exchange gap.  Results do not depend on it.
// The group of a row is (row * gmul) >> 16 with gmul = groups * 2^16 / rows
// from the host (a multiply, not a division, ahead of the loads; any split
// of the rows into groups gives the same results).
__device__ __forceinline__ void x_stagger(unsigned row, unsigned gmul, unsigned quanta) {
    const unsigned n = ((row * gmul) >> 16) * quanta;  // row < 8192, gmul <= 2^20
    for (unsigned i = 0; i < n; ++i) __builtin_amdgcn_s_sleep(2);
}

__device__ __forceinline__ unsigned long long xld(const unsigned long long *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void xst(unsigned long long *p, float v, unsigned tag) {
    __hip_atomic_store(p, (static_cast<unsigned long long>(tag) << 32) | __builtin_bit_cast(unsigned, v),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float xval(unsigned long long u) {
    return __builtin_bit_cast(float, static_cast<unsigned>(u));
}
__device__ __forceinline__ unsigned xtag(unsigned long long u) { return static_cast<unsigned>(u >> 32); }

// The row's epoch (one request per wave: the address is uniform).  The tag
// of this call's slots is epoch + 1.
__device__ __forceinline__ unsigned x_epoch(const unsigned *h) {
    return __hip_atomic_load(h + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Thread 0, after publishing: take the arrival ticket.  The epoch read
// returned before (its value went into the published tag), so every
// workgroup has read the epoch when the last ticket is taken.
__device__ __forceinline__ unsigned x_ticket(unsigned *h) {
    return __hip_atomic_fetch_add(h, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Thread 0, after the workgroup's stores.
__device__ __forceinline__ void x_leave(unsigned *h, unsigned ticket, unsigned segs, unsigned tag) {
    if (ticket == segs - 1) {
        __hip_atomic_store(h, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(h + 1, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Lanes b < segs of wave 0 wait (bounded) for slot word `w` of segment b;
// returns the mask of segments not seen.  The own segment is not read.
template <int W>
__device__ __forceinline__ unsigned long long x_gather(const unsigned long long *sl, unsigned segs,
                                                       unsigned own, unsigned tag, unsigned limit,
                                                       float (*out)[kXMaxSegs]) {
    const unsigned b = threadIdx.x;
    bool miss = false;
    if (b < segs && b != own) {
        unsigned long long u[W];
        for (unsigned tries = 0;; ++tries) {
            bool ok = true;
#pragma unroll
            for (int w = 0; w < W; ++w) {
                u[w] = xld(sl + 2 * b + w);
                ok = ok && xtag(u[w]) == tag;
            }
            if (ok) break;
            if (tries >= limit) {
                miss = true;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
#pragma unroll
        for (int w = 0; w < W; ++w) out[w][b] = xval(u[w]);
    }
    return __ballot(miss);
}

// Loading the thread's NV float4 of a segment of n4 >= 1 float4: x_issue
// issues every load as straight-line code (an index past the end re-reads
// the segment's last float4), x_pad then overwrites those with `pad`.
// Loads under a per-load branch were compiled with a wait for each pair of
// loads at the branch's end, which halved the bytes in flight; all of a
// kernel's x_issue calls come before its first x_pad.
template <int NV>
__device__ __forceinline__ unsigned x_last(size_t n4) {
    return static_cast<unsigned>(n4 < kBlock * NV ? n4 : kBlock * NV) - 1u;
}
template <int NV>
__device__ __forceinline__ void x_issue(float4 (&v)[NV], const float *p, unsigned last) {
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const unsigned i = k * kBlock + threadIdx.x;
        v[k] = ld4_stream_at(p, 16u * (i < last ? i : last));
    }
}
template <int NV>
__device__ __forceinline__ void x_pad(float4 (&v)[NV], unsigned last, float4 pad) {
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        if (k * kBlock + threadIdx.x > last) v[k] = pad;
    }
}

__device__ __forceinline__ float max4(float m, float4 v) { return vmax(vmax(vmax(vmax(m, v.x), v.y), v.z), v.w); }
__device__ __forceinline__ float4 exp4(float4 v, float m) {
    return make_float4(expf(v.x - m), expf(v.y - m), expf(v.z - m), expf(v.w - m));
}
__device__ __forceinline__ float sum4(float4 e) { return (e.x + e.y) + (e.z + e.w); }
// sum(dy*y) partial, one rounding order pinned by explicit fmas
__device__ __forceinline__ float dot4(float r, float4 g, float4 y) {
    return fmaf(g.w, y.w, fmaf(g.z, y.z, fmaf(g.y, y.y, fmaf(g.x, y.x, r))));
}

// Forward.  Softmax keeps e = exp(x - m_t) (m_t the thread's max) and writes
// e * (exp(m_t - M) * (1/S)); log-softmax keeps x and writes (x - M) - log S.
template <bool LOG>
__global__ __launch_bounds__(kBlock) void k_sm_fwd_x(const float *__restrict__ x, float *__restrict__ y,
                                                     size_t cols, unsigned segs, unsigned *hdr,
                                                     unsigned long long *slots, unsigned limit,
                                                     unsigned gmul, unsigned quanta) {
    constexpr int NV = kXNV;
    __shared__ float lds[kWavesPerBlock];
    __shared__ float part[2][kXMaxSegs];
    __shared__ unsigned long long s_miss;
    // grid (segs, rows): no division ahead of the loads
    const unsigned seg = blockIdx.x, row = blockIdx.y;
    constexpr unsigned tl = LOG ? 1u : 0u;
    sm_tl_mark(tl, 0);
    x_stagger(row, gmul, quanta);
    sm_tl_mark(tl, 1);
    unsigned *h = hdr + row * kCtr;
    const unsigned tag = x_epoch(h) + 1;  // every wave: a load behind a branch would be waited for at its end
    const float *__restrict__ xr = x + static_cast<size_t>(row) * cols;
    const size_t n4 = (cols - static_cast<size_t>(seg) * kXSeg) / 4;
    const float4 ninf = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
    float4 v[NV];
    const unsigned last = x_last<NV>(n4);
    x_issue(v, xr + seg * kXSeg, last);
    __builtin_amdgcn_sched_barrier(0);
    x_pad(v, last, ninf);
    float mt = kLowest;
#pragma unroll
    for (int k = 0; k < NV; ++k) mt = max4(mt, v[k]);
    float st = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const float4 e = exp4(v[k], mt);
        st += sum4(e);
        if constexpr (!LOG) v[k] = e;
    }
    const float Mb = block_reduce<MaxOp, kBlock>(mt, lds);
    const float Sb = block_reduce<SumOp, kBlock>(st * expf(mt - Mb), lds);
    unsigned long long *sl = slots + static_cast<size_t>(row) * kXMaxSegs * 2;
    unsigned ticket = 0;
    if (threadIdx.x == 0) {
        xst(sl + 2 * seg, Mb, tag);
        xst(sl + 2 * seg + 1, Sb, tag);
        ticket = x_ticket(h);
        part[0][seg] = Mb;
        part[1][seg] = Sb;
    }
    sm_tl_mark(tl, 2);
    if (threadIdx.x < kWave) {
        const unsigned long long miss = x_gather<2>(sl, segs, seg, tag, limit, part);
        if (threadIdx.x == 0) s_miss = miss;
    }
    __syncthreads();
    sm_tl_mark(tl, 3);
    // peers not seen: recompute their partials from the input, same arithmetic
    for (unsigned long long miss = s_miss; miss; miss &= miss - 1) {
        const unsigned b = static_cast<unsigned>(__builtin_ctzll(miss));
        const float *xb = xr + b * kXSeg;
        const size_t nb = (cols - static_cast<size_t>(b) * kXSeg) / 4;
        float m = kLowest;
#pragma unroll 1
        for (int k = 0; k < NV; ++k) {
            const size_t i = static_cast<size_t>(k) * kBlock + threadIdx.x;
            m = max4(m, i < nb ? ld4(xb + 4 * i) : ninf);
        }
        float s = 0.0f;
#pragma unroll 1
        for (int k = 0; k < NV; ++k) {
            const size_t i = static_cast<size_t>(k) * kBlock + threadIdx.x;
            s += sum4(exp4(i < nb ? ld4(xb + 4 * i) : ninf, m));
        }
        const float M1 = block_reduce<MaxOp, kBlock>(m, lds);
        const float S1 = block_reduce<SumOp, kBlock>(s * expf(m - M1), lds);
        if (threadIdx.x == 0) {
            part[0][b] = M1;
            part[1][b] = S1;
        }
    }
    __syncthreads();
    const bool has = threadIdx.x < segs;
    const float M = block_reduce<MaxOp, kBlock>(has ? part[0][threadIdx.x] : kLowest, lds);
    const float S =
        block_reduce<SumOp, kBlock>(has ? part[1][threadIdx.x] * expf(part[0][threadIdx.x] - M) : 0.0f, lds);
    float *__restrict__ ys = y + static_cast<size_t>(row) * cols + seg * kXSeg;
    if constexpr (LOG) {
        const float ls = logf(S);
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const size_t i = static_cast<size_t>(k) * kBlock + threadIdx.x;
            if (i < n4)
                st4_stream(ys + 4 * i, make_float4((v[k].x - M) - ls, (v[k].y - M) - ls, (v[k].z - M) - ls,
                                                   (v[k].w - M) - ls));
        }
    } else {
        const float f = expf(mt - M) * (1.0f / S);
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const size_t i = static_cast<size_t>(k) * kBlock + threadIdx.x;
            if (i < n4) st4_stream(ys + 4 * i, make_float4(v[k].x * f, v[k].y * f, v[k].z * f, v[k].w * f));
        }
    }
    if (threadIdx.x == 0) x_leave(h, ticket, segs, tag);
#ifdef CXM_TIMELINE
    __syncthreads();
    sm_tl_mark(tl, 4);
#endif
}

// Backward: partial r_b = sum(dy*y) or sum(dy) per segment, r = sum_b r_b
// in segment order, then dx as the wave kernel writes it.
template <bool LOG>
__global__ __launch_bounds__(kBlock) void k_sm_bwd_x(const float *__restrict__ y, const float *__restrict__ dy,
                                                     float *__restrict__ dx, size_t cols, unsigned segs,
                                                     unsigned *hdr, unsigned long long *slots,
                                                     unsigned limit) {
    constexpr int NV = kXNV;
    __shared__ float lds[kWavesPerBlock];
    __shared__ float part[1][kXMaxSegs];
    __shared__ unsigned long long s_miss;
    const unsigned seg = blockIdx.x, row = blockIdx.y;  // grid (segs, rows)
    constexpr unsigned tl = LOG ? 3u : 2u;
    sm_tl_mark(tl, 0);
    unsigned *h = hdr + row * kCtr;
    const unsigned tag = x_epoch(h) + 1;  // every wave: a load behind a branch would be waited for at its end
    const size_t rbase = static_cast<size_t>(row) * cols;
    const size_t base = rbase + seg * kXSeg;
    const size_t n4 = (cols - static_cast<size_t>(seg) * kXSeg) / 4;
    const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
    float4 yv[NV], gv[NV];
    const unsigned last = x_last<NV>(n4);
    x_issue(yv, y + base, last);
    x_issue(gv, dy + base, last);
    __builtin_amdgcn_sched_barrier(0);
    x_pad(yv, last, zero);
    x_pad(gv, last, zero);
    float r = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) r = LOG ? r + sum4(gv[k]) : dot4(r, gv[k], yv[k]);
    const float rb = block_reduce<SumOp, kBlock>(r, lds);
    unsigned long long *sl = slots + static_cast<size_t>(row) * kXMaxSegs * 2;
    unsigned ticket = 0;
    if (threadIdx.x == 0) {
        xst(sl + 2 * seg, rb, tag);
        ticket = x_ticket(h);
        part[0][seg] = rb;
    }
    sm_tl_mark(tl, 2);
    if (threadIdx.x < kWave) {
        const unsigned long long miss = x_gather<1>(sl, segs, seg, tag, limit, part);
        if (threadIdx.x == 0) s_miss = miss;
    }
    __syncthreads();
    sm_tl_mark(tl, 3);
    for (unsigned long long miss = s_miss; miss; miss &= miss - 1) {
        const unsigned b = static_cast<unsigned>(__builtin_ctzll(miss));
        const size_t bb = rbase + b * kXSeg;
        const size_t nb = (cols - static_cast<size_t>(b) * kXSeg) / 4;
        float q = 0.0f;
#pragma unroll 1
        for (int k = 0; k < NV; ++k) {
            const size_t i = static_cast<size_t>(k) * kBlock + threadIdx.x;
            const bool in = i < nb;
            const float4 g = in ? ld4(dy + bb + 4 * i) : zero;
            if constexpr (LOG) q = q + sum4(g);
            else q = dot4(q, g, in ? ld4(y + bb + 4 * i) : zero);
        }
        const float q1 = block_reduce<SumOp, kBlock>(q, lds);
        if (threadIdx.x == 0) part[0][b] = q1;
    }
    __syncthreads();
    const float R = block_reduce<SumOp, kBlock>(threadIdx.x < segs ? part[0][threadIdx.x] : 0.0f, lds);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const size_t i = static_cast<size_t>(k) * kBlock + threadIdx.x;
        if (i >= n4) continue;
        float4 o;
        if constexpr (LOG) {
            o.x = gv[k].x - exp_lsm(yv[k].x) * R; o.y = gv[k].y - exp_lsm(yv[k].y) * R;
            o.z = gv[k].z - exp_lsm(yv[k].z) * R; o.w = gv[k].w - exp_lsm(yv[k].w) * R;
        } else {
            o.x = yv[k].x * (gv[k].x - R); o.y = yv[k].y * (gv[k].y - R);
            o.z = yv[k].z * (gv[k].z - R); o.w = yv[k].w * (gv[k].w - R);
        }
        st4_stream(dx + base + 4 * i, o);
    }
    if (threadIdx.x == 0) x_leave(h, ticket, segs, tag);
#ifdef CXM_TIMELINE
    __syncthreads();
    sm_tl_mark(tl, 4);
#endif
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
        dx[off + j] = LOG ? g - exp_lsm(yy) * r : yy * (g - r);
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

// Single pass when the row has at most kXMaxSegs segments and the exchange
// region stays small (rows * 1.25 KiB).
bool use_x(size_t rows, size_t cols) { return rows <= kXRowsMax && (cols + kXSeg - 1) / kXSeg <= kXMaxSegs; }

// Stagger of the single-pass forward: up to 16 row groups, the last one
// starting about pct% of the time the input takes to stream in (at 6 TB/s,
// 2.4 GHz) after the first.  Only when the whole grid is resident at once
// (at most 1024 workgroups, four per CU); beyond that the dispatch order
// staggers the rows already.  Measured on gfx950 with 32 MiB inputs
// (pct 0 -> 60 -> 70): [64, 131072] 14.6 -> 13.9 -> 13.6 us, [128, 65536]
// 13.3 -> 12.4 -> 12.4, [256, 32768] 13.1 -> 12.1 -> 12.1; at 80 the
// forward slows again, and an 8 MiB input gains nothing.  The backward
// (two inputs, one output) was slower at every setting (with the arrival
// ticket after the publish, [64, 131072]: 16.9 us at once, 17.5 / 18.2 /
// 20.0 us at pct 30 / 65 / 100) and starts at once.
std::atomic<int> g_x_stagger_pct{65};

// groups as the multiplier gmul = groups * 2^16 / rows (see x_stagger)
void x_stagger_for(int pct, size_t rows, unsigned segs, size_t bytes_in, unsigned *gmul, unsigned *quanta) {
    *gmul = 0;
    *quanta = 0;
    if (pct <= 0 || rows < 2 || rows * segs > 1024) return;
    const unsigned groups = rows < 16 ? static_cast<unsigned>(rows) : 16u;
    *gmul = static_cast<unsigned>((static_cast<size_t>(groups) << 16) / rows);
    const double total = static_cast<double>(bytes_in) / 6.0e12 * (pct / 100.0) * 2.4e9 / 128.0;
    *quanta = static_cast<unsigned>(total / (groups - 1));
}

int sm_fwd_x(const float *x, float *y, size_t rows, size_t cols, int log_mode, cxm_stream_t st) {
    const unsigned segs = static_cast<unsigned>((cols + kXSeg - 1) / kXSeg);
    Exchange xc;
    const int rc = get_exchange(st, rows, &xc);
    if (rc) return rc;
    const dim3 grid(segs, static_cast<unsigned>(rows));  // rows <= kXRowsMax
    const unsigned lim = exchange_wait_limit();
    unsigned g, q;
    x_stagger_for(g_x_stagger_pct.load(std::memory_order_relaxed), rows, segs, rows * cols * sizeof(float), &g, &q);
    if (log_mode)
        hipLaunchKernelGGL(k_sm_fwd_x<true>, grid, dim3(kBlock), 0, hs(st), x, y, cols, segs, xc.hdr, xc.slots, lim,
                           g, q);
    else
        hipLaunchKernelGGL(k_sm_fwd_x<false>, grid, dim3(kBlock), 0, hs(st), x, y, cols, segs, xc.hdr, xc.slots,
                           lim, g, q);
    return launch_status();
}

int sm_bwd_x(const float *y, const float *dy, float *dx, size_t rows, size_t cols, int log_mode,
             cxm_stream_t st) {
    const unsigned segs = static_cast<unsigned>((cols + kXSeg - 1) / kXSeg);
    Exchange xc;
    const int rc = get_exchange(st, rows, &xc);
    if (rc) return rc;
    const dim3 grid(segs, static_cast<unsigned>(rows));  // rows <= kXRowsMax
    const unsigned lim = exchange_wait_limit();
    if (log_mode)
        hipLaunchKernelGGL(k_sm_bwd_x<true>, grid, dim3(kBlock), 0, hs(st), y, dy, dx, cols, segs, xc.hdr, xc.slots,
                           lim);
    else
        hipLaunchKernelGGL(k_sm_bwd_x<false>, grid, dim3(kBlock), 0, hs(st), y, dy, dx, cols, segs, xc.hdr,
                           xc.slots, lim);
    return launch_status();
}

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

// [a, a + bytes) and [b, b + bytes) share at least one byte.
bool overlaps(const void *a, const void *b, size_t bytes) {
    const uintptr_t pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
    return pa < pb + bytes && pb < pa + bytes;
}

// Aliasing rules of the softmax entry points.  An output may be one of the
// inputs exactly (in place): every kernel but the single-pass long-row one
// reads an element in the thread that later writes it, and the single-pass
// kernel, whose waiting workgroups may re-read a peer's input segment, is
// not used in place (the two-pass kernels run instead).  Any other overlap
// is rejected.
bool bad_alias(const void *out, const void *in, size_t bytes) { return out != in && overlaps(out, in, bytes); }

int softmax_fwd(const float *x, float *y, size_t rows, size_t cols, int log_mode, cxm_stream_t st) {
    if (!x || !y || (log_mode != 0 && log_mode != 1)) return CXM_E_INVALID;
    if (rows == 0 || cols == 0) return CXM_OK;
    if (rows > SIZE_MAX / sizeof(float) / cols) return CXM_E_TOO_LARGE;
    const size_t bytes = rows * cols * sizeof(float);
    if (bad_alias(y, x, bytes)) return CXM_E_INVALID;
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
    if (use_x(rows, cols) && x != y) return sm_fwd_x(x, y, rows, cols, log_mode, st);
    return sm_fwd_split<kSegNV>(x, y, rows, cols, log_mode, st);
}

int softmax_bwd(const float *y, const float *dy, float *dx, size_t rows, size_t cols, int log_mode,
                cxm_stream_t st) {
    if (!y || !dy || !dx || (log_mode != 0 && log_mode != 1)) return CXM_E_INVALID;
    if (rows == 0 || cols == 0) return CXM_OK;
    if (rows > SIZE_MAX / sizeof(float) / cols) return CXM_E_TOO_LARGE;
    const size_t bytes = rows * cols * sizeof(float);
    if (bad_alias(dx, y, bytes) || bad_alias(dx, dy, bytes)) return CXM_E_INVALID;
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
    if (use_x(rows, cols) && dx != y && dx != dy) return sm_bwd_x(y, dy, dx, rows, cols, log_mode, st);
    return sm_bwd_split<kSegNV>(y, dy, dx, rows, cols, log_mode, st);
}

}  // namespace
}  // namespace cxm

#ifdef CXM_TIMELINE
// Diagnostics build only (not declared in include/cxm_hip.h): copies the
// long-row softmax timeline tables (kSmTlKinds x kSmTlWgs x kSmTlMarks 64-bit
// words) to host memory, after the caller's synchronisation.
extern "C" int cxm_timeline_softmax_read(unsigned long long *host, size_t words) {
    if (!host || words != static_cast<size_t>(kSmTlKinds) * kSmTlWgs * kSmTlMarks) return CXM_E_INVALID;
    const hipError_t e = hipMemcpyFromSymbol(host, HIP_SYMBOL(sm_timeline), words * sizeof(unsigned long long));
    return e == hipSuccess ? CXM_OK : static_cast<int>(e);
}
#endif

using namespace cxm;

extern "C" {

int cxm_softmax_stagger(int pct, int *previous) {
    if (pct < 0 || pct > 100) return CXM_E_INVALID;
    const int old = cxm::g_x_stagger_pct.exchange(pct);
    if (previous) *previous = old;
    return CXM_OK;
}

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
