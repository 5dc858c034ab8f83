// Shared device helpers and host plumbing of the gfx950 kernels.
//
// Wave64 throughout: a wavefront is 64 lanes, a workgroup of 256 threads is
// four waves.  Cross-lane reductions use DPP inside a row of 16 lanes
// (quad_perm, row_half_mirror, row_mirror) and readlane across the four rows.
// No float atomics anywhere: cross-workgroup combines are done in a fixed
// order by the last workgroup to finish (an integer ticket per output), so
// every result is deterministic run to run.
#pragma once

#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstddef>
#include <cstdint>

#include "../../include/cxm_hip.h"

namespace cxm {

constexpr int kWave = 64;
constexpr int kBlock = 256;  // threads per workgroup used by most kernels
constexpr int kWavesPerBlock = kBlock / kWave;

// ------------------------------------------------------------ host side

// Returns CXM_OK, or the HIP error of the last launch.
int launch_status();

// Ticket counters sit kCtr words (256 bytes) apart, one per cache line:
// atomics from many workgroups on counters that share a line serialise
// (16 counters in one line made a 4096-workgroup reduction 4x slower).
constexpr size_t kCtr = 64;

// Scratch memory of the multi-pass kernels, one region per (device, stream).
// It starts with `counters` ticket counters (kCtr words each), zero on
// entry to every kernel (each kernel's last workgroup puts its tickets back
// to zero); the rest is partial results.  Grows on demand (after a stream
// sync).  ctr(ws.counters, i) is counter i.
struct Workspace {
    unsigned *counters;
    size_t counters_n;
    void *scratch;
    size_t scratch_bytes;
};
int get_workspace(cxm_stream_t s, size_t counters, size_t scratch_bytes, Workspace *ws);

// Exchange region of the single-pass long-row softmax, one per (device,
// stream), kept apart from the workspace scratch (which other kernels
// overwrite).  Row r owns a header of kCtr words at hdr + r * kCtr (word 0:
// arrival ticket, word 1: epoch) and kXMaxSegs slot pairs at
// slots + r * kXMaxSegs * 2; each slot is a 64-bit (value, tag) word.
// Zero-filled when allocated; grows on demand (after a stream sync).
constexpr unsigned kXMaxSegs = 64;
struct Exchange {
    unsigned *hdr;
    unsigned long long *slots;
};
int get_exchange(cxm_stream_t s, size_t rows, Exchange *x);

// Tagged partial slots of the flat reductions, one region per (device,
// stream), kept apart from the workspace scratch.  Slot i is a 64-bit word
// (32-bit partial | tag << 32).  Each call takes a new tag (`epoch`, never
// 0, from next_tag()): its writers store their partials with it and its
// reader waits for it, so a slot an earlier call left, of any shape, on any
// stream, never carries the current tag; calls on one stream are ordered,
// so a write of an earlier call has landed before a later call starts.  A
// graph replays its launches with the tags they were captured with, so a
// call made under stream capture (`clear`) also has its reader put every
// slot it consumed back to tag 0.  Zero-filled when allocated; grows on
// demand (after a stream sync).  Under capture, a region that is missing or
// too small is CXM_E_CAPTURE (nothing is allocated, filled or waited for);
// one handed to a captured launch stays allocated until the stream is
// destroyed or cxm_release_workspaces runs.  get_workspace and
// get_exchange follow the same rules.
struct TaggedSlots {
    unsigned long long *slots;
    size_t n;
    unsigned epoch;
    int clear;
};
int get_tagged(cxm_stream_t s, size_t n, TaggedSlots *t);

// A new tag for the tagged slots, from one counter for the whole process
// (never 0, the empty slot's tag).
unsigned next_tag();

// Compute units and XCDs (each with its own L2) of the current device,
// read once per device.  Workgroups of a dispatch go to the XCDs round
// robin by linear workgroup id.
struct DevLayout {
    int cus;
    int xccs;
};
int device_layout(DevLayout *out);
// The current device's compute units (256 when the query fails).
inline size_t device_cus() {
    DevLayout l{0, 1};
    return device_layout(&l) == CXM_OK && l.cus > 0 ? static_cast<size_t>(l.cus) : 256;
}

// The current device's region `which` (0 workspace, 1 exchange, 2 tagged
// slots) of stream s: base, size and whether a captured launch holds it.
int workspace_query(cxm_stream_t s, int which, void **base, size_t *bytes, int *pinned);

// Polls a waiting workgroup makes for a peer's partial before it computes
// that partial itself (cxm_exchange_wait_limit).
unsigned exchange_wait_limit();

// Returns the caching pool's blocks of a stream to the device (pool.hip).
int pool_drop_stream(cxm_stream_t s);

__host__ __device__ inline unsigned *ctr(unsigned *base, size_t i) { return base + i * kCtr; }

// Epilogue of the GEMM (gemm.hip), applied to each finished sum
// v = (op(A) op(B))[row, col] before it is stored in C (row-major [M, N]).
struct Epilogue {
    const float *bias;  // [N] or null: v + bias[col]
    const float *gate;  // [M, N] or null: v * (gate > 0 ? 1 : 0) (ReLU backward)
    int act;            // CXM_ACT_NONE or CXM_ACT_RELU
    int sgd;            // 1: C is a weight and gets C - v*lr (SGD fused on the gradient)
    float lr;
};
// C[M, N] = op(A) op(B) with the epilogue; the engine of cxm_gemm_f32.
int gemm_ex(const float *A, const float *B, float *C, size_t M, size_t K, size_t N, int ta, int tb,
            const Epilogue &epi, cxm_stream_t s);
// Two independent products (no operand of one is written by the other) as
// one launch of the ring kernel when both take it at its whole-stage
// instance with the same operand layouts (gemm.hip: k_gemm_ring_pair);
// returns 1 when they do not, and the caller runs gemm_ex twice.
struct GemmSpec {
    const float *A, *B;
    float *C;
    size_t M, K, N;
    int ta, tb;
    Epilogue epi;
};
// With `side`, the launch also runs the MLP step's side work (mlp_side.hpp)
// on the CUs the products leave free when there are at least 8 of them;
// side->wgs says how many workgroups took it (0: none, the caller runs it).
struct StepSide;
int gemm_ex_pair(const GemmSpec &a, const GemmSpec &b, cxm_stream_t st, StepSide *side = nullptr);
// b[j] = b[j] - lr * sum_i x[i, j] over x [rows, cols]: a bias gradient
// (reduce::sum over axis 0) and its SGD step in one pass (reduce.hip).
int colsum_sgd(const float *x, float *b, size_t rows, size_t cols, float lr, cxm_stream_t s);

__host__ __device__ inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline unsigned ceil_div(size_t a, size_t b) { return static_cast<unsigned>((a + b - 1) / b); }

// ---------------------------------------------------------- device side

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL,
                                                               0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, false);
}

// DPP controls (all sources in range, so every lane is written).
constexpr int kQuadXor1 = 0xB1;      // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;      // quad_perm [2,3,0,1]
constexpr int kRowHalfMirror = 0x141;
constexpr int kRowMirror = 0x140;

__device__ __forceinline__ float readlane(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
__device__ __forceinline__ int readlane(int v, int lane) {
    return __builtin_amdgcn_readlane(v, lane);
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// 128-bit loads/stores.  The streaming forms set the non-temporal hint for
// data touched once (inputs of a reduction, outputs of an elementwise op).
__device__ __forceinline__ float4 ld4(const float *p) {
    const f32x4 v = *reinterpret_cast<const f32x4 *>(p);
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float4 ld4_stream(const float *p) {
    const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}
// A streaming 128-bit load at base + byte_off, with base uniform across the
// wave and byte_off a 32-bit value: the scalar-base + 32-bit vector-offset
// form of global_load, one address register per load where a 64-bit
// per-lane address takes two (and the register pressure can split a batch
// of loads).
__device__ __forceinline__ float4 ld4_stream_at(const float *base, unsigned byte_off) {
    return ld4_stream(reinterpret_cast<const float *>(reinterpret_cast<const char *>(base) + byte_off));
}
__device__ __forceinline__ void st4(float *p, float4 v) {
    *reinterpret_cast<f32x4 *>(p) = f32x4{v.x, v.y, v.z, v.w};
}
__device__ __forceinline__ void st4_stream(float *p, float4 v) {
    __builtin_nontemporal_store(f32x4{v.x, v.y, v.z, v.w}, reinterpret_cast<f32x4 *>(p));
}

// Direct global-to-LDS load of 16 bytes per lane (global_load_lds_dwordx4):
// lane L's 16 bytes at gsrc land at LDS byte lds + 16 L (lds wave-uniform,
// placed in M0).  Issued through inline asm so that the compiler's wait
// insertion does not see an LDS write in flight: it cannot always tell which
// LDS array such a load fills and then waits for every outstanding load
// (vmcnt(0)) before unrelated LDS reads.  The caller orders the load against
// LDS reads and writes itself (s_waitcnt vmcnt plus a barrier before the
// data is read; no read of the destination in flight when it is issued) and
// waits for it before the workgroup ends.
__device__ __forceinline__ void lds_load16(const void *gsrc, const void *lds) {
    const unsigned a = __builtin_amdgcn_readfirstlane(
        static_cast<unsigned>(reinterpret_cast<size_t>((const __attribute__((address_space(3))) void *)lds)));
    asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(gsrc), "{m0}"(a) : "memory");
}

// The same load from a wave-uniform base (an SGPR pair) plus a 32-bit
// per-lane byte offset (the saddr form): the lane's address costs no 64-bit
// vector arithmetic.
// `base` and `lds` (the LDS byte address, lds_addr) are the same in every
// lane; read from the first lane, they are scalar values for the
// instruction's SGPR operands whatever registers the compiler held them in.
__device__ __forceinline__ void lds_load16_at(const void *base, unsigned off, unsigned lds) {
    const size_t b = reinterpret_cast<size_t>(base);
    const unsigned lo = __builtin_amdgcn_readfirstlane(static_cast<unsigned>(b));
    const unsigned hi = __builtin_amdgcn_readfirstlane(static_cast<unsigned>(b >> 32));
    const void *sb = reinterpret_cast<const void *>((static_cast<size_t>(hi) << 32) | lo);
    asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(sb), "{m0}"(__builtin_amdgcn_readfirstlane(lds))
                 : "memory");
}
// LDS byte address of a __shared__ location, as a wave-uniform value.
__device__ __forceinline__ unsigned lds_addr(const void *p) {
    return __builtin_amdgcn_readfirstlane(
        static_cast<unsigned>(reinterpret_cast<size_t>((const __attribute__((address_space(3))) void *)p)));
}

// Barrier of an LDS ring filled by lds_load16: this wave waits until at
// most PENDING of its global loads are outstanding (loads retire in order,
// so every older fill has landed in LDS) and for its own LDS reads, then
// joins the workgroup barrier; after it, every wave's older fills are
// visible and every wave's reads of the stage about to be refilled are
// done.  Not __syncthreads(): its workgroup-scope fence makes the compiler
// wait for all outstanding global loads (vmcnt(0)), the fills the ring
// means to keep in flight included.  The memory clobber keeps the compiler
// from moving LDS accesses across it.
template <int PENDING>
__device__ __forceinline__ void ring_barrier() {
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(PENDING) : "memory");
}

// IEEE max as _mm256_max_ps(a, b): a when a > b, else b.
__device__ __forceinline__ float vmax(float a, float b) { return a > b ? a : b; }

// Reduction operators.  `combine` must be associative and commutative on the
// values the kernels feed it (sum: up to rounding; max/argmax: exactly, for
// non-NaN inputs).  `accum(a, v, i)` folds one input element v at index i
// into a running value; for kShift operators the kernel passes v - K, K the
// first element of the row or column (see Pow2Op).
struct SumOp {
    using T = float;
    static constexpr bool kShift = false;
    __device__ static T identity() { return 0.0f; }
    __device__ static T combine(T a, T b) { return a + b; }
    __device__ static T accum(T a, float v, int) { return a + v; }
};

// sum |x| (norm1)
struct AbsSumOp : SumOp {
    __device__ static T accum(T a, float v, int) { return a + fabsf(v); }
};

// sum x*x with the product unrounded, as fma::add(v, v, acc) (norm2)
struct SqSumOp : SumOp {
    __device__ static T accum(T a, float v, int) { return fmaf(v, v, a); }
};

// max / min of the reductions (and the softmax's row max): IEEE 754-2019
// maximum / minimum, one v_maximum3_f32 / v_minimum3_f32 on gfx950: NaN
// when either operand is NaN, and +0 above -0.  Both are associative and
// commutative on every input, NaN and signed zeros included, so any tree
// gives the same bits.  The reference folds _mm256_max_ps lane by lane
// (Engine/AVX2/functions.hpp:314-316: the second operand on NaN and on
// ties), whose result with a NaN or a +0/-0 tie depends on where they sit;
// without them the two agree bit for bit.  The flat and row forms start
// from -FLT_MAX (max) / FLT_MAX (min) as the reference does.
struct MaxOp {
    using T = float;
    static constexpr bool kShift = false;
    __device__ static T identity() { return -FLT_MAX; }
    __device__ static T combine(T a, T b) { return __builtin_elementwise_maximum(a, b); }
    __device__ static T accum(T a, float v, int) { return __builtin_elementwise_maximum(a, v); }
};

struct MinOp {
    using T = float;
    static constexpr bool kShift = false;
    __device__ static T identity() { return FLT_MAX; }
    __device__ static T combine(T a, T b) { return __builtin_elementwise_minimum(a, b); }
    __device__ static T accum(T a, float v, int) { return __builtin_elementwise_minimum(a, v); }
};

// Lexicographic (value, index): larger value wins; equal values (+0 and -0
// among them) keep the smaller index, i.e. the first maximum in storage
// order.  A NaN element never wins a comparison, so NaNs are skipped --
// except the first element of the row, column or flat array: the reference
// starts from it and takes only strictly greater values after it
// (reduce.cpp:442-455, 483-521), so a NaN there stays the answer.  The
// kernels fold that case in by replacing the first element's pair with
// first_nan(), which beats every pair, and write its index -1 as 0.
struct ArgPair {
    float v;
    int i;
};
struct ArgMaxOp {
    using T = ArgPair;
    static constexpr bool kShift = false;
    __device__ static T identity() { return {-INFINITY, 0x7fffffff}; }
    __device__ static T first_nan() { return {INFINITY, -1}; }
    __device__ static T combine(T a, T b) {
        const bool take_b = (b.v > a.v) || (b.v == a.v && b.i < a.i);
        return take_b ? b : a;
    }
    __device__ static T accum(T a, float v, int i) { return combine(a, T{v, i}); }
};
// Smaller value wins; equal values keep the smaller index (first minimum).
struct ArgMinOp {
    using T = ArgPair;
    static constexpr bool kShift = false;
    __device__ static T identity() { return {INFINITY, 0x7fffffff}; }
    __device__ static T first_nan() { return {-INFINITY, -1}; }
    __device__ static T combine(T a, T b) {
        const bool take_b = (b.v < a.v) || (b.v == a.v && b.i < a.i);
        return take_b ? b : a;
    }
    __device__ static T accum(T a, float v, int i) { return combine(a, T{v, i}); }
};
// argmax / argmin: the pair of a NaN first element (x0) wins outright.
template <class Op>
__device__ __forceinline__ void first_nan_fix(typename Op::T &a, float x0) {
    if constexpr (__is_same(typename Op::T, ArgPair)) {
        if (__builtin_isnan(x0)) a = Op::first_nan();
    }
}

template <int CTRL>
__device__ __forceinline__ ArgPair dpp(ArgPair p) {
    return {dpp<CTRL>(p.v), dpp<CTRL>(p.i)};
}
__device__ __forceinline__ ArgPair readlane(ArgPair p, int lane) {
    return {readlane(p.v, lane), readlane(p.i, lane)};
}

// Shifted power sums for the variance: s1 = sum(d), s2 = sum(d*d) with
// d = x - K, where the kernel subtracts K = the first element of the row
// or column being reduced.  Accumulated in fp64 (exact squares of fp32
// differences; fp64 throughput is far above what HBM feeds), the variance
// m2 = s2 - s1^2/n loses nothing to cancellation unless the data's mean is
// more than ~1e5 standard deviations from K.  Combining is plain addition,
// so any merge tree gives the same value up to fp64 rounding.
struct Pow2 {
    double s1, s2;
};
struct Pow2Op {
    using T = Pow2;
    static constexpr bool kShift = true;
    __device__ static T identity() { return {0.0, 0.0}; }
    __device__ static T combine(T a, T b) { return {a.s1 + b.s1, a.s2 + b.s2}; }
    __device__ static T accum(T a, float d, int) {
        const double e = d;
        return {a.s1 + e, fma(e, e, a.s2)};
    }
};

__device__ __forceinline__ double dbl_from(int lo, int hi) {
    return __builtin_bit_cast(double, (static_cast<unsigned long long>(static_cast<unsigned>(hi)) << 32) |
                                          static_cast<unsigned>(lo));
}
template <int CTRL>
__device__ __forceinline__ double dpp(double v) {
    const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
    return dbl_from(dpp<CTRL>(static_cast<int>(u)), dpp<CTRL>(static_cast<int>(u >> 32)));
}
__device__ __forceinline__ double readlane(double v, int lane) {
    const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
    return dbl_from(readlane(static_cast<int>(u), lane), readlane(static_cast<int>(u >> 32), lane));
}
template <int CTRL>
__device__ __forceinline__ Pow2 dpp(Pow2 p) {
    return {dpp<CTRL>(p.s1), dpp<CTRL>(p.s2)};
}
__device__ __forceinline__ Pow2 readlane(Pow2 p, int lane) {
    return {readlane(p.s1, lane), readlane(p.s2, lane)};
}

// Reduce across the 64 lanes of a wave; every lane gets the result.
// Must be called with all 64 lanes active.
template <class Op>
__device__ __forceinline__ typename Op::T wave_reduce(typename Op::T v) {
    v = Op::combine(v, dpp<kQuadXor1>(v));
    v = Op::combine(v, dpp<kQuadXor2>(v));
    v = Op::combine(v, dpp<kRowHalfMirror>(v));
    v = Op::combine(v, dpp<kRowMirror>(v));
    typename Op::T r = Op::combine(Op::combine(readlane(v, 0), readlane(v, 16)),
                                   Op::combine(readlane(v, 32), readlane(v, 48)));
    return r;
}

// Reduce across a workgroup of NT threads; the result is valid in every
// thread.  `lds` must hold NT/64 elements.  Contains barriers: call from
// uniform control flow.
template <class Op, int NT>
__device__ __forceinline__ typename Op::T block_reduce(typename Op::T v, typename Op::T *lds) {
    constexpr int NW = NT / kWave;
    v = wave_reduce<Op>(v);
    if constexpr (NW == 1) {
        return v;
    } else {
        const int w = threadIdx.x / kWave;
        if ((threadIdx.x & (kWave - 1)) == 0) lds[w] = v;
        __syncthreads();
        typename Op::T r = lds[0];
#pragma unroll
        for (int i = 1; i < NW; ++i) r = Op::combine(r, lds[i]);
        __syncthreads();  // lds may be reused by the caller
        return r;
    }
}

// Device-coherent stores and loads for data that one workgroup hands to
// another within a kernel (partial results).  They are agent-scope relaxed
// atomics: the store is written through past this XCD's L2 (sc1) and the
// load does not trust the reader's L2, so no L2 write-back or invalidate of
// the whole cache is needed (a __threadfence() per workgroup costs that on
// a multi-XCD part, and dominated the run time of a 2048-workgroup grid).
__device__ __forceinline__ void st_dev(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(ArgPair *p, ArgPair v) {
    const unsigned long long u = (static_cast<unsigned long long>(static_cast<unsigned>(v.i)) << 32) |
                                 __builtin_bit_cast(unsigned, v.v);
    __hip_atomic_store(reinterpret_cast<unsigned long long *>(p), u, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ ArgPair ld_dev(const ArgPair *p) {
    const unsigned long long u = __hip_atomic_load(reinterpret_cast<const unsigned long long *>(p),
                                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return {__builtin_bit_cast(float, static_cast<unsigned>(u)), static_cast<int>(u >> 32)};
}
// Power sums: two 64-bit words; the reader is ordered after both by the
// last-workgroup ticket.
__device__ __forceinline__ void st_dev(Pow2 *p, Pow2 v) {
    auto *u = reinterpret_cast<unsigned long long *>(p);
    __hip_atomic_store(u, __builtin_bit_cast(unsigned long long, v.s1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(u + 1, __builtin_bit_cast(unsigned long long, v.s2), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ Pow2 ld_dev(const Pow2 *p) {
    const auto *u = reinterpret_cast<const unsigned long long *>(p);
    return {__builtin_bit_cast(double, __hip_atomic_load(u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)),
            __builtin_bit_cast(double, __hip_atomic_load(u + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))};
}

// Combines n partials p[0], p[stride], ..., p[(n-1)*stride] into `a` in
// index order.  The device-coherent loads go out 16 at a time so their
// latencies overlap (one at a time, a 64-partial combine costs ~30 us).
template <class Op>
__device__ __forceinline__ typename Op::T combine_partials(const typename Op::T *p, unsigned n,
                                                           size_t stride, typename Op::T a) {
    constexpr unsigned G = 16;
    for (unsigned c0 = 0; c0 < n; c0 += G) {
        typename Op::T v[G];
#pragma unroll
        for (unsigned u = 0; u < G; ++u) v[u] = c0 + u < n ? ld_dev(p + (c0 + u) * stride) : Op::identity();
#pragma unroll
        for (unsigned u = 0; u < G; ++u) a = Op::combine(a, v[u]);
    }
    return a;
}

// Last-workgroup ticket.  Every thread of the workgroup calls it after
// storing its share of the workgroup's partials with st_dev; returns true in
// all threads of the one workgroup that arrives last among `expected`, which
// then reads every partial with ld_dev.  Ordering: each thread waits for its
// own stores to complete (vmcnt 0) before the barrier, and the ticket is an
// agent-scope atomic issued after the barrier, so every partial is at the
// coherent level before the count can reach `expected`.
__device__ __forceinline__ bool last_block_ticket(unsigned *counter, unsigned expected,
                                                  int *lds_flag) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned t =
            __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const bool last = (t == expected - 1);
        // ready for the next kernel that uses this workspace
        if (last) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *lds_flag = last ? 1 : 0;
    }
    __syncthreads();
    return *lds_flag != 0;
}

// Two-level form of the ticket for many arrivals on one output: arrival
// `idx` (0..expected-1) checks in on group counter idx % G; the last of each
// group checks in on the top counter counters[G]; the last there is last
// overall.  Spreads what would be `expected` atomics on one address over
// G + 1 counters.  `counters` is counter 0 of G + 1 consecutive ones.
template <unsigned G>
__device__ __forceinline__ bool last_block_ticket2(unsigned *counters, unsigned expected,
                                                   unsigned idx, int *lds_flag) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned ng = expected < G ? expected : G;
        const unsigned g = idx % ng;
        const unsigned gsize = (expected - g + ng - 1) / ng;
        bool last = false;
        const unsigned t =
            __hip_atomic_fetch_add(ctr(counters, g), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (t == gsize - 1) {
            __hip_atomic_store(ctr(counters, g), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const unsigned t2 =
                __hip_atomic_fetch_add(ctr(counters, G), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last = (t2 == ng - 1);
            if (last) __hip_atomic_store(ctr(counters, G), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        *lds_flag = last ? 1 : 0;
    }
    __syncthreads();
    return *lds_flag != 0;
}

// ------------------------------------------------------ streaming maps
//
// Elementwise kernels over n floats with 16-byte aligned pointers: one
// float4 per thread, 256-thread workgroups, non-temporal loads and stores,
// and the n % 4 tail done by the one thread whose vector index is n / 4.
// An output may alias an input: each element is read and written by the
// same thread.
//
// Layout: the array is cut into 1 KiB pieces (one wave's 64 float4), and
// the pieces into virtual rows of kPieceRow; workgroup b's four waves take
// piece b % kPieceRow of virtual rows 4 (b / kPieceRow) + 0..3, the layout
// of k_rowmap4 below.  Consecutive workgroups, which the dispatcher deals
// to the XCDs in turn, read consecutive 1 KiB pieces.  Measured on gfx950
// at 256 MiB in + 256 MiB out (events around back-to-back launches): a
// workgroup of four consecutive pieces (4 KiB) 80.2-80.8 us, this layout
// 78.2-78.5 us, one 64-thread workgroup per piece 78.7-79.2 us; two and four
// float4 per thread 87.4-87.7 us; blocks regrouped so each XCD reads one
// contiguous eighth 82.5 us; temporal loads and stores 87 us.  Two inputs
// and one output: 122.2-122.6 against 117.1 us.
constexpr size_t kPieceRow = 32;

// Vector (float4, or 8 x 16-bit) index of this thread.
__device__ __forceinline__ size_t stream_vec() {
    const unsigned b = blockIdx.x, w = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
    const size_t piece = (static_cast<size_t>(b / kPieceRow) * kWavesPerBlock + w) * kPieceRow + b % kPieceRow;
    return piece * kWave + lane;
}
// Workgroups that cover vector indices 0 .. nv (nv itself: the tail
// thread) in that layout; 0 when beyond the grid.  Also a grid of at least
// nv + 1 threads for kernels that index threads contiguously.
inline unsigned stream_grid_for(size_t nv) {
    const size_t pieces = nv / kWave + 1;
    const size_t rows = (pieces + kWavesPerBlock * kPieceRow - 1) / (kWavesPerBlock * kPieceRow);
    const size_t b = rows * kPieceRow;
    return b > 0xffffffffu ? 0u : static_cast<unsigned>(b);
}

template <class F>
__device__ __forceinline__ float4 map4(const F &f, float4 v) {
    return make_float4(f(v.x), f(v.y), f(v.z), f(v.w));
}

template <class F>
__global__ __launch_bounds__(kBlock) void k_map4(F f, const float *x, float *z, size_t n) {
    const size_t i = stream_vec();
    const size_t n4 = n / 4;
    if (i < n4) {
        st4_stream(z + 4 * i, map4(f, ld4_stream(x + 4 * i)));
    } else if (i == n4) {
        for (size_t j = 4 * n4; j < n; ++j) z[j] = f(x[j]);
    }
}

template <class F>
__global__ __launch_bounds__(kBlock) void k_zip4(F f, const float *x, const float *y, float *z, size_t n) {
    const size_t i = stream_vec();
    const size_t n4 = n / 4;
    if (i < n4) {
        const float4 a = ld4_stream(x + 4 * i), b = ld4_stream(y + 4 * i);
        st4_stream(z + 4 * i, make_float4(f(a.x, b.x), f(a.y, b.y), f(a.z, b.z), f(a.w, b.w)));
    } else if (i == n4) {
        for (size_t j = 4 * n4; j < n; ++j) z[j] = f(x[j], y[j]);
    }
}

// Workgroups for k_map4 / k_zip4 over n floats (0 when n is beyond the grid).
inline unsigned map4_grid(size_t n) { return stream_grid_for(n / 4); }

// Row-structured streaming map over a row-major [m, 4*n4] matrix: one
// float4 per thread.  The four waves of workgroup b take four consecutive
// rows (row quad b / tpr) of one 64-float4 column tile (b % tpr, tpr =
// tiles per row), so the per-column operands a functor loads (scale, bias,
// a broadcast row) are the same addresses for all four waves and cross
// from L2 once per workgroup.  On gfx950 at [8192, 8192] this layout moves
// 6.8 TB/s for y = relu(x*scale + bias); one row of 256 float4 per
// workgroup moved 6.3 TB/s, its column operands costing as many L2 bytes
// as x itself.  f(v, row, j4) returns the output float4 for input v at
// (row, columns 4*j4 .. 4*j4+3) and loads any per-row or per-column
// operands itself (they stay in cache).
constexpr int kRowMapRows = kBlock / kWave;

template <class F>
__global__ __launch_bounds__(kBlock) void k_rowmap4(F f, const float *x, float *z, size_t m, size_t n4,
                                                    unsigned tpr) {
    const unsigned quad = blockIdx.x / tpr;
    const unsigned tile = blockIdx.x - quad * tpr;
    const size_t row = static_cast<size_t>(quad) * kRowMapRows + threadIdx.x / kWave;
    const size_t j4 = static_cast<size_t>(tile) * kWave + (threadIdx.x & (kWave - 1));
    if (row >= m || j4 >= n4) return;
    const size_t o = row * n4 * 4 + 4 * j4;
    st4_stream(z + o, f(ld4_stream(x + o), static_cast<unsigned>(row), j4));
}

// Workgroups and tiles per row for k_rowmap4 (false when beyond the grid or
// when a row index does not fit 32 bits).
inline bool rowmap4_grid(size_t m, size_t n4, unsigned *grid, unsigned *tpr) {
    const size_t t = (n4 + kWave - 1) / kWave;
    const size_t q = (m + kRowMapRows - 1) / kRowMapRows;
    if (t == 0 || q == 0 || m > 0xffffffffu || q * t > 0xffffffffu) return false;
    *tpr = static_cast<unsigned>(t);
    *grid = static_cast<unsigned>(q * t);
    return true;
}

}  // namespace cxm
