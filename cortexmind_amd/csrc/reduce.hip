// fp32 reductions sum / mean / max / argmax / min / argmin / norm1 / norm2 /
// var / stdv, flat and over the middle axis
// of [outer, dim, inner].
//
// Replaces avx2::reduce (source/CortexMind/framework/Engine/AVX2/
// reduce.hpp:49-329, reduce.cpp:17-621).  Semantics the
// kernels keep from it are listed in include/cxm_hip.h.
//
// Two kernels cover every shape:
//  * k_rows: inner == 1 (row reductions, and the flat form as one row).
//    Each row is cut into `segs` segments; one 256-thread workgroup reduces
//    a segment with 128-bit loads (an unaligned head and a ragged tail of
//    fewer than 4 elements each are folded in by segment 0), several in
//    flight per thread, then a DPP wave reduce and a 4-entry LDS combine.
//    With segs > 1 the segment results are combined in segment order: by
//    the row's last workgroup (ticket) or, for a flat reduction, by one
//    reader workgroup that polls tagged slots.
//  * k_cols: inner > 1.  A workgroup owns 256 adjacent columns of one outer
//    slice and a chunk of the reduced rows; each thread keeps one float4 of
//    columns, the four waves take interleaved rows and meet in LDS.  Chunks
//    are combined in chunk order by the last workgroup of the column tile.
#include <atomic>
#include <mutex>
#include <type_traits>

#include "cxm_common.hpp"

// Scratch of cxm_reduce_sum_noalloc_f32: ticket counters first (kCtr words
// each), then the tagged slots of flat reductions (64-bit words), then
// partial results.  One copy per device, held
// until the process ends.  Host code never passes this name to a kernel:
// the address of each device's copy comes from hipGetSymbolAddress
// (fixed_scratch below).
constexpr size_t kFixedCounterBytes = size_t(1) << 20;  // 4096 counters
constexpr size_t kFixedTagged = 2048;                    // tagged slots (the flat plan's largest split)
constexpr size_t kFixedTaggedBytes = kFixedTagged * sizeof(unsigned long long);
constexpr size_t kFixedPartBytes = size_t(1) << 20;
constexpr size_t kFixedZeroBytes = kFixedCounterBytes + kFixedTaggedBytes;  // cleared at set-up
static __device__ __align__(256) unsigned char scratch[kFixedZeroBytes + kFixedPartBytes];
static_assert(kFixedZeroBytes % 256 == 0, "partials stay 256-byte aligned");

// Per-workgroup timeline of the C2 kernels, for the diagnostics build only
// (`make -C cortexmind_amd/csrc timeline`: this file compiled with
// -DCXM_TIMELINE into libcxm_hip_timeline.so; `bench.py --timeline` reads
// it).  Thread 0 of a workgroup writes the 100 MHz s_memrealtime clock to
// mark i of its record in table `kind`: 0 entry, 1 all its waves' loads
// folded (past the workgroup's first barrier after them), 2 its partial
// published (ticket taken, or tagged slot stored), 3 the last workgroup's
// (or the reader's) final store issued.  Records are indexed by
// the linear workgroup id modulo kTimelineWgs; a launch overwrites the
// previous launch's records of its kind.  Without CXM_TIMELINE the marks
// compile to nothing.
enum TimelineKind : unsigned { kTlRows = 0, kTlCols = 1, kTlFlat = 2, kTlColsArg = 3 };
#ifdef CXM_TIMELINE
constexpr unsigned kTimelineKinds = 4, kTimelineWgs = 4096, kTimelineMarks = 4;
static __device__ unsigned long long timeline[kTimelineKinds][kTimelineWgs][kTimelineMarks];
__device__ __forceinline__ void tl_mark(unsigned kind, unsigned i) {
    if (threadIdx.x == 0) {
        const unsigned wg = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
        __builtin_nontemporal_store(__builtin_amdgcn_s_memrealtime(), &timeline[kind][wg % kTimelineWgs][i]);
    }
}
#else
__device__ __forceinline__ void tl_mark(unsigned, unsigned) {}
#endif

namespace cxm {
namespace {

__global__ void k_zero_words(unsigned *p, size_t n) {
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<size_t>(gridDim.x) * blockDim.x)
        p[i] = 0u;
}

constexpr int kMaxDevices = 64;
std::atomic<unsigned char *> g_fixed[kMaxDevices];
std::mutex g_fixed_mu;

// Device address of the current device's `scratch`, looked up once per
// device (with that device current) on its first use; the counters and the
// tagged slots are then cleared by a fill kernel on stream s.  Every kernel
// that takes a ticket puts its counter back to zero and every tagged slot
// written is consumed in the same kernel, so they stay in that state
// between calls.
int fixed_scratch(cxm_stream_t s, unsigned char **out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return static_cast<int>(e);
    if (dev < 0 || dev >= kMaxDevices) return CXM_E_TOO_LARGE;
    unsigned char *p = g_fixed[dev].load(std::memory_order_acquire);
    if (p == nullptr) {
        std::lock_guard<std::mutex> lk(g_fixed_mu);
        p = g_fixed[dev].load(std::memory_order_relaxed);
        if (p == nullptr) {
            void *a = nullptr;
            e = hipGetSymbolAddress(&a, HIP_SYMBOL(scratch));
            if (e != hipSuccess) return static_cast<int>(e);
            if (a == nullptr) return CXM_E_INVALID;
            hipLaunchKernelGGL(k_zero_words, dim3(256), dim3(256), 0, reinterpret_cast<hipStream_t>(s),
                               static_cast<unsigned *>(a), kFixedZeroBytes / sizeof(unsigned));
            e = hipGetLastError();
            if (e != hipSuccess) return static_cast<int>(e);
            p = static_cast<unsigned char *>(a);
            g_fixed[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return CXM_OK;
}

// Scratch of one launch: `counters` ticket counters and `bytes` of partials
// (the per-stream workspace), or `tagged` tagged slots (their own region);
// with `fixed`, all from the static region, for callers that cannot
// allocate.
struct Scratch {
    unsigned *counters = nullptr;
    void *part = nullptr;
    TaggedSlots tagged{nullptr, 0, 0, 0};
};
int acquire(bool fixed, cxm_stream_t s, size_t counters, size_t bytes, size_t tagged, Scratch *sc) {
    if (!fixed) {
        if (counters || bytes) {
            Workspace ws;
            const int rc = get_workspace(s, counters, bytes, &ws);
            if (rc) return rc;
            sc->counters = ws.counters;
            sc->part = ws.scratch;
        }
        if (tagged) return get_tagged(s, tagged, &sc->tagged);
        return CXM_OK;
    }
    if (counters * kCtr * sizeof(unsigned) > kFixedCounterBytes || bytes > kFixedPartBytes || tagged > kFixedTagged)
        return CXM_E_TOO_LARGE;
    unsigned char *base = nullptr;
    const int rc = fixed_scratch(s, &base);
    if (rc) return rc;
    sc->counters = reinterpret_cast<unsigned *>(base);
    sc->part = base + kFixedZeroBytes;
    if (tagged) {
        // the static slots serve any caller, captured or not: always cleared
        sc->tagged = TaggedSlots{reinterpret_cast<unsigned long long *>(base + kFixedCounterBytes), kFixedTagged,
                                 next_tag(), 1};
    }
    return CXM_OK;
}

// Max / min over a column path start from the first slice (reduce.cpp:
// 230-236, 285-293), which is the same as starting from -inf / +inf.
struct MaxColOp : MaxOp {
    __device__ static T identity() { return -INFINITY; }
};
struct MinColOp : MinOp {
    __device__ static T identity() { return INFINITY; }
};

// kOutMean / kOutVar scale like reduce.cpp:77-83 / 173-182: outputs below
// `body` multiply by inv (= 1/dim), the rest divide by dimf.
enum OutKind : int {
    kOutValue = 0, kOutMean = 1, kOutIndex = 2, kOutSgd = 3, kOutSqrt = 4, kOutVar = 5, kOutStd = 6
};

struct OutDesc {
    void *z;
    int kind;
    size_t body;  // mean: outputs [0, body) multiply by inv, the rest divide by dimf
    float inv;    // sgd: the learning rate
    float dimf;
};

template <class Op>
__device__ __forceinline__ void write_out(const OutDesc &o, size_t q, typename Op::T r) {
    if constexpr (std::is_same_v<typename Op::T, ArgPair>) {
        static_cast<int32_t *>(o.z)[q] = r.i < 0 ? 0 : r.i;  // -1: a NaN first element
    } else if constexpr (std::is_same_v<typename Op::T, Pow2>) {
        // sum of squared deviations, rounded once to fp32, then scaled as
        // reduce.cpp scales it (population variance)
        const double n = o.dimf;
        const double m2d = r.s2 - r.s1 * (r.s1 / n);
        const float m2 = m2d > 0.0 ? static_cast<float>(m2d) : 0.0f;
        float v = q < o.body ? m2 * o.inv : m2 / o.dimf;
        if (o.kind == kOutStd) v = __builtin_sqrtf(v);
        static_cast<float *>(o.z)[q] = v;
    } else {
        float v = r;
        float *z = static_cast<float *>(o.z);
        if (o.kind == kOutSgd) {  // z is a bias: z - sum*lr, two roundings
            const float t = v * o.inv;
            z[q] = z[q] - t;
            return;
        }
        if (o.kind == kOutMean) v = q < o.body ? v * o.inv : v / o.dimf;
        if (o.kind == kOutSqrt) v = __builtin_sqrtf(v);
        z[q] = v;
    }
}

// Component c of v has index base + c*cstep (rows: consecutive elements,
// cstep 1; columns: four columns of one row, cstep 0).  kShift operators
// get v - k (k: the first element of each component's row or column).
template <class Op>
__device__ __forceinline__ void fold4(typename Op::T (&acc)[4], float4 v, int base, int cstep,
                                      float4 k) {
    if constexpr (Op::kShift) {
        v.x = v.x - k.x;
        v.y = v.y - k.y;
        v.z = v.z - k.z;
        v.w = v.w - k.w;
    }
    acc[0] = Op::accum(acc[0], v.x, base);
    acc[1] = Op::accum(acc[1], v.y, base + cstep);
    acc[2] = Op::accum(acc[2], v.z, base + 2 * cstep);
    acc[3] = Op::accum(acc[3], v.w, base + 3 * cstep);
}

// ------------------------------------------------------------------ rows

constexpr unsigned kTicketGroups = 32;  // per-row ticket counters: 32 groups + 1 top
constexpr unsigned kMaxFlatSegs = 2048;  // segments of a flat reduction (the row plan's largest split)
constexpr size_t kMaxSeg4 = size_t(1) << 27;  // float4s of one segment (byte offsets stay below 2^31)

// A row of `dim` floats at xr (4-byte aligned) read with 128-bit loads: its
// first h (< 4) elements come before the first 16-byte aligned address,
// then v float4s, then t (< 4) elements.
struct RowSplit {
    unsigned h, t;
    size_t v;
};
__device__ __forceinline__ RowSplit split_row(const float *xr, size_t dim) {
    unsigned h = static_cast<unsigned>(((16u - (reinterpret_cast<uintptr_t>(xr) & 15u)) & 15u) / 4u);
    if (h > dim) h = static_cast<unsigned>(dim);
    const size_t v = (dim - h) / 4;
    return {h, static_cast<unsigned>(dim - h - 4 * v), v};
}

// The partial of segment `seg` of one row, block-reduced (valid in every
// thread): float4s [seg * seg4, min(seg * seg4 + seg4, v)) of the row's
// aligned body, UNR loads in flight per thread, folded into four lane
// accumulators in load order; segment 0 also folds the row's head and
// tail elements.  Writers and a reader that recomputes a segment both call
// it, so a recomputed partial has the writer's bits.  Element indices (the
// arg operators) count from the row start; kShift operators get x - xr[0].
template <class Op, int UNR, bool ONE = false>
__device__ __forceinline__ typename Op::T row_segment(const float *__restrict__ xr, size_t dim, unsigned seg,
                                                      size_t seg4, typename Op::T *lds) {
    using T = typename Op::T;
    const int tid = threadIdx.x;
    const RowSplit sp = split_row(xr, dim);
    T acc[4] = {Op::identity(), Op::identity(), Op::identity(), Op::identity()};
    float k = 0.0f;
    if constexpr (Op::kShift) k = xr[0];
    const float4 k4 = make_float4(k, k, k, k);
    const size_t b4 = static_cast<size_t>(seg) * seg4;
    // the segment's float4s as a uniform base and 32-bit per-thread byte
    // offsets (the host keeps a segment under 2^27 float4s): a 64-bit address
    // per load costs two registers each, and the register pressure made the
    // compiler split a batch of loads in two, each waiting for the last
    const unsigned n4 = b4 < sp.v ? static_cast<unsigned>((b4 + seg4 < sp.v ? b4 + seg4 : sp.v) - b4) : 0u;
    const float *__restrict__ sb = xr + sp.h + 4 * b4;
    const int off = static_cast<int>(sp.h + 4 * b4);
    unsigned j = tid;
    if (ONE && __builtin_expect(n4 == UNR * kBlock, 1)) {
        // ONE (the flat writers): one whole batch, every segment but the
        // last in the flat plan, as straight-line code, the loads leaving
        // before any fold.  Without the scheduling barrier the compiler
        // folded the first float4 before issuing the other seven, a memory
        // round trip per workgroup; with it the flat sum went 12.8 -> 12.3
        // us (with the reader's one-barrier check below).  The row plans
        // keep the loop: the row argmax lost 0.2 us to this form
        float4 v[UNR];
#pragma unroll
        for (int u = 0; u < UNR; ++u) v[u] = ld4_stream_at(sb, 16u * (j + u * kBlock));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < UNR; ++u) fold4<Op>(acc, v[u], off + static_cast<int>(4 * (j + u * kBlock)), 1, k4);
        j = n4;
    }
    for (; j + (UNR - 1) * kBlock < n4; j += UNR * kBlock) {
        float4 v[UNR];
#pragma unroll
        for (int u = 0; u < UNR; ++u) v[u] = ld4_stream_at(sb, 16u * (j + u * kBlock));
#pragma unroll
        for (int u = 0; u < UNR; ++u) fold4<Op>(acc, v[u], off + static_cast<int>(4 * (j + u * kBlock)), 1, k4);
    }
    for (; j < n4; j += kBlock) fold4<Op>(acc, ld4_stream_at(sb, 16u * j), off + static_cast<int>(4 * j), 1, k4);
    if (seg == 0) {
        // head elements to threads 0..h-1, tail elements to threads 4..4+t-1
        int i = -1;
        if (tid < static_cast<int>(sp.h)) i = tid;
        else if (tid >= 4 && tid < 4 + static_cast<int>(sp.t)) i = static_cast<int>(sp.h + 4 * sp.v) + (tid - 4);
        if (i >= 0) {
            float e = xr[i];
            if constexpr (Op::kShift) e = e - k;
            acc[0] = Op::accum(acc[0], e, i);
        }
        if (tid == 0) first_nan_fix<Op>(acc[0], xr[0]);
    }
    T r = Op::combine(Op::combine(acc[0], acc[1]), Op::combine(acc[2], acc[3]));
    return block_reduce<Op, kBlock>(r, lds);
}

// Whole rows of exactly NT * UNR float4 from 16-byte aligned bases (every
// row aligned, no head or tail): one NT-thread workgroup per row, its loads
// as straight-line code, then the folds in load order, the wave reductions
// and one LDS exchange; thread 0 writes.  k_rows' one-segment form spent a
// division, segment bounds, a loop test and head/tail code ahead of the
// loads.  Measured A/B at C2's rows: sum 11.5 -> 11.3 us with 256 threads a
// row, 11.2 with 128; max 11.7 -> 11.5 either way; argmax 12.0 -> 11.9 with
// 256 but 12.1 with 128 (its (value, index) fold is twice the work), so the
// 32-bit operators take 128 and the rest 256.
template <class Op>
constexpr int whole_block() { return sizeof(typename Op::T) == 4 ? 128 : 256; }
template <class Op, int UNR>
__global__ __launch_bounds__(whole_block<Op>()) void k_rows_whole(const float *__restrict__ x, size_t dim,
                                                                   OutDesc out) {
    using T = typename Op::T;
    constexpr int NT = whole_block<Op>(), NW = NT / kWave;
    __shared__ T lds[NW];
    const int tid = threadIdx.x;
    tl_mark(kTlRows, 0);
    const float *__restrict__ xr = x + static_cast<size_t>(blockIdx.x) * dim;
    float k = 0.0f;
    if constexpr (Op::kShift) k = xr[0];
    const float4 k4 = make_float4(k, k, k, k);
    float4 v[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u) v[u] = ld4_stream_at(xr, 16u * (tid + u * NT));
    __builtin_amdgcn_sched_barrier(0);
    T acc[4] = {Op::identity(), Op::identity(), Op::identity(), Op::identity()};
#pragma unroll
    for (int u = 0; u < UNR; ++u) fold4<Op>(acc, v[u], 4 * (tid + u * NT), 1, k4);
    if (tid == 0) first_nan_fix<Op>(acc[0], v[0].x);
    T r = Op::combine(Op::combine(acc[0], acc[1]), Op::combine(acc[2], acc[3]));
    r = wave_reduce<Op>(r);
    if ((tid & (kWave - 1)) == 0) lds[tid / kWave] = r;
    __syncthreads();
    tl_mark(kTlRows, 1);
    if (tid == 0) {  // waves in order
        T a = lds[0];
#pragma unroll
        for (int w = 1; w < NW; ++w) a = Op::combine(a, lds[w]);
        write_out<Op>(out, blockIdx.x, a);
    }
    tl_mark(kTlRows, 3);
}

// Reductions over the last axis: workgroup b reduces segment b % segs of
// row b / segs.  MODE 0: one segment per row, written out directly (whole
// aligned rows of one load batch go to k_rows_whole instead).
// MODE 1: segment partials to `part`; the last workgroup of a row (integer
// ticket: one counter per row up to 32 segments, two levels beyond)
// combines them in segment order.  MODE 2 (one row, 32-bit partials, at
// most kMaxFlatSegs segments): the writers store tagged partials and exit,
// with no atomics; one extra workgroup (the last of the grid, dispatched
// after every writer) waits for each tag with at most poll_limit polls,
// recomputes any partial it did not see in time from the input with the
// writer's arithmetic, and combines them in segment order.  A ticket with
// every workgroup of a 2048-segment row arriving on the counters at the end
// serialised there (about 10 ns per atomic on one address): measured on
// gfx950 for a 64 MiB flat sum, two-level ticket 13.1 us, one reader
// polling tagged slots 12.0-12.3 us, streaming alone 11.2 us.  Both combine
// the same partials in the same order, so their results are bit-identical.
// MODE 3 is MODE 2 under a tag that recurs (a graph replays the captured
// one; the static region's callers may be captured): the reader empties
// each slot it used and marks each one it gave up on, and a writer that
// finds the mark empties its slot, so that no partial outlives the kernel
// (`clear` is the host's record of that choice: 1 exactly in MODE 3).
// MODE 2 leaves slots as they are: no later call carries their tag.
//
// The mark is the tag ~epoch, which no partial of the call carries.
__device__ __forceinline__ unsigned long long miss_mark(unsigned epoch) {
    return static_cast<unsigned long long>(~epoch) << 32;
}

template <class Op, int UNR, int MODE>
__global__ __launch_bounds__(kBlock) void k_rows(const float *__restrict__ x, size_t dim, unsigned segs, size_t seg4,
                                                 typename Op::T *__restrict__ part, unsigned *__restrict__ counters,
                                                 unsigned long long *__restrict__ slots, unsigned epoch, int clear,
                                                 unsigned poll_limit, OutDesc out) {
    using T = typename Op::T;
    __shared__ T lds[kWavesPerBlock];
    __shared__ int flag;
    const int tid = threadIdx.x;

    if constexpr (MODE == 2 || MODE == 3) {
        static_assert(sizeof(T) == 4, "tagged slots carry 32-bit partials");
        // MODE 3: the tag is one a graph replays (or the static region's),
        // so slots are emptied after use and given-up ones marked
        constexpr bool CLEAR = MODE == 3;
        constexpr int IT = kMaxFlatSegs / kBlock;
        if (blockIdx.x == segs) {  // the reader
            tl_mark(kTlFlat, 0);
            // The first loads are unconditional (the slot regions hold at
            // least kMaxFlatSegs entries): a load in a branch makes the
            // compiler wait for it at the branch's end, serialising the
            // round trips.  Every writer was dispatched before
            // this workgroup and none waits for anything, so each tag
            // arrives; the poll limit only bounds the wait regardless.
            __shared__ unsigned lmiss[kBlock];
            unsigned long long v[IT];
            T val[IT];
#pragma unroll
            for (int k = 0; k < IT; ++k)
                v[k] = __hip_atomic_load(slots + tid + k * kBlock, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            // then, per slot not yet tagged, in segment order (segments finish
            // roughly in dispatch order): one 8-byte load per thread per round,
            // so the polling traffic stays negligible
            unsigned miss = 0;
#pragma unroll
            for (int k = 0; k < IT; ++k) {
                const unsigned i = tid + k * kBlock;
                val[k] = Op::identity();
                if (i < segs) {
                    unsigned long long w = v[k];
                    unsigned polls = 0;
                    while (static_cast<unsigned>(w >> 32) != epoch && polls < poll_limit) {
                        ++polls;
                        __builtin_amdgcn_s_sleep(1);
                        w = __hip_atomic_load(slots + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
                    if (static_cast<unsigned>(w >> 32) == epoch) {
                        val[k] = __builtin_bit_cast(T, static_cast<unsigned>(w));
                        // `clear` is 0 in MODE 2; tested at run time there all
                        // the same: with the store compiled out, the compiler
                        // kept every copy of val[] live (70 registers, not 46)
                        if (CLEAR || clear) __hip_atomic_store(slots + i, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    } else if constexpr (CLEAR) {
                        // Given up under a tag that a graph replays: leave a
                        // mark, so that the late writer empties the slot
                        // rather than leave its partial, tagged, for the next
                        // replay to take as its own.  A partial that landed
                        // in between is taken after all.
                        const unsigned long long o = __hip_atomic_exchange(slots + i, miss_mark(epoch), __ATOMIC_RELAXED,
                                                                           __HIP_MEMORY_SCOPE_AGENT);
                        if (static_cast<unsigned>(o >> 32) == epoch) {
                            val[k] = __builtin_bit_cast(T, static_cast<unsigned>(o));
                            __hip_atomic_store(slots + i, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        } else {
                            miss |= 1u << k;
                        }
                    } else {
                        miss |= 1u << k;
                    }
                }
            }
            // The block's combine carries whether any slot was missed: with
            // none (the rule) the result is out after one barrier.  A
            // __syncthreads_or ahead of the combine cost three barriers on
            // the kernel's critical path (0.2-0.3 us).
            T a = Op::identity();
#pragma unroll
            for (int k = 0; k < IT; ++k)
                if (tid + k * kBlock < segs) a = Op::combine(a, val[k]);
            {
                __shared__ unsigned wmiss[kWavesPerBlock];
                a = wave_reduce<Op>(a);
                const unsigned wm = __ballot(miss != 0u) != 0ull ? 1u : 0u;
                if ((tid & (kWave - 1)) == 0) {
                    lds[tid / kWave] = a;
                    wmiss[tid / kWave] = wm;
                }
                __syncthreads();
                unsigned any = 0;
#pragma unroll
                for (int w = 0; w < kWavesPerBlock; ++w) any |= wmiss[w];
                if (any == 0u) {  // block_reduce's order: waves 0, 1, 2, 3
                    if (tid == 0) {
                        T r = lds[0];
#pragma unroll
                        for (int w = 1; w < kWavesPerBlock; ++w) r = Op::combine(r, lds[w]);
                        write_out<Op>(out, 0, r);
                    }
                    tl_mark(kTlFlat, 3);
                    return;
                }
                __syncthreads();  // lds is reused below
            }
            // segments not seen in time (none, unless the wait limit is
            // small): recomputed by the whole workgroup with one load in
            // flight per thread -- the writer's fold order (each thread folds
            // its float4s in index order whatever the unroll), so its bits
            lmiss[tid] = miss;
            __syncthreads();
            for (unsigned i = 0; i < segs; ++i) {
                const unsigned t = i % kBlock, k = i / kBlock;
                if (!((lmiss[t] >> k) & 1u)) continue;  // uniform: every thread reads the same word
                const T r = row_segment<Op, 1>(x, dim, i, seg4, lds);
                if (tid == static_cast<int>(t)) {
#pragma unroll
                    for (int q = 0; q < IT; ++q)
                        if (q == static_cast<int>(k)) val[q] = r;
                }
            }
            a = Op::identity();
#pragma unroll
            for (int k = 0; k < IT; ++k)
                if (tid + k * kBlock < segs) a = Op::combine(a, val[k]);
            a = block_reduce<Op, kBlock>(a, lds);
            if (tid == 0) write_out<Op>(out, 0, a);
            return;
        }
        // a writer
        tl_mark(kTlFlat, 0);
        const T r = row_segment<Op, UNR, true>(x, dim, blockIdx.x, seg4, lds);
        tl_mark(kTlFlat, 1);
        if (tid == 0) {
            const unsigned long long v = (static_cast<unsigned long long>(epoch) << 32) | __builtin_bit_cast(unsigned, r);
            if constexpr (CLEAR) {
                // the reader's mark: it recomputed this partial, and the slot
                // goes back to empty (under a replayed tag nothing else would
                // clear it)
                if (__hip_atomic_exchange(slots + blockIdx.x, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                    miss_mark(epoch))
                    __hip_atomic_store(slots + blockIdx.x, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            } else {
                __hip_atomic_store(slots + blockIdx.x, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        tl_mark(kTlFlat, 2);
        return;
    } else {
        // MODE 0 has one segment per row: no division ahead of the loads
        // (its software sequence delayed every workgroup's first load)
        const unsigned b = blockIdx.x;
        const size_t row = MODE == 0 ? b : b / segs;
        const unsigned seg = MODE == 0 ? 0u : b - static_cast<unsigned>(row) * segs;
        const T r = row_segment<Op, UNR>(x + row * dim, dim, seg, seg4, lds);
        if constexpr (MODE == 0) {
            if (tid == 0) write_out<Op>(out, row, r);
        } else {
            if (tid == 0) st_dev(&part[row * segs + seg], r);
            const bool last = segs <= kTicketGroups
                                  ? last_block_ticket(ctr(counters, row), segs, &flag)
                                  : last_block_ticket2<kTicketGroups>(ctr(counters, row * (kTicketGroups + 1)),
                                                                      segs, seg, &flag);
            if (!last) return;
            const unsigned mine = tid < static_cast<int>(segs) ? (segs - tid + kBlock - 1) / kBlock : 0;
            T a = combine_partials<Op>(part + row * segs + tid, mine, kBlock, Op::identity());
            a = block_reduce<Op, kBlock>(a, lds);
            if (tid == 0) write_out<Op>(out, row, a);
        }
    }
}

// Rows whose base is not 4-byte aligned: element by element, one
// workgroup per row.
template <class Op>
__global__ __launch_bounds__(kBlock) void k_rows_bytes(const float *__restrict__ x, size_t dim, OutDesc out) {
    using T = typename Op::T;
    __shared__ T lds[kWavesPerBlock];
    const size_t row = blockIdx.x;
    const float *xr = x + row * dim;
    float k = 0.0f;
    if constexpr (Op::kShift) k = xr[0];
    T acc = Op::identity();
    for (size_t i = threadIdx.x; i < dim; i += kBlock) {
        float e = xr[i];
        if constexpr (Op::kShift) e = e - k;
        acc = Op::accum(acc, e, static_cast<int>(i));
    }
    if (threadIdx.x == 0) first_nan_fix<Op>(acc, xr[0]);
    acc = block_reduce<Op, kBlock>(acc, lds);
    if (threadIdx.x == 0) write_out<Op>(out, row, acc);
}

// ------------------------------------------------------------------ cols

constexpr int kColTile = 256;  // columns per workgroup

// NW waves per workgroup.  Vector path: a wave covers the 256 columns with
// one float4 per lane and wave w takes rows r0+w, r0+w+NW, ...; scalar
// path: thread t owns column t%256 and rows r0+t/256, step NW/4.  The
// per-slot results meet in LDS and threads 0..255 combine them in slot
// order.  Workgroup b -> (chunk, tile, outer slice), chunk fastest: the
// chunks of one tile are adjacent in launch order, so its combine runs
// while later tiles still stream.
template <class Op, bool VEC, int UNR, int NW, bool FAST = false>
__global__ __launch_bounds__(NW * kWave) void k_cols(const float *__restrict__ x, size_t dim,
                                                     size_t inner, unsigned ntiles, unsigned chunks,
                                                     size_t rows_per_chunk, typename Op::T *__restrict__ part,
                                                     unsigned *__restrict__ counters, OutDesc out) {
    using T = typename Op::T;
    constexpr int NSLOT = VEC ? NW : NW / 4;
    __shared__ T lds[NSLOT][kColTile];
    __shared__ int flag;

    // FAST launches a (chunks, tiles, outer) grid: no index arithmetic ahead
    // of the first load (the two divisions of a flat grid's index took some
    // 60 instructions; decoding either form behind a branch made the
    // compiler load the kernel arguments in two rounds).  Other forms take a
    // flat grid, decoded with 32-bit divisions (fewer than 2^31 workgroups).
    unsigned chunk, tile;
    size_t o;
    if constexpr (FAST) {
        chunk = blockIdx.x;
        tile = blockIdx.y;
        o = blockIdx.z;
    } else {
        const unsigned b = blockIdx.x;
        const unsigned q = b / chunks;
        chunk = b - q * chunks;
        tile = q % ntiles;
        o = q / ntiles;
    }
    const int tid = threadIdx.x;
    tl_mark(kTlColsArg, 0);
    const float *__restrict__ xo = x + o * dim * inner;
    const size_t r0 = chunk * rows_per_chunk;
    const size_t r1 = r0 + rows_per_chunk < dim ? r0 + rows_per_chunk : dim;

    if constexpr (VEC) {
        const int lane = tid & (kWave - 1);
        const int w = tid / kWave;
        const size_t col = static_cast<size_t>(tile) * kColTile + lane * 4;
        T acc[4] = {Op::identity(), Op::identity(), Op::identity(), Op::identity()};
        // FAST (whole tiles, a chunk under 2^31 bytes): no column bound to
        // branch on, so every operand is at hand from the start -- behind
        // the branch the compiler fetched the input pointer in a second
        // round of kernel-argument loads after the index arithmetic, a
        // scalar-cache miss in every workgroup (one per CU here)
        if (FAST || col < inner) {
            const float *__restrict__ xc = xo + col;
            float4 k4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if constexpr (Op::kShift) k4 = ld4(xc);
            if constexpr (FAST) {
                // the chunk as a uniform base and 32-bit byte offsets: one
                // address register per load instead of two
                const float *__restrict__ cb = xo + r0 * inner + static_cast<size_t>(tile) * kColTile;
                const unsigned rowb = static_cast<unsigned>(inner * sizeof(float)), nr = static_cast<unsigned>(r1 - r0);
                const unsigned c16 = static_cast<unsigned>(lane * 16);
                // row offsets as a per-lane column offset plus uniform row
                // offsets (the wave index made uniform, so the products are
                // scalar): a multiply per load had put 16 quarter-rate vector
                // multiplies between the index arithmetic and the first load
                const unsigned wu = __builtin_amdgcn_readfirstlane(static_cast<unsigned>(w));
                const unsigned step = NW * rowb;
                unsigned r = wu, ro = wu * rowb + c16;
                for (; r + (UNR - 1) * NW < nr; r += UNR * NW, ro += UNR * step) {
                    float4 v[UNR];
#pragma unroll
                    for (int u = 0; u < UNR; ++u) v[u] = ld4_stream_at(cb, ro + u * step);
                    // all UNR loads leave before any is folded: left alone, the
                    // scheduler interleaved the folds to stay at 64 registers
                    // and kept 5-6 loads in flight (one 16-wave workgroup per
                    // CU leaves room for 128); streaming 12.1 -> 11.8 us at C2
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int u = 0; u < UNR; ++u) fold4<Op>(acc, v[u], static_cast<int>(r0 + r + u * NW), 0, k4);
                }
                for (; r < nr; r += NW, ro += step) fold4<Op>(acc, ld4_stream_at(cb, ro), static_cast<int>(r0 + r), 0, k4);
            } else {
                size_t r = r0 + w;
                for (; r + (UNR - 1) * NW < r1; r += UNR * NW) {
                    float4 v[UNR];
#pragma unroll
                    for (int u = 0; u < UNR; ++u) v[u] = ld4_stream(xc + (r + u * NW) * inner);
#pragma unroll
                    for (int u = 0; u < UNR; ++u) fold4<Op>(acc, v[u], static_cast<int>(r + u * NW), 0, k4);
                }
                for (; r < r1; r += NW) fold4<Op>(acc, ld4_stream(xc + r * inner), static_cast<int>(r), 0, k4);
            }
            if constexpr (std::is_same_v<T, ArgPair>) {
                if (r0 == 0 && w == 0) {  // row 0 of these four columns
                    const float4 x0 = ld4(xc);
                    first_nan_fix<Op>(acc[0], x0.x);
                    first_nan_fix<Op>(acc[1], x0.y);
                    first_nan_fix<Op>(acc[2], x0.z);
                    first_nan_fix<Op>(acc[3], x0.w);
                }
            }
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) lds[w][lane * 4 + c] = acc[c];
    } else {
        const int c = tid % kColTile, ph = tid / kColTile;
        const size_t col = static_cast<size_t>(tile) * kColTile + c;
        T mine = Op::identity();
        if (col < inner) {
            float k = 0.0f;
            if constexpr (Op::kShift) k = xo[col];
            for (size_t r = r0 + ph; r < r1; r += NSLOT) {
                float v = xo[r * inner + col];
                if constexpr (Op::kShift) v = v - k;
                mine = Op::accum(mine, v, static_cast<int>(r));
            }
            if (r0 == 0 && ph == 0) first_nan_fix<Op>(mine, xo[col]);
        }
        lds[ph][c] = mine;
    }
    __syncthreads();
    tl_mark(kTlColsArg, 1);
    const bool owner = tid < kColTile;  // threads 0..255 own one column each from here
    T mine = Op::identity();
    if (owner) {
        mine = lds[0][tid];
#pragma unroll
        for (int k = 1; k < NSLOT; ++k) mine = Op::combine(mine, lds[k][tid]);
    }
    const size_t col = static_cast<size_t>(tile) * kColTile + tid;
    if (chunks == 1) {
        if (owner && (FAST || col < inner)) write_out<Op>(out, o * inner + col, mine);
        return;
    }
    const size_t slot = (o * ntiles + tile) * chunks;
    if (owner) st_dev(&part[(slot + chunk) * kColTile + tid], mine);
    const bool last = last_block_ticket(ctr(counters, o * ntiles + tile), chunks, &flag);
    tl_mark(kTlColsArg, 2);
    if (!last) return;
    if (owner) {
        const T a = combine_partials<Op>(part + slot * kColTile + tid, chunks, kColTile, Op::identity());
        if (FAST || col < inner) write_out<Op>(out, o * inner + col, a);
    }
    tl_mark(kTlColsArg, 3);
}

// Column chunks of exactly 256 rows over whole 256-column tiles (C2's
// column reductions: 16 chunks of 256 rows): k_cols' FAST form with its one
// 16-load batch per wave as straight-line code and the index arithmetic cut
// to a few scalar products (no chunk bounds, no loop tests); same fold,
// combine and ticket order, so the same bits.  Grid (chunks, tiles, outer).
// Measured A/B at C2: column sum 13.4 -> 13.3 us, max 13.6 -> 13.4.
constexpr int kWholeRows = 256;  // rows of a chunk: 16 waves x 16 loads
template <class Op>
__global__ __launch_bounds__(16 * kWave) void k_cols_whole(const float *__restrict__ x, size_t slice,
                                                           unsigned inner, unsigned ntiles, unsigned chunks,
                                                           typename Op::T *__restrict__ part,
                                                           unsigned *__restrict__ counters, OutDesc out) {
    using T = typename Op::T;
    constexpr int NW = 16, UNR = 16;
    __shared__ T lds[NW][kColTile];
    __shared__ int flag;
    const unsigned chunk = blockIdx.x, tile = blockIdx.y, o = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    tl_mark(kTlCols, 0);
    const unsigned w = __builtin_amdgcn_readfirstlane(static_cast<unsigned>(tid / kWave));
    const float *__restrict__ xo = x + o * slice + static_cast<size_t>(tile) * kColTile;
    // this wave's first row of the chunk: row chunk * 256 + w, then every 16th
    const float *__restrict__ wb = xo + (static_cast<size_t>(chunk) * kWholeRows + w) * inner;
    const unsigned step = NW * inner * 4u, c16 = static_cast<unsigned>(lane * 16);
    float4 k4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if constexpr (Op::kShift) k4 = ld4(xo + lane * 4);
    float4 v[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u) v[u] = ld4_stream_at(wb, c16 + u * step);
    __builtin_amdgcn_sched_barrier(0);
    T acc[4] = {Op::identity(), Op::identity(), Op::identity(), Op::identity()};
    const int r0 = static_cast<int>(chunk * kWholeRows + w);
#pragma unroll
    for (int u = 0; u < UNR; ++u) fold4<Op>(acc, v[u], r0 + u * NW, 0, k4);
#pragma unroll
    for (int c = 0; c < 4; ++c) lds[w][lane * 4 + c] = acc[c];
    __syncthreads();
    tl_mark(kTlCols, 1);
    const bool owner = tid < kColTile;
    T mine = Op::identity();
    if (owner) {
        mine = lds[0][tid];
#pragma unroll
        for (int k = 1; k < NW; ++k) mine = Op::combine(mine, lds[k][tid]);
    }
    const size_t slot = (static_cast<size_t>(o) * ntiles + tile) * chunks;
    if (owner) st_dev(&part[(slot + chunk) * kColTile + tid], mine);
    const bool last = last_block_ticket(ctr(counters, static_cast<size_t>(o) * ntiles + tile), chunks, &flag);
    tl_mark(kTlCols, 2);
    if (!last) return;
    if (owner) {
        const T a = combine_partials<Op>(part + slot * kColTile + tid, chunks, kColTile, Op::identity());
        write_out<Op>(out, static_cast<size_t>(o) * inner + static_cast<size_t>(tile) * kColTile + tid, a);
    }
    tl_mark(kTlCols, 3);
}

__global__ void k_fill_f32(float *z, float v) { *z = v; }

// ------------------------------------------------------------------ host

constexpr unsigned kTargetBlocks = 2048;

template <class Op, int UNR, int MODE>
void launch_rows(unsigned nb, hipStream_t hs, const float *x, size_t dim, unsigned segs, size_t seg4,
                 typename Op::T *part, unsigned *counters, const TaggedSlots &tg, OutDesc out) {
    hipLaunchKernelGGL((k_rows<Op, UNR, MODE>), dim3(nb), dim3(kBlock), 0, hs, x, dim, segs, seg4, part, counters,
                       tg.slots, tg.epoch, tg.clear, exchange_wait_limit(), out);
}

// Row plan: each row cut into `segs` segments of seg4 float4s (a multiple
// of 256, i.e. 1024 floats), so that the grid has about kTargetBlocks
// workgroups when rows are few.
template <class Op>
int run_rows(const float *x, size_t rows, size_t dim, OutDesc out, cxm_stream_t s, bool fixed = false) {
    using T = typename Op::T;
    hipStream_t hs = reinterpret_cast<hipStream_t>(s);
    if ((reinterpret_cast<uintptr_t>(x) & 3u) != 0) {
        if (rows > 0x7fffffffu) return CXM_E_TOO_LARGE;
        hipLaunchKernelGGL(k_rows_bytes<Op>, dim3(static_cast<unsigned>(rows)), dim3(kBlock), 0, hs, x, dim, out);
        return launch_status();
    }
    const size_t v4 = (dim + 3) / 4;  // float4s of the longest aligned body (rounded up; a row has at most this many)
    size_t segs = 1;
    if (rows < kTargetBlocks) {
        const size_t want = (kTargetBlocks + rows - 1) / rows;
        const size_t max_segs = (v4 + 255) / 256;
        segs = want < max_segs ? want : max_segs;
        if (segs == 0) segs = 1;
    }
    size_t seg4 = (v4 + segs - 1) / segs;
    seg4 = (seg4 + 255) / 256 * 256;
    if (seg4 == 0) seg4 = 256;
    if (seg4 > kMaxSeg4) seg4 = kMaxSeg4;  // 32-bit byte offsets within a segment
    segs = (v4 + seg4 - 1) / seg4;
    if (segs == 0) segs = 1;
    const size_t blocks = rows * segs;
    if (blocks > 0x7fffffffu) return CXM_E_TOO_LARGE;
    const unsigned nb = static_cast<unsigned>(blocks), sg = static_cast<unsigned>(segs);
    const bool unr8 = seg4 / kBlock >= 8;  // float4 loads per thread per segment
    T *part = nullptr;
    unsigned *counters = nullptr;
    TaggedSlots tg{nullptr, 0, 0, 0};
    const int mode = segs == 1 ? 0 : (rows == 1 && sizeof(T) == 4 && segs <= kMaxFlatSegs ? 2 : 1);
    // whole aligned rows of one batch (every row starts 16-byte aligned)
    if (mode == 0 && aligned16(x) && dim % 4 == 0) {
        const unsigned nr = static_cast<unsigned>(rows);
        constexpr int nt = whole_block<Op>();
#define CXM_WHOLE(U)                                                                                    \
    if (v4 == static_cast<size_t>(U) * nt) {                                                            \
        hipLaunchKernelGGL((k_rows_whole<Op, U>), dim3(nr), dim3(nt), 0, hs, x, dim, out);             \
        return launch_status();                                                                         \
    }
        CXM_WHOLE(4)
        CXM_WHOLE(8)
        CXM_WHOLE(16)
#undef CXM_WHOLE
    }
    if (mode == 1) {
        const size_t nctr = segs <= kTicketGroups ? rows : rows * (kTicketGroups + 1);
        Scratch sc;
        int rc = acquire(fixed, s, nctr, rows * segs * sizeof(T), 0, &sc);
        if (rc) return rc;
        part = static_cast<T *>(sc.part);
        counters = sc.counters;
    } else if (mode == 2) {
        Scratch sc;
        int rc = acquire(fixed, s, 0, 0, segs, &sc);
        if (rc) return rc;
        tg = sc.tagged;
    }
    const unsigned grid = mode == 2 ? nb + 1 : nb;
    const bool replayed = mode == 2 && tg.clear;  // MODE 3
#define CXM_ROWS(U, M) launch_rows<Op, U, M>(grid, hs, x, dim, sg, seg4, part, counters, tg, out)
    if (mode == 0) { if (unr8) CXM_ROWS(8, 0); else CXM_ROWS(4, 0); }
    else if (mode == 1) { if (unr8) CXM_ROWS(8, 1); else CXM_ROWS(4, 1); }
    else if constexpr (sizeof(T) == 4) {
        if (replayed) { if (unr8) CXM_ROWS(8, 3); else CXM_ROWS(4, 3); }
        else { if (unr8) CXM_ROWS(8, 2); else CXM_ROWS(4, 2); }
    }
#undef CXM_ROWS
    return launch_status();
}

struct ColPlan {
    int nw;          // waves per workgroup (4 or 16)
    size_t chunks;   // row chunks per column tile
};

// Default plan: 16-wave workgroups, about one per CU in total from 16
// column tiles up and about 128 below (few chunks, so the last-workgroup
// combine reads few partials).  Measured chunk sweeps (column sum, us):
// [4096, 1024] 64 chunks 8.2, 32 chunks 7.0; [2048, 2048] 32: 7.2, 16: 6.5;
// [8192, 512] 128: 11.0, 64: 8.1; [4096, 4096] 16: 13.1, 8: 14.8.
ColPlan col_plan(size_t tiles, size_t dim) {
    ColPlan p{16, 1};
    const size_t target = tiles >= 16 ? 256 : 128;
    if (tiles < target) {
        size_t want = (target + tiles - 1) / tiles;
        const size_t max_chunks = (dim + 63) / 64;  // >= 4 rows per wave
        p.chunks = want < max_chunks ? want : max_chunks;
        if (p.chunks == 0) p.chunks = 1;
    }
    return p;
}

template <class Op, int UNRC = 8>
int run_cols_plan(const float *x, size_t outer, size_t dim, size_t inner, OutDesc out, ColPlan plan,
                  cxm_stream_t s, bool fixed = false) {
    using T = typename Op::T;
    hipStream_t hs = reinterpret_cast<hipStream_t>(s);
    const bool vec = aligned16(x) && inner % 4 == 0;
    const size_t ntiles = (inner + kColTile - 1) / kColTile;
    const size_t tiles = ntiles * outer;
    size_t chunks = plan.chunks < 1 ? 1 : plan.chunks;
    size_t rpc = (dim + chunks - 1) / chunks;
    rpc = (rpc + 15) / 16 * 16;
    chunks = (dim + rpc - 1) / rpc;
    if (chunks == 0) chunks = 1;
    const size_t blocks = tiles * chunks;
    if (blocks > 0x7fffffffu || ntiles > 0xffffffffu) return CXM_E_TOO_LARGE;

    T *part = nullptr;
    unsigned *counters = nullptr;
    if (chunks > 1) {
        Scratch sc;
        int rc = acquire(fixed, s, tiles, tiles * chunks * kColTile * sizeof(T), 0, &sc);
        if (rc) return rc;
        part = static_cast<T *>(sc.part);
        counters = sc.counters;
    }
    const unsigned nt = static_cast<unsigned>(ntiles), nc = static_cast<unsigned>(chunks);
    // FAST: whole float4 tiles and 32-bit byte offsets within a chunk (under
    // 2^31 bytes), on a (chunks, tiles, outer) grid, so tiles and outer
    // slices must fit its y and z dimensions; other forms take a flat grid,
    // whose work-item count is a 32-bit field of the dispatch
    const bool fast = vec && inner % kColTile == 0 &&
                      (rpc * inner + kColTile) * sizeof(float) < (size_t(1) << 31) && ntiles <= 65535 &&
                      outer <= 65535;
    if (!fast && blocks * static_cast<size_t>(plan.nw) * kWave > 0xffffffffu) return CXM_E_TOO_LARGE;
    const dim3 grid = fast ? dim3(nc, nt, static_cast<unsigned>(outer)) : dim3(static_cast<unsigned>(blocks));
#define CXM_COLS(VEC_, UNR_, NW_)                                                                              \
    do {                                                                                                       \
        if (VEC_ && fast)                                                                                      \
            hipLaunchKernelGGL((k_cols<Op, VEC_, UNR_, NW_, true>), grid, dim3(NW_ * kWave), 0, hs, x, dim,      \
                               inner, nt, nc, rpc, part, counters, out);                                       \
        else                                                                                                   \
            hipLaunchKernelGGL((k_cols<Op, VEC_, UNR_, NW_>), grid, dim3(NW_ * kWave), 0, hs, x, dim, inner,      \
                               nt, nc, rpc, part, counters, out);                                              \
    } while (0)
    if constexpr (sizeof(T) == 4) {  // the column argmax measured 14.3 -> 14.5 us in this form
        if (fast && plan.nw == 16 && chunks > 1 && rpc == kWholeRows && dim == chunks * kWholeRows &&
            inner <= 0xffffffffu) {
            hipLaunchKernelGGL(k_cols_whole<Op>, grid, dim3(16 * kWave), 0, hs, x, dim * inner,
                               static_cast<unsigned>(inner), nt, nc, part, counters, out);
            return launch_status();
        }
    }
    if (plan.nw == 16) {
        // With a multiple of 16 rows per wave, all 16 loads of a batch are in
        // flight together (C2's column reductions: 13.4 against 13.8 us with
        // batches of 8); other chunk sizes keep batches of UNRC, since rows
        // past the last whole batch load one at a time.
        if (vec && (rpc / 16) % 16 == 0) CXM_COLS(true, 16, 16);
        else if (vec) CXM_COLS(true, UNRC, 16);
        else CXM_COLS(false, 1, 16);
    } else {
        if (vec) CXM_COLS(true, UNRC, 4);
        else CXM_COLS(false, 1, 4);
    }
#undef CXM_COLS
    return launch_status();
}

template <class Op>
int run_cols(const float *x, size_t outer, size_t dim, size_t inner, OutDesc out, cxm_stream_t s,
             bool fixed = false) {
    const size_t tiles = (inner + kColTile - 1) / kColTile * outer;
    return run_cols_plan<Op>(x, outer, dim, inner, out, col_plan(tiles, dim), s, fixed);
}

enum Which { kSum, kMean, kMax, kArgMax, kMin, kArgMin, kNorm1, kNorm2, kVar, kStdv };

OutKind out_kind(Which w) {
    switch (w) {
        case kMean: return kOutMean;
        case kArgMax:
        case kArgMin: return kOutIndex;
        case kNorm2: return kOutSqrt;
        case kVar: return kOutVar;
        case kStdv: return kOutStd;
        default: return kOutValue;
    }
}

int reduce_axis(Which which, const float *x, void *z, size_t outer, size_t dim, size_t inner,
                cxm_stream_t s) {
    if (!x || !z) return CXM_E_INVALID;
    if (outer == 0 || inner == 0) return CXM_OK;  // empty output
    if (dim == 0) return CXM_E_INVALID;
    if ((which == kArgMax || which == kArgMin) && dim > 0x7fffffffu) return CXM_E_TOO_LARGE;
    const size_t total = outer * inner;
    // var over rows divides (reduce.cpp:135); over columns it scales like mean
    const size_t body = (which == kVar || which == kStdv) && inner == 1 ? 0 : total - total % 8;
    OutDesc out{z, out_kind(which), body, 1.0f / static_cast<float>(dim), static_cast<float>(dim)};
    if (inner == 1) {
        switch (which) {
            case kSum:
            case kMean: return run_rows<SumOp>(x, outer, dim, out, s);
            case kMax: return run_rows<MaxOp>(x, outer, dim, out, s);
            case kArgMax: return run_rows<ArgMaxOp>(x, outer, dim, out, s);
            case kMin: return run_rows<MinOp>(x, outer, dim, out, s);
            case kArgMin: return run_rows<ArgMinOp>(x, outer, dim, out, s);
            case kNorm1: return run_rows<AbsSumOp>(x, outer, dim, out, s);
            case kNorm2: return run_rows<SqSumOp>(x, outer, dim, out, s);
            default: return run_rows<Pow2Op>(x, outer, dim, out, s);
        }
    }
    switch (which) {
        case kSum:
        case kMean: return run_cols<SumOp>(x, outer, dim, inner, out, s);
        case kMax: return run_cols<MaxColOp>(x, outer, dim, inner, out, s);
        case kArgMax: return run_cols<ArgMaxOp>(x, outer, dim, inner, out, s);
        case kMin: return run_cols<MinColOp>(x, outer, dim, inner, out, s);
        case kArgMin: return run_cols<ArgMinOp>(x, outer, dim, inner, out, s);
        case kNorm1: return run_cols<AbsSumOp>(x, outer, dim, inner, out, s);
        case kNorm2: return run_cols<SqSumOp>(x, outer, dim, inner, out, s);
        default: return run_cols<Pow2Op>(x, outer, dim, inner, out, s);
    }
}

// cxm_reduce_sum_f32 with its scratch in the static region: the same
// checks, plan and kernels, so the same bits.
int reduce_sum_fixed(const float *x, float *z, size_t outer, size_t dim, size_t inner, cxm_stream_t s) {
    if (!x || !z) return CXM_E_INVALID;
    if (outer == 0 || inner == 0) return CXM_OK;
    if (dim == 0) return CXM_E_INVALID;
    OutDesc out{z, kOutValue, 0, 1.0f / static_cast<float>(dim), static_cast<float>(dim)};
    if (inner == 1) return run_rows<SumOp>(x, outer, dim, out, s, true);
    return run_cols<SumOp>(x, outer, dim, inner, out, s, true);
}

int reduce_flat(Which which, const float *x, void *z, size_t n, cxm_stream_t s) {
    if (!z) return CXM_E_INVALID;
    hipStream_t hs = reinterpret_cast<hipStream_t>(s);
    if (n == 0) {
        // The reference on zero elements: sum/norm1/norm2 0 (reduce.cpp:17-28,
        // 311-322, 369-381), mean/var/stdv 0/0 (:66-69, 86-104), max -FLT_MAX
        // (:204-215), min FLT_MAX (:253-264).  argmax/argmin read x[0].
        if (which == kArgMax || which == kArgMin) return CXM_E_INVALID;
        float v = 0.0f;
        if (which == kMean || which == kVar || which == kStdv) v = NAN;
        if (which == kMax) v = -FLT_MAX;
        if (which == kMin) v = FLT_MAX;
        hipLaunchKernelGGL(k_fill_f32, dim3(1), dim3(1), 0, hs, static_cast<float *>(z), v);
        return launch_status();
    }
    if (!x) return CXM_E_INVALID;
    if ((which == kArgMax || which == kArgMin) && n > 0x7fffffffu) return CXM_E_TOO_LARGE;
    OutDesc out{z, out_kind(which), 0, 0.0f, static_cast<float>(n)};
    switch (which) {
        case kSum:
        case kMean: return run_rows<SumOp>(x, 1, n, out, s);
        case kMax: return run_rows<MaxOp>(x, 1, n, out, s);
        case kArgMax: return run_rows<ArgMaxOp>(x, 1, n, out, s);
        case kMin: return run_rows<MinOp>(x, 1, n, out, s);
        case kArgMin: return run_rows<ArgMinOp>(x, 1, n, out, s);
        case kNorm1: return run_rows<AbsSumOp>(x, 1, n, out, s);
        case kNorm2: return run_rows<SqSumOp>(x, 1, n, out, s);
        default: return run_rows<Pow2Op>(x, 1, n, out, s);
    }
}

}  // namespace

int colsum_sgd(const float *x, float *b, size_t rows, size_t cols, float lr, cxm_stream_t s) {
    if (!x || !b || rows == 0) return CXM_E_INVALID;
    if (cols == 0) return CXM_OK;
    OutDesc out{b, kOutSgd, 0, lr, 0.0f};
    return run_cols<SumOp>(x, 1, rows, cols, out, s);
}

}  // namespace cxm

#ifdef CXM_TIMELINE
// Diagnostics build only (not declared in include/cxm_hip.h): copies the
// timeline tables, kTimelineKinds x kTimelineWgs x kTimelineMarks 64-bit
// words, to host memory (after the caller's synchronisation).
extern "C" int cxm_timeline_read(unsigned long long *host, size_t words) {
    if (!host || words != static_cast<size_t>(kTimelineKinds) * kTimelineWgs * kTimelineMarks) return CXM_E_INVALID;
    const hipError_t e = hipMemcpyFromSymbol(host, HIP_SYMBOL(timeline), words * sizeof(unsigned long long));
    return e == hipSuccess ? CXM_OK : static_cast<int>(e);
}
#endif

extern "C" {

int cxm_reduce_sum_flat_f32(const float *x, float *z, size_t n, cxm_stream_t s) {
    return cxm::reduce_flat(cxm::kSum, x, z, n, s);
}
int cxm_reduce_mean_flat_f32(const float *x, float *z, size_t n, cxm_stream_t s) {
    return cxm::reduce_flat(cxm::kMean, x, z, n, s);
}
int cxm_reduce_max_flat_f32(const float *x, float *z, size_t n, cxm_stream_t s) {
    return cxm::reduce_flat(cxm::kMax, x, z, n, s);
}
int cxm_reduce_argmax_flat_f32(const float *x, int32_t *z, size_t n, cxm_stream_t s) {
    return cxm::reduce_flat(cxm::kArgMax, x, z, n, s);
}
int cxm_reduce_sum_f32(const float *x, float *z, size_t outer, size_t dim, size_t inner,
                       cxm_stream_t s) {
    return cxm::reduce_axis(cxm::kSum, x, z, outer, dim, inner, s);
}
int cxm_reduce_mean_f32(const float *x, float *z, size_t outer, size_t dim, size_t inner,
                        cxm_stream_t s) {
    return cxm::reduce_axis(cxm::kMean, x, z, outer, dim, inner, s);
}
int cxm_reduce_max_f32(const float *x, float *z, size_t outer, size_t dim, size_t inner,
                       cxm_stream_t s) {
    return cxm::reduce_axis(cxm::kMax, x, z, outer, dim, inner, s);
}
int cxm_reduce_argmax_f32(const float *x, int32_t *z, size_t outer, size_t dim, size_t inner,
                          cxm_stream_t s) {
    return cxm::reduce_axis(cxm::kArgMax, x, z, outer, dim, inner, s);
}

int cxm_reduce_sum_noalloc_f32(const float *x, float *z, size_t outer, size_t dim, size_t inner,
                               cxm_stream_t s) {
    return cxm::reduce_sum_fixed(x, z, outer, dim, inner, s);
}

#define CXM_REDUCE_ENTRY(NAME, WHICH, ZT)                                                            \
    int cxm_reduce_##NAME##_flat_f32(const float *x, ZT *z, size_t n, cxm_stream_t s) {             \
        return cxm::reduce_flat(cxm::WHICH, x, z, n, s);                                           \
    }                                                                                               \
    int cxm_reduce_##NAME##_f32(const float *x, ZT *z, size_t outer, size_t dim, size_t inner,     \
                                cxm_stream_t s) {                                                   \
        return cxm::reduce_axis(cxm::WHICH, x, z, outer, dim, inner, s);                           \
    }
CXM_REDUCE_ENTRY(min, kMin, float)
CXM_REDUCE_ENTRY(argmin, kArgMin, int32_t)
CXM_REDUCE_ENTRY(norm1, kNorm1, float)
CXM_REDUCE_ENTRY(norm2, kNorm2, float)
CXM_REDUCE_ENTRY(var, kVar, float)
CXM_REDUCE_ENTRY(stdv, kStdv, float)
#undef CXM_REDUCE_ENTRY

}  // extern "C"
