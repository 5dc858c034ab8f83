/*
 * cxm_hip.h -- C ABI of the CortexMind MI355X (gfx950) backend.
 *
 * Plain C: raw pointers, element counts and an opaque stream handle; no
 * torch, no HIP or CUDA types in the signatures.  Every entry point returns
 * an int status: CXM_OK (0) on success, a negative CXM_E_* code for an
 * argument error detected on the host before anything is launched, or a
 * positive HIP runtime error code.  Kernels launch asynchronously on the
 * given stream (NULL = the device's null stream); only the d2h copy and the
 * *_sync calls block the host.
 *
 * Ownership follows the reference engine: the caller owns every buffer and
 * ops write into a preallocated output (reference
 * source/CortexMind/framework/Engine/AVX2/reduce.hpp:49-329 and
 * Engine/CUDA/matrix.cuh:11-26: no op allocates its output).  Multi-pass
 * kernels take their scratch from a per-(device, stream) workspace that the
 * library allocates on first use and keeps until cxm_release_workspaces();
 * calls on distinct streams are independent, calls on one stream are ordered.
 *
 * Reference paths below are relative to source/CortexMind/framework/.
 */
#ifndef CXM_HIP_H
#define CXM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t *cxm_stream_t; /* a hipStream_t; NULL = null stream */
typedef struct ihipEvent_t *cxm_event_t;   /* a hipEvent_t */

/* ---------------------------------------------------------------- status */
#define CXM_OK 0
#define CXM_E_INVALID (-1)     /* null pointer, zero/mismatched size, bad enum */
#define CXM_E_TOO_LARGE (-2)   /* size beyond what the kernel indexes (int32 argmax etc.) */
#define CXM_E_NO_DEVICE (-3)   /* no gfx950 device visible */
/* The stream is capturing a HIP graph and the call needs scratch (the
 * stream's workspace, exchange region or tagged slots) that the stream does
 * not have yet, or not large enough: nothing was allocated, filled, waited
 * for or launched.  Make one eager call of the same shapes on the stream
 * before capture. */
#define CXM_E_CAPTURE (-4)

/* Binary operator codes (Engine/AVX2/broadcast.hpp:29-56, Engine/AVX2/matrix.hpp:38-94). */
#define CXM_OP_ADD 0
#define CXM_OP_SUB 1
#define CXM_OP_MUL 2
#define CXM_OP_DIV 3
#define CXM_OP_MAX 4
#define CXM_OP_MIN 5
#define CXM_OP_POW 6 /* powf(x, y): same-shape and scalar forms only */

/* Activation codes (Engine/AVX2/functions.hpp:186-188 exp, 372-374 relu,
 * 381-383 tanh, 405-411 sigmoid). */
#define CXM_ACT_NONE 0
#define CXM_ACT_RELU 1
#define CXM_ACT_SIGMOID 2
#define CXM_ACT_TANH 3
#define CXM_ACT_EXP 4

/* Elementwise math codes for cxm_wise_f32: nv::ElementWise
 * (Engine/CUDA/element_wise.cuh:11-27) and avx2::wise (Engine/AVX2/wise.hpp:28-42). */
#define CXM_FN_SQUARE 0
#define CXM_FN_SQRT 1
#define CXM_FN_RSQRT 2
#define CXM_FN_LOG 3
#define CXM_FN_EXP 4
#define CXM_FN_ERF 5
#define CXM_FN_SIN 6
#define CXM_FN_COS 7
#define CXM_FN_ABS 8
#define CXM_FN_NEG 9
#define CXM_FN_RCP 10
#define CXM_FN_INVERSE 11
#define CXM_FN_SIGN 12

/* Element types of the dtype-generic entry points (Type/dtype.hpp's
 * Float32 / BFloat16 / Float16). */
#define CXM_DT_F32 0
#define CXM_DT_BF16 1
#define CXM_DT_F16 2

/* Human-readable text for a status code (never NULL). */
const char *cxm_error_string(int status);

/* ------------------------------------------------ device, memory, streams
 * Replace the reference's device pool and copies:
 *   ForgeChunk::allocate / deallocate (Memory/forge.cu:28-89),
 *   transform::upload / download / copy_d2d (Memory/transform.cu:17-40),
 *   nv::stream (Engine/CUDA/stream.cu:10-43). */
int cxm_device_count(int *count);
int cxm_set_device(int device);
/* Name, compute-unit count and gcn arch string ("gfx950...") of the current device. */
int cxm_device_info(char *name, size_t name_len, int *cu_count, char *arch, size_t arch_len);
int cxm_device_sync(void);
int cxm_dev_malloc(void **ptr, size_t bytes);
int cxm_dev_free(void *ptr);
int cxm_memcpy_h2d(void *dst, const void *src, size_t bytes, cxm_stream_t s);
/* Copies and then waits for the stream, like the reference's blocking download. */
int cxm_memcpy_d2h(void *dst, const void *src, size_t bytes, cxm_stream_t s);
int cxm_memcpy_d2d(void *dst, const void *src, size_t bytes, cxm_stream_t s);
int cxm_memset(void *dst, int byte_value, size_t bytes, cxm_stream_t s);
int cxm_stream_create(cxm_stream_t *s);
int cxm_stream_sync(cxm_stream_t s);
int cxm_stream_destroy(cxm_stream_t s);
int cxm_event_create(cxm_event_t *e);
int cxm_event_record(cxm_event_t e, cxm_stream_t s);
int cxm_event_sync(cxm_event_t e);
int cxm_event_elapsed_ms(float *ms, cxm_event_t start, cxm_event_t stop);
int cxm_event_destroy(cxm_event_t e);
/* Frees every workspace the library holds (waits for their streams first).
 * Scratch regions are per (device, stream) and only grow.  A region handed
 * to a launch recorded under stream capture is pinned: a later growth keeps
 * it allocated, so the graph stays valid; it is freed by
 * cxm_release_workspaces or by cxm_stream_destroy of its stream, which end
 * every graph captured on that stream.  Under capture a missing or too
 * small region is CXM_E_CAPTURE (see above). */
int cxm_release_workspaces(void);
/* Diagnostics, no reference counterpart: the current device's scratch
 * region `which` (0 workspace, 1 exchange region, 2 tagged slots) of
 * stream s -- its base (NULL if none yet), size in bytes, and whether a
 * captured launch holds it (pinned). */
int cxm_workspace_query(cxm_stream_t s, int which, void **base, size_t *bytes, int *pinned);

/* Stream-ordered caching allocator: the replacement for ForgeChunk
 * (Memory/forge.cuh:30-90, forge.cu:13-122), the device branch of
 * TensorStorage (Storage/storage.cpp:20-35).  Requests round up to a size
 * class (powers of two from 512 B to 1 MiB, then multiples of 2 MiB).  A
 * block belongs to the stream it was allocated on: freeing it returns it to
 * that stream's cache, and only later allocations on the same stream reuse
 * it, so the stream order makes reuse safe without host synchronisation.
 * A block used on another stream needs the caller's synchronisation before
 * it is freed.  When the device is out of memory the cache is returned to
 * the device (after a device sync) and the allocation retried once.
 * cxm_pool_free of a pointer the pool did not return is CXM_E_INVALID. */
typedef struct cxm_pool_stats_t {
    size_t bytes_in_use;   /* size classes of live blocks */
    size_t bytes_cached;   /* size classes of freed blocks held for reuse */
    size_t peak_in_use;
    uint64_t allocs;       /* successful allocations */
    uint64_t hits;         /* of which served from the cache */
    uint64_t frees;
    uint64_t device_allocs;  /* allocations that called hipMalloc */
} cxm_pool_stats_t;
int cxm_pool_alloc(void **ptr, size_t bytes, cxm_stream_t s);
int cxm_pool_free(void *ptr);
/* Returns all cached blocks to the device (waits for the device first). */
int cxm_pool_release(void);
int cxm_pool_stats(cxm_pool_stats_t *stats);

/* ------------------------------------------------------------ reductions
 * avx2::reduce (Engine/AVX2/reduce.hpp:49-296, reduce.cpp:17-84,204-251,
 * 439-528).  The flat form reduces N elements to z[0]; the axis form treats
 * x as row-major [outer, dim, inner] and writes z[outer, inner].
 * Semantics kept from the reference:
 *   max, flat form and inner == 1: starts from -FLT_MAX (reduce.cpp:206),
 *       so an all -inf row gives -FLT_MAX; inner > 1 starts from slice 0;
 *   argmax: index (int32) of the first maximum, 0 for an all-equal slice;
 *   mean, flat: sum / (float)N; axis: the first floor(outer*inner/8)*8
 *       outputs are sum * rn(1/dim), the rest sum / (float)dim (reduce.cpp:77-83).
 * Sums are deterministic (fixed tree order) and differ from the reference's
 * 8-lane sequential order only in rounding.
 * NaN and signed zeros (max, min, argmax, argmin, all forms):
 *   max / min are IEEE 754-2019 maximum / minimum: the result is a quiet NaN
 *       when any element is NaN, and a +0/-0 tie gives +0 (max) / -0 (min).
 *       The reference's _mm256_max_ps / _mm256_min_ps fold (functions.hpp:
 *       314-325) returns the later operand on a NaN or a tie, so its result
 *       then depends on where the NaN or the zeros sit in its 8-lane order;
 *       without NaN and +0/-0 ties the two are the same bit for bit.
 *   argmax / argmin: NaN elements are skipped (no comparison selects them),
 *       except a NaN first element of the row, column or flat array, which
 *       gives index 0 -- the reference starts from that element and takes
 *       only strictly greater (smaller) values after it (reduce.cpp:442-455,
 *       483-521, 530-621); +0 and -0 compare equal, so the first of them wins.  This
 *       is the reference's axis form exactly; its flat form agrees except
 *       where a NaN inside an 8-element block makes it read the element 32
 *       places on (horizontal.hpp:154-159: countr_zero of an empty mask). */
int cxm_reduce_sum_flat_f32(const float *x, float *z, size_t n, cxm_stream_t s);
int cxm_reduce_mean_flat_f32(const float *x, float *z, size_t n, cxm_stream_t s);
int cxm_reduce_max_flat_f32(const float *x, float *z, size_t n, cxm_stream_t s);
int cxm_reduce_argmax_flat_f32(const float *x, int32_t *z, size_t n, cxm_stream_t s);
int cxm_reduce_sum_f32(const float *x, float *z, size_t outer, size_t dim, size_t inner,
                       cxm_stream_t s);
int cxm_reduce_mean_f32(const float *x, float *z, size_t outer, size_t dim, size_t inner,
                        cxm_stream_t s);
int cxm_reduce_max_f32(const float *x, float *z, size_t outer, size_t dim, size_t inner,
                       cxm_stream_t s);
int cxm_reduce_argmax_f32(const float *x, int32_t *z, size_t outer, size_t dim, size_t inner,
                          cxm_stream_t s);
/* cxm_reduce_sum_f32 for callers that cannot allocate device memory (code
 * under HIP graph capture, serving loops, harnesses that forbid hipMalloc).
 * No counterpart in the reference.  Same arguments, kernels and bits as
 * cxm_reduce_sum_f32 (the flat sum is (1, n, 1)); its partial sums, ticket
 * counters and tagged slots live in a static region per device (1 MiB of
 * counters, 16 KiB of slots, 1 MiB of partials) instead of the per-stream
 * workspace, and it calls no hipMalloc or hipFree.  That region covers every
 * shape the reduction plan produces; a shape needing more gives
 * CXM_E_TOO_LARGE.  The first call on a device looks the region up and
 * clears its counters and slots with a kernel on stream s.  All calls on one device share the region: two calls
 * that overlap in time on one device (different streams, or host threads)
 * race and must be serialised by the caller. */
int cxm_reduce_sum_noalloc_f32(const float *x, float *z, size_t outer, size_t dim, size_t inner,
                               cxm_stream_t s);
/* The rest of avx2::reduce (Engine/AVX2/reduce.hpp:96-329), same two forms:
 *  - min (reduce.cpp:253-309): smallest value; the flat and row forms start
 *    from FLT_MAX (an all-+inf input gives FLT_MAX), the column form from
 *    the first slice.  Exact.
 *  - argmin (reduce.cpp:530-621): int32 index of the first minimum.  Exact.
 *  - norm1 (reduce.cpp:311-367): sum of |x|.
 *  - norm2 (reduce.cpp:369-437): sqrt of the sum of x*x (products unrounded,
 *    as fma::add).
 *  - var (reduce.cpp:86-183): population variance, sum((x - mean)^2) / dim;
 *    flat and row results divide by the count, column results multiply by
 *    1/dim except the last total % 8 outputs, which divide (reduce.cpp:
 *    173-182).  One pass over x, where the reference reads it twice: the
 *    device sums d and d*d in fp64 with d = x - (first element of the row
 *    or column), so there is no cancellation between large sums.
 *  - stdv (reduce.cpp:185-202): sqrt(var).
 * Sums, norms and variances are within 1e-5 relative of the exact value for
 * the data sizes of the reference workloads.  n == 0 gives what the
 * reference's loops give (min FLT_MAX, norms 0, var/stdv NaN); argmin of
 * zero elements is CXM_E_INVALID. */
int cxm_reduce_min_flat_f32(const float *x, float *z, size_t n, cxm_stream_t s);
int cxm_reduce_argmin_flat_f32(const float *x, int32_t *z, size_t n, cxm_stream_t s);
int cxm_reduce_norm1_flat_f32(const float *x, float *z, size_t n, cxm_stream_t s);
int cxm_reduce_norm2_flat_f32(const float *x, float *z, size_t n, cxm_stream_t s);
int cxm_reduce_var_flat_f32(const float *x, float *z, size_t n, cxm_stream_t s);
int cxm_reduce_stdv_flat_f32(const float *x, float *z, size_t n, cxm_stream_t s);
int cxm_reduce_min_f32(const float *x, float *z, size_t outer, size_t dim, size_t inner,
                       cxm_stream_t s);
int cxm_reduce_argmin_f32(const float *x, int32_t *z, size_t outer, size_t dim, size_t inner,
                          cxm_stream_t s);
int cxm_reduce_norm1_f32(const float *x, float *z, size_t outer, size_t dim, size_t inner,
                         cxm_stream_t s);
int cxm_reduce_norm2_f32(const float *x, float *z, size_t outer, size_t dim, size_t inner,
                         cxm_stream_t s);
int cxm_reduce_var_f32(const float *x, float *z, size_t outer, size_t dim, size_t inner,
                       cxm_stream_t s);
int cxm_reduce_stdv_f32(const float *x, float *z, size_t outer, size_t dim, size_t inner,
                        cxm_stream_t s);

/* ------------------------------------------------------------ elementwise
 * Same-shape binary z = x op y: matrix_t::{add,sub,mul,div,max,min}
 * (Engine/AVX2/matrix.hpp:38-94) and nv::Matrix (Engine/CUDA/matrix.cuh:12-25).
 * z may alias x (the in-place forms, matrix.hpp:130-160).  max/min are
 * (x > y ? x : y) / (x < y ? x : y), as _mm256_max_ps / _mm256_min_ps.
 * CXM_OP_POW is powf(x, y): nv::ElementWise::pow(Xx, Xy, Xz)
 * (Engine/CUDA/element_wise.cu:39-49; ops::Power, Operations/kernel_ops.cuh:88-100). */
int cxm_binary_f32(const float *x, const float *y, float *z, size_t n, int op, cxm_stream_t s);
/* Row broadcast z[i,j] = x[i,j] op y[j] over [m, n]: Broadcast::row
 * (Engine/AVX2/broadcast.hpp:28-37).  Column broadcast z[i,j] = x[i,j] op y[i]:
 * Broadcast::col (broadcast.hpp:47-56).  z may alias x.  op in ADD..DIV. */
int cxm_bcast_row_f32(const float *x, const float *y, float *z, size_t m, size_t n, int op,
                      cxm_stream_t s);
int cxm_bcast_col_f32(const float *x, const float *y, float *z, size_t m, size_t n, int op,
                      cxm_stream_t s);
/* Tensor-op-scalar z = x op value: ScalarOp (Engine/AVX2/scalar.cpp:89-119),
 * nv::ScalarKernel (Engine/CUDA/scalar.cu:16-134).  z may alias x.
 * CXM_OP_POW is powf(x, value): nv::ElementWise::pow(Xx, value, Xz)
 * (Engine/CUDA/element_wise.cu:28-37) and avx2::wise::pow (Engine/AVX2/wise.cpp:60-91). */
int cxm_scalar_f32(const float *x, float value, float *z, size_t n, int op, cxm_stream_t s);
/* z = act(x) for act in RELU, SIGMOID, TANH, EXP (Engine/AVX2/functions.hpp:
 * 372-374, 405-411, 381-383, 186-188; nv::ElementWise::exp,
 * Engine/CUDA/element_wise.cu:84-93).  relu(x) = (0 > x) ? 0 : x. */
int cxm_unary_f32(const float *x, float *z, size_t n, int act, cxm_stream_t s);
/* z = fn(x) for fn in CXM_FN_*: nv::ElementWise::{square, sqrt, rsqrt, log,
 * exp, erf, sin, cos, abs, neg, rcp, inverse, sign} (Engine/CUDA/element_wise.cu:
 * 17-181; ops in Operations/kernel_ops.cuh:73-284) and avx2::wise
 * (Engine/AVX2/wise.cpp:56-143).  z may alias x.  Results: square, abs, neg,
 * sign exact; sqrt, rcp (= inverse = 1/x) correctly rounded; rsqrt, log, exp,
 * erf, sin, cos within 2 ulp of the exact value.  sign(x) = (x > 0) - (x < 0),
 * so sign(NaN) = sign(-0) = +0. */
int cxm_wise_f32(const float *x, float *z, size_t n, int fn, cxm_stream_t s);
/* z = fma(v2, v1 - x, x), i.e. x + v2*(v1 - x) with the product and the sum
 * rounded once: avx2::wise::lerp (Engine/AVX2/wise.cpp:145-155,
 * functions.hpp:271-274). */
int cxm_lerp_f32(const float *x, float v1, float v2, float *z, size_t n, cxm_stream_t s);
/* z = min(max(x, lo), hi) with _mm256_max_ps / _mm256_min_ps operand rules:
 * avx2::wise::clamp (Engine/AVX2/wise.cpp:157-167, functions.hpp:332-335).
 * A NaN x gives lo. */
int cxm_clamp_f32(const float *x, float lo, float hi, float *z, size_t n, cxm_stream_t s);
/* z[i] = x[idx[i]] for i < n: avx2::wise::gather (Engine/AVX2/wise.cpp:169-194).
 * x holds x_n elements; an index outside [0, x_n) yields NaN (f32) or
 * INT32_MIN (i32) instead of reading out of bounds. */
int cxm_gather_f32(const float *x, size_t x_n, const int32_t *idx, float *z, size_t n,
                   cxm_stream_t s);
int cxm_gather_i32(const int32_t *x, size_t x_n, const int32_t *idx, int32_t *z, size_t n,
                   cxm_stream_t s);

/* ---------------------------------------------------- 16-bit element types
 * convert() (Tools/cast.cpp:7-90): dst[i] = src[i] between CXM_DT_F32,
 * CXM_DT_BF16 and CXM_DT_F16.  bf16 -> f32 and f16 -> f32 are exact;
 * f32 -> bf16 rounds to nearest-even (cast.cpp:55-68's bias formula; NaN
 * stays a quiet NaN); f32 -> f16 is the IEEE round-to-nearest-even
 * conversion (_mm256_cvtps_ph).  16-bit data are arrays of uint16. */
int cxm_convert(void *dst, int dst_dtype, const void *src, int src_dtype, size_t n, cxm_stream_t s);
/* The elementwise surface for any CXM_DT_*: binary (ops ADD..POW), scalar,
 * activation (RELU..EXP) and math (CXM_FN_*).  CXM_DT_F32 runs the *_f32
 * entry points above.  bf16/f16 (the reference's CPU kernel_t, wise.cpp:
 * 17-52, and its CUDA __nv_bfloat162 / __half2 kernels, Kernels/unary.cuh:
 * 42-90, binary.cuh:41-89, scalar.cuh:69-130): each element is widened to
 * fp32, the fp32 operator applied, and the result rounded once to nearest-
 * even, which is the correctly rounded 16-bit result for + - * / and sqrt.
 * A scalar operand is first rounded to the 16-bit type, as the CUDA path
 * passes it. */
int cxm_binary_t(const void *x, const void *y, void *z, size_t n, int op, int dtype, cxm_stream_t s);
int cxm_scalar_t(const void *x, float value, void *z, size_t n, int op, int dtype, cxm_stream_t s);
int cxm_unary_t(const void *x, void *z, size_t n, int act, int dtype, cxm_stream_t s);
int cxm_wise_t(const void *x, void *z, size_t n, int fn, int dtype, cxm_stream_t s);

/* Fused y = act(x * scale[j] + bias[j]) over [m, n]: Broadcast::row::mul then
 * Broadcast::row::add in place (broadcast.cpp:206-216, 230-240), then the
 * activation; the product and the sum are rounded separately (no fma). */
int cxm_affine_act_fwd_f32(const float *x, const float *scale, const float *bias, float *y,
                           size_t m, size_t n, int act, cxm_stream_t s);
/* Backward of the above from the saved output y: g = act'(y) (relu: y > 0,
 * sigmoid: y*(1-y), tanh: 1-y*y), dz = dy*g, dx = dz*scale[j],
 * dscale[j] = sum_i dz*x, dbias[j] = sum_i dz.  No reference counterpart
 * (the reference has no backward); composed of matrix_t::mul,
 * Broadcast::row::mul and reduce::sum over axis 0. */
int cxm_affine_act_bwd_f32(const float *x, const float *scale, const float *y, const float *dy,
                           float *dx, float *dscale, float *dbias, size_t m, size_t n, int act,
                           cxm_stream_t s);

/* --------------------------------------------------------------- softmax
 * Row softmax (log_mode = 0) or log-softmax (log_mode = 1) over the last axis
 * of [rows, cols].  The reference has none; it is the composition
 * m = reduce::max (reduce.cpp:204-215), z = Broadcast::col::sub(x, m),
 * e = exp(z), s = reduce::sum(e), y = Broadcast::col::div(e, s) or z - log(s).
 * -inf entries give exactly 0 (softmax) and -inf (log-softmax).
 * y may be x itself (in place); an output that overlaps an input in any
 * other way is CXM_E_INVALID.  The same holds for dx against y and dy in
 * the backward. */
int cxm_softmax_fwd_f32(const float *x, float *y, size_t rows, size_t cols, int log_mode,
                        cxm_stream_t s);
/* Backward from the saved output y: softmax dx = y*(dy - sum(dy*y));
 * log-softmax dx = dy - exp(y)*sum(dy). */
int cxm_softmax_bwd_f32(const float *y, const float *dy, float *dx, size_t rows, size_t cols,
                        int log_mode, cxm_stream_t s);
/* Kernels whose workgroups exchange partial results through device memory
 * -- the one-pass softmax of rows of 4097..524288 columns (up to 8192
 * rows), and the flat sum / mean / max / min / norm1 / norm2 over more than
 * 1024 elements -- let a workgroup wait at most `polls` polls (default
 * 65536) for a peer's partial before it computes that partial from the
 * input itself.  Either way the result is the same bit
 * for bit; 0 makes every waiting workgroup compute (for tests of that
 * path).  Process-wide; *previous (if not NULL) gets the old value.  No
 * reference counterpart. */
int cxm_exchange_wait_limit(unsigned polls, unsigned *previous);
/* Row-group stagger of the single-pass long-row softmax forward,
 * process-wide: the last of up to 16 row groups starts about pct% (0..100,
 * default 65) of the input's streaming time after the first; 0 starts every
 * workgroup at once.  Results do not depend on it.  The previous value goes
 * to *previous when not NULL.  For tests and tuning; no reference
 * counterpart. */
int cxm_softmax_stagger(int pct, int *previous);

/* ---------------------------------------------------------------- matmul
 * Row-major C[xN, zN] = A[xN, yN] * B[yN, zN]: matrix_t::matmul
 * (Engine/AVX2/matrix.hpp:119, matrix.cpp:75-147) and nv::Matrix::matmul
 * (Engine/CUDA/matrix.cu:112-159, which uses TF32; this one is true fp32 on
 * v_mfma_f32_32x32x2_f32). */
int cxm_matmul_f32(const float *a, const float *b, float *c, size_t xN, size_t yN, size_t zN,
                   cxm_stream_t s);
/* General form: C[m,n] = op(A)[m,k] * op(B)[k,n], then the epilogue.
 * A is stored [m,k] ([k,m] when trans_a), B is [k,n] ([n,k] when trans_b).
 * bias (length n, or NULL) is added to every row; act is NONE or RELU;
 * gate (an [m,n] array, or NULL) multiplies the result by (gate > 0 ? 1 : 0),
 * which is the ReLU backward from the saved activation.  No reference
 * counterpart for the transposed and fused forms (matrix.cpp has only NN). */
int cxm_gemm_f32(const float *a, const float *b, float *c, size_t m, size_t k, size_t n,
                 int trans_a, int trans_b, const float *bias, int act, const float *gate,
                 cxm_stream_t s);
/* Kernel choice of the fp32 GEMM, process-wide: -1 automatic (default),
 * 0..6 the register-staged variants, 7 the four-stage direct-to-LDS ring
 * (M, N, K multiples of 128 and 16-byte aligned bases, else variant 1).
 * Results agree within the fp32 tolerance; the ring and variant 1 sum each
 * output over k in the same order and give the same bits for A B and
 * A B^T.  For tests and tuning; no reference counterpart. */
int cxm_gemm_f32_kernel(int variant);
/* matmul for any CXM_DT_*: nv::Matrix::matmul (Engine/CUDA/matrix.cu:112-159)
 * with its per-dtype cublasGemmEx (BlasTraits, matrix.cu:18-37).  bf16 and
 * fp16 operands and output (16-bit element arrays), fp32 accumulation on
 * v_mfma_f32_32x32x16_{bf16,f16}, one round-to-nearest-even at the end (the
 * reference's fp16 form accumulates in fp16).  CXM_DT_F32 runs cxm_matmul_f32.
 * cxm_gemm_t adds the transposed forms of cxm_gemm_f32 (no epilogue). */
int cxm_matmul_t(const void *a, const void *b, void *c, size_t xN, size_t yN, size_t zN, int dtype,
                 cxm_stream_t s);
int cxm_gemm_t(const void *a, const void *b, void *c, size_t m, size_t k, size_t n, int trans_a,
               int trans_b, int dtype, cxm_stream_t s);
/* Kernel choice of the 16-bit GEMM, process-wide: -1 automatic (default),
 * 0 the 128x128-tile register-staged kernel, 1 the 256x256-tile one, 2 the
 * 256x256 four-stage direct-to-LDS kernel, 3 the 128x128 one; 2 and 3 need
 * M, N multiples of their tile, K of 128 and 16-byte aligned bases, else
 * 1 and 0 run.  All give the same bits.  For tests and tuning; no
 * reference counterpart. */
int cxm_gemm16_kernel(int kernel);

/* ----------------------------------------------------------- training step
 * Softmax cross-entropy on logits [b, c] with int32 labels in [0, c):
 * loss[0] = mean_r(-log_softmax(logits)[r, label_r]) and
 * dlogits = (softmax(logits) - onehot) / b.  No reference counterpart. */
int cxm_softmax_xent_f32(const float *logits, const int32_t *labels, float *loss, float *dlogits,
                         size_t b, size_t c, cxm_stream_t s);
/* dx = dy * act'(y) from the saved output y, act in RELU, SIGMOID, TANH:
 * relu' = (y > 0 ? 1 : 0), sigmoid' = y*(1-y), tanh' = 1 - y*y, each factor
 * rounded, then one product.  dx may alias dy.  No reference counterpart:
 * the backward of avx2::relu/sigmoid/tanh (functions.hpp:372-411) that a
 * concrete GradientFlow would run. */
int cxm_act_bwd_f32(const float *y, const float *dy, float *dx, size_t n, int act, cxm_stream_t s);
/* Backward of reduce::sum / reduce::mean over the middle axis of [outer,
 * dim, inner]: dx[o, d, i] = dz[o, i] (sum, mean = 0) or dz[o, i] / dim
 * (mean = 1, the correctly rounded quotient).  dz holds outer * inner
 * elements; dx must not overlap it.  No reference counterpart: the
 * backward a Sum / Mean GradientFlow (Graph/flow.hpp:15-24) runs. */
int cxm_reduce_sum_bwd_f32(const float *dz, float *dx, size_t outer, size_t dim, size_t inner, int mean,
                           cxm_stream_t s);
/* w -= lr * g, as matrix_t::sub(w, ScalarOp::mul(g, lr)): two roundings. */
int cxm_sgd_f32(float *w, const float *g, float lr, size_t n, cxm_stream_t s);

/* ------------------------------------------------------------- MLP step
 * One SGD training step of a 3-layer ReLU MLP, d0 -> d1 -> d2 -> d3, on a
 * batch of `batch` rows: forward, softmax cross-entropy on int32 labels,
 * reverse-mode backward, then W -= lr*gW and b -= lr*gb for all six
 * parameters (weights stored [fan_in, fan_out], row-major).  No reference
 * counterpart: the reference's autograd has only the abstract
 * meta::GradientFlow::backward (Graph/flow.hpp:15-24) and no layers, loss or
 * optimizer; this is the step its concrete flows would perform.
 * The handle owns the activations and gradients (allocated once). */
typedef struct cxm_mlp3 cxm_mlp3;
int cxm_mlp3_create(cxm_mlp3 **handle, size_t batch, size_t d0, size_t d1, size_t d2, size_t d3);
int cxm_mlp3_step_f32(cxm_mlp3 *handle, const float *x, const int32_t *labels, float *w1, float *b1,
                      float *w2, float *b2, float *w3, float *b3, float lr, float *loss,
                      cxm_stream_t s);
int cxm_mlp3_destroy(cxm_mlp3 *handle);
/* Diagnostics, no reference counterpart: how many workgroups of the last
 * step's paired weight-gradient launch ran the output layer's finish and
 * the layer-1 bias step on the CUs the products left free (0: they ran as
 * kernels of their own). */
int cxm_mlp3_last_side(const cxm_mlp3 *handle, unsigned *wgs);

#ifdef __cplusplus
}
#endif

#endif /* CXM_HIP_H */
