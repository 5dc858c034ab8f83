/*
 * cxm_oracle.c -- CPU restatement of the CortexMind AVX2 hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * backend in cortexmind_amd/.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it.  The product path never calls it
 * and has no CPU fallback.
 *
 * Every function restates, in plain C, the loop order of the reference
 * function it cites (paths relative to source/CortexMind/framework/ in the
 * reference tree).  The 8-wide AVX2 registers become arrays of 8 floats; the
 * fold orders of horizontal.hpp are spelled out so that results are bit-exact
 * with the reference's own arithmetic.  Build with -ffp-contract=off so that
 * a*b+c stays two roundings wherever the reference uses separate mul/add, and
 * fmaf() appears exactly where the reference uses fma::add.
 *
 * Parts of the path that the reference lacks (softmax, log-softmax, their
 * backward, the affine+activation backward, softmax cross-entropy, SGD and the
 * MLP step) are defined here as compositions of the reference primitives;
 * each composition names the primitives it chains.
 *
 * Deviations from the reference, on purpose:
 *  - Broadcast::row::div uses division (the reference's SIMD body multiplies,
 *    Engine/AVX2/broadcast.cpp:222, a defect).
 *  - exp/tanh: the reference calls Intel SVML (_mm256_exp_ps/_mm256_tanh_ps,
 *    Engine/AVX2/functions.hpp:186-188,381-383), which no compiler here ships.
 *    The oracle calls glibc expf/tanhf/logf; the pass criterion for these is an
 *    error bound against float64, not bit equality.
 *  - argmax over a block whose horizontal max is NaN: the reference takes
 *    countr_zero(0)=32 and reads past the block (horizontal.hpp:154-159).  The
 *    oracle skips such a block.  NaN inputs are outside the parity contract.
 */
#include <float.h>
#include <immintrin.h>
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define L8 8

/* _mm_max_ps / _mm256_max_ps(a, b): returns a when a > b, else b. */
static inline float simd_max(float a, float b) { return a > b ? a : b; }
/* std::max(a, b): returns b when a < b, else a. */
static inline float std_max(float a, float b) { return a < b ? b : a; }

/* horizontal::sum (Engine/AVX2/horizontal.hpp:30-37): hi+lo, hadd, hadd. */
static float fold_sum8(const float a[L8]) {
    const float s0 = a[4] + a[0], s1 = a[5] + a[1];
    const float s2 = a[6] + a[2], s3 = a[7] + a[3];
    return (s0 + s1) + (s2 + s3);
}

/* horizontal::max (horizontal.hpp:63-70): max(lo,hi), movehl, shuffle 1. */
static float fold_max8(const float a[L8]) {
    const float m0 = simd_max(a[0], a[4]), m1 = simd_max(a[1], a[5]);
    const float m2 = simd_max(a[2], a[6]), m3 = simd_max(a[3], a[7]);
    const float n0 = simd_max(m0, m2), n1 = simd_max(m1, m3);
    return simd_max(n0, n1);
}

/* _mm_min_ps / _mm256_min_ps(a, b): returns a when a < b, else b. */
static inline float simd_min(float a, float b) { return a < b ? a : b; }
/* std::min(a, b): returns b when b < a, else a. */
static inline float std_min(float a, float b) { return b < a ? b : a; }

/* horizontal::min (horizontal.hpp:95-102): min(lo,hi), movehl, shuffle 1. */
static float fold_min8(const float a[L8]) {
    const float m0 = simd_min(a[0], a[4]), m1 = simd_min(a[1], a[5]);
    const float m2 = simd_min(a[2], a[6]), m3 = simd_min(a[3], a[7]);
    const float n0 = simd_min(m0, m2), n1 = simd_min(m1, m3);
    return simd_min(n0, n1);
}

/* horizontal::argmin (horizontal.hpp:171-176): first lane equal to the min. */
static int fold_argmin8(const float a[L8]) {
    const float m = fold_min8(a);
    for (int l = 0; l < L8; ++l)
        if (a[l] == m) return l;
    return -1;
}

/* horizontal::argmax (horizontal.hpp:154-159): first lane equal to the max. */
static int fold_argmax8(const float a[L8]) {
    const float m = fold_max8(a);
    for (int l = 0; l < L8; ++l)
        if (a[l] == m) return l;
    return -1;
}

/* ------------------------------------------------------------------ sum */

/* reduce::sum flat (Engine/AVX2/reduce.cpp:17-28). */
void orc_reduce_sum_flat(const float *x, float *z, size_t n) {
    float acc[L8] = {0, 0, 0, 0, 0, 0, 0, 0};
    size_t i = 0;
    for (; i + L8 <= n; i += L8)
        for (int l = 0; l < L8; ++l) acc[l] = acc[l] + x[i + l];
    float r = fold_sum8(acc);
    for (; i < n; ++i) r += x[i];
    z[0] = r;
}

/* reduce::sum axis (reduce.cpp:30-64): inner==1 -> flat sum per row;
 * otherwise copy slice 0 and add slices 1..dim-1 in order. */
void orc_reduce_sum(const float *x, float *z, size_t outer, size_t dim, size_t inner) {
    if (inner == 1) {
        for (size_t o = 0; o < outer; ++o) orc_reduce_sum_flat(x + o * dim, z + o, dim);
        return;
    }
    for (size_t o = 0; o < outer; ++o) {
        float *dst = z + o * inner;
        const float *src = x + o * dim * inner;
        memcpy(dst, src, inner * sizeof(float));
        for (size_t d = 1; d < dim; ++d) {
            const float *row = src + d * inner;
            for (size_t j = 0; j < inner; ++j) dst[j] = dst[j] + row[j];
        }
    }
}

/* ----------------------------------------------------------------- mean */

/* reduce::mean flat (reduce.cpp:66-69): sum, then true division by N. */
void orc_reduce_mean_flat(const float *x, float *z, size_t n) {
    orc_reduce_sum_flat(x, z, n);
    z[0] = z[0] / (float)n;
}

/* reduce::mean axis (reduce.cpp:71-84): the first floor(total/8)*8 outputs
 * are multiplied by the rounded reciprocal 1/dim, the rest are divided. */
void orc_reduce_mean(const float *x, float *z, size_t outer, size_t dim, size_t inner) {
    orc_reduce_sum(x, z, outer, dim, inner);
    const size_t total = outer * inner;
    const size_t body = total - total % L8;
    const float scale = 1.0f / (float)dim;
    size_t i = 0;
    for (; i < body; ++i) z[i] = z[i] * scale;
    for (; i < total; ++i) z[i] = z[i] / (float)dim;
}

/* ------------------------------------------------------------------ max */

/* reduce::max flat (reduce.cpp:204-215): lanes start at -FLT_MAX. */
void orc_reduce_max_flat(const float *x, float *z, size_t n) {
    float acc[L8];
    for (int l = 0; l < L8; ++l) acc[l] = -FLT_MAX;
    size_t i = 0;
    for (; i + L8 <= n; i += L8)
        for (int l = 0; l < L8; ++l) acc[l] = simd_max(acc[l], x[i + l]);
    float r = fold_max8(acc);
    for (; i < n; ++i) r = std_max(r, x[i]);
    z[0] = r;
}

/* reduce::max axis (reduce.cpp:217-251): inner==1 -> flat per row; otherwise
 * start from slice 0 (so an all -inf column yields -inf, not -FLT_MAX). */
void orc_reduce_max(const float *x, float *z, size_t outer, size_t dim, size_t inner) {
    if (inner == 1) {
        for (size_t o = 0; o < outer; ++o) orc_reduce_max_flat(x + o * dim, z + o, dim);
        return;
    }
    const size_t body = inner - inner % L8;
    for (size_t o = 0; o < outer; ++o) {
        float *dst = z + o * inner;
        const float *src = x + o * dim * inner;
        memcpy(dst, src, inner * sizeof(float));
        for (size_t d = 1; d < dim; ++d) {
            const float *row = src + d * inner;
            size_t j = 0;
            for (; j < body; ++j) dst[j] = simd_max(dst[j], row[j]);
            for (; j < inner; ++j) dst[j] = std_max(dst[j], row[j]);
        }
    }
}

/* --------------------------------------------------------------- argmax */

/* reduce::argmax flat (reduce.cpp:439-466): per 8-block lane argmax, then a
 * strict '>' against the running best; tail elements with strict '>'. */
void orc_reduce_argmax_flat(const float *x, int32_t *z, size_t n) {
    size_t i = 0;
    float best = x[0];
    int32_t best_i = 0;
    for (; i + L8 <= n; i += L8) {
        const int lane = fold_argmax8(x + i);
        if (lane < 0) continue;
        const float cand = x[i + lane];
        if (cand > best) {
            best = cand;
            best_i = (int32_t)(i + lane);
        }
    }
    for (; i < n; ++i) {
        if (x[i] > best) {
            best = x[i];
            best_i = (int32_t)i;
        }
    }
    z[0] = best_i;
}

/* reduce::argmax axis (reduce.cpp:468-528): inner==1 -> flat per row;
 * otherwise a running (value, index) per column, replaced on strict '>'. */
void orc_reduce_argmax(const float *x, int32_t *z, size_t outer, size_t dim, size_t inner) {
    if (inner == 1) {
        for (size_t o = 0; o < outer; ++o) orc_reduce_argmax_flat(x + o * dim, z + o, dim);
        return;
    }
    float *best = (float *)malloc(inner * sizeof(float));
    for (size_t o = 0; o < outer; ++o) {
        const float *src = x + o * dim * inner;
        int32_t *dst = z + o * inner;
        for (size_t j = 0; j < inner; ++j) {
            best[j] = src[j];
            dst[j] = 0;
        }
        for (size_t d = 1; d < dim; ++d) {
            const float *row = src + d * inner;
            for (size_t j = 0; j < inner; ++j) {
                if (row[j] > best[j]) {
                    best[j] = row[j];
                    dst[j] = (int32_t)d;
                }
            }
        }
    }
    free(best);
}

/* ------------------------------------------------------------------ min */

/* reduce::min flat (reduce.cpp:253-264): lanes start at FLT_MAX. */
void orc_reduce_min_flat(const float *x, float *z, size_t n) {
    float acc[L8];
    for (int l = 0; l < L8; ++l) acc[l] = FLT_MAX;
    size_t i = 0;
    for (; i + L8 <= n; i += L8)
        for (int l = 0; l < L8; ++l) acc[l] = simd_min(acc[l], x[i + l]);
    float r = fold_min8(acc);
    for (; i < n; ++i) r = std_min(r, x[i]);
    z[0] = r;
}

/* reduce::min axis (reduce.cpp:266-309): inner==1 -> the flat loop per row;
 * otherwise start from slice 0 and fold slices 1..dim-1 with
 * _mm256_min_ps(out, in) (body) / std::min(out, in) (tail). */
void orc_reduce_min(const float *x, float *z, size_t outer, size_t dim, size_t inner) {
    if (inner == 1) {
        for (size_t o = 0; o < outer; ++o) orc_reduce_min_flat(x + o * dim, z + o, dim);
        return;
    }
    const size_t body = inner - inner % L8;
    for (size_t o = 0; o < outer; ++o) {
        float *dst = z + o * inner;
        const float *src = x + o * dim * inner;
        memcpy(dst, src, inner * sizeof(float));
        for (size_t d = 1; d < dim; ++d) {
            const float *row = src + d * inner;
            size_t j = 0;
            for (; j < body; ++j) dst[j] = simd_min(dst[j], row[j]);
            for (; j < inner; ++j) dst[j] = std_min(dst[j], row[j]);
        }
    }
}

/* --------------------------------------------------------------- argmin */

/* reduce::argmin flat (reduce.cpp:530-557): per 8-block lane argmin, then a
 * strict '<' against the running best (starting at x[0], index 0). */
void orc_reduce_argmin_flat(const float *x, int32_t *z, size_t n) {
    size_t i = 0;
    float best = x[0];
    int32_t best_i = 0;
    for (; i + L8 <= n; i += L8) {
        const int lane = fold_argmin8(x + i);
        if (lane < 0) continue;
        const float cand = x[i + lane];
        if (cand < best) {
            best = cand;
            best_i = (int32_t)(i + lane);
        }
    }
    for (; i < n; ++i) {
        if (x[i] < best) {
            best = x[i];
            best_i = (int32_t)i;
        }
    }
    z[0] = best_i;
}

/* reduce::argmin axis (reduce.cpp:559-621): inner==1 -> flat per row;
 * otherwise a running (value, index) per column, replaced on strict '<'. */
void orc_reduce_argmin(const float *x, int32_t *z, size_t outer, size_t dim, size_t inner) {
    if (inner == 1) {
        for (size_t o = 0; o < outer; ++o) orc_reduce_argmin_flat(x + o * dim, z + o, dim);
        return;
    }
    float *best = (float *)malloc(inner * sizeof(float));
    for (size_t o = 0; o < outer; ++o) {
        const float *src = x + o * dim * inner;
        int32_t *dst = z + o * inner;
        for (size_t j = 0; j < inner; ++j) {
            best[j] = src[j];
            dst[j] = 0;
        }
        for (size_t d = 1; d < dim; ++d) {
            const float *row = src + d * inner;
            for (size_t j = 0; j < inner; ++j) {
                if (row[j] < best[j]) {
                    best[j] = row[j];
                    dst[j] = (int32_t)d;
                }
            }
        }
    }
    free(best);
}

/* ---------------------------------------------------------------- norms */

/* reduce::norm1 flat (reduce.cpp:311-322): 8 lane sums of |x|, fold, tail. */
void orc_reduce_norm1_flat(const float *x, float *z, size_t n) {
    float acc[L8] = {0, 0, 0, 0, 0, 0, 0, 0};
    size_t i = 0;
    for (; i + L8 <= n; i += L8)
        for (int l = 0; l < L8; ++l) acc[l] = acc[l] + fabsf(x[i + l]);
    float r = fold_sum8(acc);
    for (; i < n; ++i) r += fabsf(x[i]);
    z[0] = r;
}

/* reduce::norm1 axis (reduce.cpp:324-367): inner==1 -> flat per row;
 * otherwise |slice 0|, then add |slice d| in order. */
void orc_reduce_norm1(const float *x, float *z, size_t outer, size_t dim, size_t inner) {
    if (inner == 1) {
        for (size_t o = 0; o < outer; ++o) orc_reduce_norm1_flat(x + o * dim, z + o, dim);
        return;
    }
    for (size_t o = 0; o < outer; ++o) {
        float *dst = z + o * inner;
        const float *src = x + o * dim * inner;
        for (size_t j = 0; j < inner; ++j) dst[j] = fabsf(src[j]);
        for (size_t d = 1; d < dim; ++d) {
            const float *row = src + d * inner;
            for (size_t j = 0; j < inner; ++j) dst[j] = dst[j] + fabsf(row[j]);
        }
    }
}

/* reduce::norm2 flat (reduce.cpp:369-381): lanes acc = fma(v, v, acc)
 * (fma::add), fold, tail adds the rounded square, then sqrt. */
void orc_reduce_norm2_flat(const float *x, float *z, size_t n) {
    float acc[L8] = {0, 0, 0, 0, 0, 0, 0, 0};
    size_t i = 0;
    for (; i + L8 <= n; i += L8)
        for (int l = 0; l < L8; ++l) acc[l] = fmaf(x[i + l], x[i + l], acc[l]);
    float r = fold_sum8(acc);
    for (; i < n; ++i) {
        const float sq = x[i] * x[i];
        r += sq;
    }
    z[0] = sqrtf(r);
}

/* reduce::norm2 axis (reduce.cpp:383-437): inner==1 -> flat per row;
 * otherwise slice 0 squared (mul), slices 1.. by fma in the 8-wide body and
 * rounded square + add in the tail, then sqrt of every output. */
void orc_reduce_norm2(const float *x, float *z, size_t outer, size_t dim, size_t inner) {
    if (inner == 1) {
        for (size_t o = 0; o < outer; ++o) orc_reduce_norm2_flat(x + o * dim, z + o, dim);
        return;
    }
    const size_t body = inner - inner % L8;
    for (size_t o = 0; o < outer; ++o) {
        float *dst = z + o * inner;
        const float *src = x + o * dim * inner;
        for (size_t j = 0; j < inner; ++j) dst[j] = src[j] * src[j];
        for (size_t d = 1; d < dim; ++d) {
            const float *row = src + d * inner;
            size_t j = 0;
            for (; j < body; ++j) dst[j] = fmaf(row[j], row[j], dst[j]);
            for (; j < inner; ++j) {
                const float sq = row[j] * row[j];
                dst[j] = dst[j] + sq;
            }
        }
    }
    for (size_t q = 0; q < outer * inner; ++q) z[q] = sqrtf(z[q]);
}

/* ------------------------------------------------------------ var, stdv */

/* reduce::var flat (reduce.cpp:86-104): mu = mean flat; lanes accumulate
 * fma(d, d, acc) with d = x - mu; fold; tail adds the rounded d*d; divide
 * by N. */
void orc_reduce_var_flat(const float *x, float *z, size_t n) {
    float mu;
    orc_reduce_mean_flat(x, &mu, n);
    float acc[L8] = {0, 0, 0, 0, 0, 0, 0, 0};
    size_t i = 0;
    for (; i + L8 <= n; i += L8)
        for (int l = 0; l < L8; ++l) {
            const float d = x[i + l] - mu;
            acc[l] = fmaf(d, d, acc[l]);
        }
    float r = fold_sum8(acc);
    for (; i < n; ++i) {
        const float d = x[i] - mu;
        const float sq = d * d;
        r += sq;
    }
    z[0] = r / (float)n;
}

/* reduce::var axis (reduce.cpp:106-183).  inner==1: per row, the flat sum
 * loop, mu = sum / dim (true division), the flat deviation loop, divide by
 * dim.  Otherwise: mu = mean axis; dst = (x0 - mu)^2 rounded; slices 1.. by
 * fma in the 8-wide body and rounded square + add in the tail; then the
 * first floor(total/8)*8 outputs multiply by 1/dim, the rest divide. */
void orc_reduce_var(const float *x, float *z, size_t outer, size_t dim, size_t inner) {
    if (inner == 1) {
        for (size_t o = 0; o < outer; ++o) {
            const float *src = x + o * dim;
            float s;
            orc_reduce_sum_flat(src, &s, dim);
            const float mu = s / (float)dim;
            float acc[L8] = {0, 0, 0, 0, 0, 0, 0, 0};
            size_t i = 0;
            for (; i + L8 <= dim; i += L8)
                for (int l = 0; l < L8; ++l) {
                    const float d = src[i + l] - mu;
                    acc[l] = fmaf(d, d, acc[l]);
                }
            float r = fold_sum8(acc);
            for (; i < dim; ++i) {
                const float d = src[i] - mu;
                const float sq = d * d;
                r += sq;
            }
            z[o] = r / (float)dim;
        }
        return;
    }
    const size_t total = outer * inner;
    float *mu = (float *)malloc(total * sizeof(float));
    orc_reduce_mean(x, mu, outer, dim, inner);
    const size_t body = inner - inner % L8;
    for (size_t o = 0; o < outer; ++o) {
        float *dst = z + o * inner;
        const float *src = x + o * dim * inner;
        const float *m = mu + o * inner;
        for (size_t j = 0; j < inner; ++j) {
            const float d = src[j] - m[j];
            dst[j] = d * d;
        }
        for (size_t dd = 1; dd < dim; ++dd) {
            const float *row = src + dd * inner;
            size_t j = 0;
            for (; j < body; ++j) {
                const float d = row[j] - m[j];
                dst[j] = fmaf(d, d, dst[j]);
            }
            for (; j < inner; ++j) {
                const float d = row[j] - m[j];
                const float sq = d * d;
                dst[j] = dst[j] + sq;
            }
        }
    }
    free(mu);
    const size_t tbody = total - total % L8;
    const float scale = 1.0f / (float)dim;
    size_t q = 0;
    for (; q < tbody; ++q) z[q] = z[q] * scale;
    for (; q < total; ++q) z[q] = z[q] / (float)dim;
}

/* reduce::stdv (reduce.cpp:185-202): sqrt of var, flat and axis. */
void orc_reduce_stdv_flat(const float *x, float *z, size_t n) {
    orc_reduce_var_flat(x, z, n);
    z[0] = sqrtf(z[0]);
}

void orc_reduce_stdv(const float *x, float *z, size_t outer, size_t dim, size_t inner) {
    orc_reduce_var(x, z, outer, dim, inner);
    for (size_t q = 0; q < outer * inner; ++q) z[q] = sqrtf(z[q]);
}

/* ---------------------------------------------------- elementwise binary */

enum { ORC_ADD = 0, ORC_SUB = 1, ORC_MUL = 2, ORC_DIV = 3, ORC_MAX = 4, ORC_MIN = 5, ORC_POW = 6 };

static inline float bin_op(int op, float a, float b) {
    switch (op) {
        case ORC_ADD: return a + b;
        case ORC_SUB: return a - b;
        case ORC_MUL: return a * b;
        case ORC_DIV: return a / b;
        case ORC_MAX: return simd_max(a, b);     /* _mm256_max_ps(x, y) */
        case ORC_MIN: return a < b ? a : b;      /* _mm256_min_ps(x, y) */
        default:      return powf(a, b);         /* ops::Power, Operations/kernel_ops.hpp:69-78 */
    }
}

/* matrix_t::{add,sub,mul,div,max,min} same shape (Engine/AVX2/matrix.cpp:15-73).
 * max/min follow the SIMD body; the scalar tail (tlx::max/min) is parity
 * unpinned because TLX is not available. */
void orc_binary(const float *x, const float *y, float *z, size_t n, int op) {
    for (size_t i = 0; i < n; ++i) z[i] = bin_op(op, x[i], y[i]);
}

/* Broadcast::row::op (Engine/AVX2/broadcast.cpp:182-276): z[i,j] = x[i,j] op y[j]. */
void orc_bcast_row(const float *x, const float *y, float *z, size_t m, size_t n, int op) {
    for (size_t i = 0; i < m; ++i)
        for (size_t j = 0; j < n; ++j) z[i * n + j] = bin_op(op, x[i * n + j], y[j]);
}

/* Broadcast::col::op (broadcast.cpp:278-388): z[i,j] = x[i,j] op y[i]. */
void orc_bcast_col(const float *x, const float *y, float *z, size_t m, size_t n, int op) {
    for (size_t i = 0; i < m; ++i) {
        const float v = y[i];
        for (size_t j = 0; j < n; ++j) z[i * n + j] = bin_op(op, x[i * n + j], v);
    }
}

/* ScalarOp::op (Engine/AVX2/scalar.cpp:89-119): z = x op value.  The
 * reference's scalar tail steps by 8 (Engine/Kernels/scalar.hpp:24); the
 * oracle applies the op to every element, the documented intent. */
void orc_scalar(const float *x, float value, float *z, size_t n, int op) {
    for (size_t i = 0; i < n; ++i) z[i] = bin_op(op, x[i], value);
}

/* ------------------------------------------------------ elementwise math */

enum {
    ORC_FN_SQUARE = 0, ORC_FN_SQRT, ORC_FN_RSQRT, ORC_FN_LOG, ORC_FN_EXP, ORC_FN_ERF, ORC_FN_SIN,
    ORC_FN_COS, ORC_FN_ABS, ORC_FN_NEG, ORC_FN_RCP, ORC_FN_INVERSE, ORC_FN_SIGN
};

/* avx2::wise::{square, sqrt, ..., sign} (Engine/AVX2/wise.cpp:56-143) through
 * kernels::Unary with the scalar operators of Operations/kernel_ops.hpp:58-210:
 * square x*x (:65), sqrt (:87), rsqrt 1/sqrt(x) (:98), log (:109), exp (:120),
 * erf (:131), sin (:142), cos (:153), abs (:164), neg (:175), rcp 1/x (:186),
 * inverse 1/x (:208).  sign follows avx2::sign (functions.hpp:342-355): 1 where
 * x > 0, -1 where x < 0 (ordered compares), else +0; the scalar tail's
 * tlx::sign is parity unpinned (TLX absent).  Deviations: the SIMD body of
 * rcp and rsqrt uses the 12-bit _mm256_rcp_ps / _mm256_rsqrt_ps
 * (functions.hpp:168-170, 240-242); the oracle uses the exact expressions of
 * the scalar operators (the CUDA path's __frcp_rn is also exact).  log, exp,
 * erf, sin and cos call glibc (the reference calls SVML, absent here). */
static inline float wise_fn(int fn, float x) {
    switch (fn) {
        case ORC_FN_SQUARE: return x * x;
        case ORC_FN_SQRT: return sqrtf(x);
        case ORC_FN_RSQRT: return 1.0f / sqrtf(x);
        case ORC_FN_LOG: return logf(x);
        case ORC_FN_EXP: return expf(x);
        case ORC_FN_ERF: return erff(x);
        case ORC_FN_SIN: return sinf(x);
        case ORC_FN_COS: return cosf(x);
        case ORC_FN_ABS: return fabsf(x);
        case ORC_FN_NEG: return -x;
        case ORC_FN_RCP:
        case ORC_FN_INVERSE: return 1.0f / x;
        default: return x > 0.0f ? 1.0f : (x < 0.0f ? -1.0f : 0.0f);
    }
}

void orc_wise(const float *x, float *z, size_t n, int fn) {
    for (size_t i = 0; i < n; ++i) z[i] = wise_fn(fn, x[i]);
}

/* avx2::wise::lerp (Engine/AVX2/wise.cpp:145-155): fma::add(t, sub(b, a), a)
 * (functions.hpp:271-274) with a = x, b = value1, t = value2: one rounding
 * for v1 - x, one for the fused multiply-add. */
void orc_lerp(const float *x, float v1, float v2, float *z, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        const float d = v1 - x[i];
        z[i] = fmaf(v2, d, x[i]);
    }
}

/* avx2::wise::clamp (Engine/AVX2/wise.cpp:157-167): min(max(x, lo), hi) with
 * _mm256_max_ps / _mm256_min_ps (functions.hpp:332-335); a NaN x gives lo.
 * The scalar tail's std::clamp (NaN stays NaN) is not followed. */
void orc_clamp(const float *x, float lo, float hi, float *z, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        const float m = simd_max(x[i], lo);
        z[i] = m < hi ? m : hi;
    }
}

/* avx2::wise::gather (Engine/AVX2/wise.cpp:169-194): z[i] = x[idx[i]].  The
 * reference reads out of bounds for a bad index; here such an index gives
 * NaN (f32) or INT32_MIN (i32). */
void orc_gather_f32(const float *x, size_t xn, const int32_t *idx, float *z, size_t n) {
    for (size_t i = 0; i < n; ++i)
        z[i] = (idx[i] >= 0 && (size_t)idx[i] < xn) ? x[idx[i]] : NAN;
}

void orc_gather_i32(const int32_t *x, size_t xn, const int32_t *idx, int32_t *z, size_t n) {
    for (size_t i = 0; i < n; ++i)
        z[i] = (idx[i] >= 0 && (size_t)idx[i] < xn) ? x[idx[i]] : INT32_MIN;
}

/* ------------------------------------------------------ 16-bit conversions */

enum { ORC_DT_F32 = 0, ORC_DT_BF16 = 1, ORC_DT_F16 = 2 };

/* convert(float*, const bfloat16*) (Tools/cast.cpp:7-23): bits << 16. */
static inline float bf16_to_f32(uint16_t h) {
    const uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* convert(bfloat16*, const float*) (cast.cpp:55-78): u + 0x7FFF + lsb, >> 16
 * (round to nearest-even).  Deliberate deviation: NaN stays a quiet NaN
 * (the formula turns NaNs with a small payload into infinity). */
static inline uint16_t f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* convert(float*, const half*) / convert(half*, const float*) (cast.cpp:25-41,
 * 80-90): _mm256_cvtph_ps / _mm256_cvtps_ph(_MM_FROUND_TO_NEAREST_INT), here
 * their scalar F16C forms. */
static inline float f16_to_f32(uint16_t h) { return _cvtsh_ss(h); }
static inline uint16_t f32_to_f16(float f) { return (uint16_t)_cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT); }

void orc_convert(void *dst, int ddt, const void *src, int sdt, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        float v;
        if (sdt == ORC_DT_F32) v = ((const float *)src)[i];
        else if (sdt == ORC_DT_BF16) v = bf16_to_f32(((const uint16_t *)src)[i]);
        else v = f16_to_f32(((const uint16_t *)src)[i]);
        if (ddt == ORC_DT_F32) ((float *)dst)[i] = v;
        else if (ddt == ORC_DT_BF16) ((uint16_t *)dst)[i] = f32_to_bf16(v);
        else ((uint16_t *)dst)[i] = f32_to_f16(v);
    }
}

/* ----------------------------------------------------------- activations */

enum { ORC_ACT_NONE = 0, ORC_ACT_RELU = 1, ORC_ACT_SIGMOID = 2, ORC_ACT_TANH = 3, ORC_ACT_EXP = 4 };

/* relu = max(0, x) = (0 > x) ? 0 : x  (Engine/AVX2/functions.hpp:372-374).
 * sigmoid = 1 / (1 + exp(-x))         (functions.hpp:405-411).
 * tanh                                (functions.hpp:381-383). */
static inline float act_fwd(int act, float t) {
    switch (act) {
        case ORC_ACT_RELU: return 0.0f > t ? 0.0f : t;
        case ORC_ACT_SIGMOID: {
            const float e = expf(-t);
            const float d = 1.0f + e;
            return 1.0f / d;
        }
        case ORC_ACT_TANH: return tanhf(t);
        case ORC_ACT_EXP: return expf(t);
        default: return t;
    }
}

void orc_unary(const float *x, float *z, size_t n, int act) {
    for (size_t i = 0; i < n; ++i) z[i] = act_fwd(act, x[i]);
}

/* Derivative factor from the saved output y, as a separate rounded value:
 * relu' = (y > 0) ? 1 : 0, sigmoid' = y * (1 - y), tanh' = 1 - y*y. */
static inline float act_grad(int act, float y) {
    switch (act) {
        case ORC_ACT_RELU: return y > 0.0f ? 1.0f : 0.0f;
        case ORC_ACT_SIGMOID: {
            const float t = 1.0f - y;
            return y * t;
        }
        case ORC_ACT_TANH: {
            const float t = y * y;
            return 1.0f - t;
        }
        default: return 1.0f;
    }
}

/* dx = dy * act'(y): the backward of relu/sigmoid/tanh from the saved
 * output, as a concrete GradientFlow would run it (matrix_t::mul(dY, G),
 * matrix.cpp:35-43, with G = act_grad(Y)). */
void orc_act_bwd(const float *y, const float *dy, float *dx, size_t n, int act) {
    for (size_t i = 0; i < n; ++i) dx[i] = dy[i] * act_grad(act, y[i]);
}

/* Affine + activation forward: T = row::mul(X, scale) (broadcast.cpp:206-216),
 * row::add(T, bias) in place (broadcast.cpp:230-240), Y = act(T). */
void orc_affine_act_fwd(const float *x, const float *scale, const float *bias, float *y,
                        size_t m, size_t n, int act) {
    for (size_t i = 0; i < m; ++i)
        for (size_t j = 0; j < n; ++j) {
            float t = x[i * n + j] * scale[j];
            t = t + bias[j];
            y[i * n + j] = act_fwd(act, t);
        }
}

/* Affine + activation backward, from dY, the saved output Y and input X:
 *   G  = act'(Y)                        (elementwise, as act_grad)
 *   dZ = matrix_t::mul(dY, G)           (matrix.cpp:35-43)
 *   dX = row::mul(dZ, scale)            (broadcast.cpp:206-216)
 *   dscale = reduce::sum axis 0 of matrix_t::mul(dZ, X)   (reduce.cpp:39-62)
 *   dbias  = reduce::sum axis 0 of dZ
 * The axis-0 sums accumulate rows in order 0..m-1. */
void orc_affine_act_bwd(const float *x, const float *scale, const float *y, const float *dy,
                        float *dx, float *dscale, float *dbias, size_t m, size_t n, int act) {
    for (size_t i = 0; i < m; ++i) {
        for (size_t j = 0; j < n; ++j) {
            const size_t k = i * n + j;
            const float g = act_grad(act, y[k]);
            const float dz = dy[k] * g;
            dx[k] = dz * scale[j];
            const float p = dz * x[k];
            if (i == 0) {
                dscale[j] = p;
                dbias[j] = dz;
            } else {
                dscale[j] = dscale[j] + p;
                dbias[j] = dbias[j] + dz;
            }
        }
    }
}

/* ---------------------------------------------------------------- softmax */

/* Row softmax / log-softmax forward, composed per row of:
 *   m = reduce::max flat (reduce.cpp:204-215)
 *   Z = Broadcast::col::sub(X, m) (broadcast.cpp:292-304)
 *   E = exp(Z)
 *   s = reduce::sum flat (reduce.cpp:17-28) of E
 *   softmax:     Y = Broadcast::col::div(E, s) (broadcast.cpp:320-332)
 *   log-softmax: Y = Broadcast::col::sub(Z, log(s)) */
void orc_softmax_fwd(const float *x, float *y, size_t rows, size_t cols, int log_mode) {
    float *e = (float *)malloc(cols * sizeof(float));
    float *zr = (float *)malloc(cols * sizeof(float));
    for (size_t r = 0; r < rows; ++r) {
        const float *xr = x + r * cols;
        float *yr = y + r * cols;
        float m, s;
        orc_reduce_max_flat(xr, &m, cols);
        for (size_t j = 0; j < cols; ++j) zr[j] = xr[j] - m;
        for (size_t j = 0; j < cols; ++j) e[j] = expf(zr[j]);
        orc_reduce_sum_flat(e, &s, cols);
        if (log_mode) {
            const float ls = logf(s);
            for (size_t j = 0; j < cols; ++j) yr[j] = zr[j] - ls;
        } else {
            for (size_t j = 0; j < cols; ++j) yr[j] = e[j] / s;
        }
    }
    free(e);
    free(zr);
}

/* Row softmax backward from the saved output:
 *   softmax:     r = reduce::sum flat of matrix_t::mul(dY, Y);
 *                dX = matrix_t::mul(Y, Broadcast::col::sub(dY, r))
 *   log-softmax: r = reduce::sum flat of dY;
 *                dX = matrix_t::sub(dY, Broadcast::col::mul(exp(Y), r)) */
void orc_softmax_bwd(const float *y, const float *dy, float *dx, size_t rows, size_t cols,
                     int log_mode) {
    float *t = (float *)malloc(cols * sizeof(float));
    for (size_t r = 0; r < rows; ++r) {
        const float *yr = y + r * cols;
        const float *gr = dy + r * cols;
        float *dr = dx + r * cols;
        float s;
        if (log_mode) {
            orc_reduce_sum_flat(gr, &s, cols);
            for (size_t j = 0; j < cols; ++j) {
                const float p = expf(yr[j]);
                const float q = p * s;
                dr[j] = gr[j] - q;
            }
        } else {
            for (size_t j = 0; j < cols; ++j) t[j] = gr[j] * yr[j];
            orc_reduce_sum_flat(t, &s, cols);
            for (size_t j = 0; j < cols; ++j) {
                const float u = gr[j] - s;
                dr[j] = yr[j] * u;
            }
        }
    }
    free(t);
}

/* ----------------------------------------------------------------- matmul */

/* matrix_t::matmul (Engine/AVX2/matrix.cpp:75-147), row-major
 * C[m,n] = A[m,k] * B[k,n].  Per output element the reference accumulates
 * each K panel of 256 as an fma chain starting from zero, then adds the
 * panel result into C (C starts at zero).  The NC/MC cache blocking does not
 * change that per-element order, so it is not restated. */
void orc_matmul(const float *a, const float *b, float *c, size_t m, size_t k, size_t n) {
    const size_t KC = 256;
    float *acc = (float *)malloc(n * sizeof(float));
    for (size_t i = 0; i < m; ++i) {
        float *ci = c + i * n;
        for (size_t j = 0; j < n; ++j) ci[j] = 0.0f;
        for (size_t kc = 0; kc < k; kc += KC) {
            const size_t kend = kc + KC < k ? kc + KC : k;
            for (size_t j = 0; j < n; ++j) acc[j] = 0.0f;
            for (size_t kk = kc; kk < kend; ++kk) {
                const float av = a[i * k + kk];
                const float *bk = b + kk * n;
                for (size_t j = 0; j < n; ++j) acc[j] = fmaf(av, bk[j], acc[j]);
            }
            for (size_t j = 0; j < n; ++j) ci[j] = ci[j] + acc[j];
        }
    }
    free(acc);
}

/* Transposed copy used to express A^T*B and A*B^T with the reference matmul,
 * which has no transposed variants. */
static float *transpose_copy(const float *a, size_t rows, size_t cols) {
    float *t = (float *)malloc(rows * cols * sizeof(float));
    for (size_t i = 0; i < rows; ++i)
        for (size_t j = 0; j < cols; ++j) t[j * rows + i] = a[i * cols + j];
    return t;
}

/* GEMM with optional transposes, through orc_matmul:
 * C[m,n] = op(A)[m,k] * op(B)[k,n]; op = transpose when the flag is set.
 * A is stored [m,k] (or [k,m] when trans_a); B is [k,n] (or [n,k]). */
void orc_gemm(const float *a, const float *b, float *c, size_t m, size_t k, size_t n,
              int trans_a, int trans_b) {
    float *at = trans_a ? transpose_copy(a, k, m) : NULL;
    float *bt = trans_b ? transpose_copy(b, n, k) : NULL;
    orc_matmul(at ? at : a, bt ? bt : b, c, m, k, n);
    free(at);
    free(bt);
}

/* ------------------------------------------------------------ MLP pieces */

/* Softmax cross-entropy on logits [b, c] with int32 labels:
 *   Yl = log-softmax(logits) (orc_softmax_fwd, log mode)
 *   loss = reduce::mean flat over rows of -Yl[r, label[r]]   (reduce.cpp:66-69)
 *   dlogits = (softmax - onehot) * (1/b)  (col::div composition, then ScalarOp::mul) */
void orc_softmax_xent(const float *logits, const int32_t *labels, float *loss, float *dlogits,
                      size_t b, size_t c) {
    float *yl = (float *)malloc(b * c * sizeof(float));
    float *nl = (float *)malloc(b * sizeof(float));
    orc_softmax_fwd(logits, yl, b, c, 1);
    orc_softmax_fwd(logits, dlogits, b, c, 0);
    const float inv_b = 1.0f / (float)b;
    for (size_t r = 0; r < b; ++r) {
        const int32_t lab = labels[r];
        nl[r] = -yl[r * c + lab];
        dlogits[r * c + lab] = dlogits[r * c + lab] - 1.0f;
        for (size_t j = 0; j < c; ++j) dlogits[r * c + j] = dlogits[r * c + j] * inv_b;
    }
    orc_reduce_mean_flat(nl, loss, b);
    free(yl);
    free(nl);
}

/* SGD: W = matrix_t::sub(W, ScalarOp::mul(G, lr))  (matrix.cpp:159-167,
 * scalar.cpp:97-99): two roundings, no fma. */
void orc_sgd(float *w, const float *g, float lr, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        const float t = g[i] * lr;
        w[i] = w[i] - t;
    }
}

/* One training step of the 3-layer ReLU MLP used by the C5 workload:
 *   h1 = relu(X W1 + b1), h2 = relu(h1 W2 + b2), logits = h2 W3 + b3,
 *   loss = softmax cross-entropy, then backward and SGD on all six tensors.
 * Bias add is Broadcast::row::add; relu is functions.hpp:372-374; the relu
 * backward multiplies by the 0/1 mask (y > 0).  Column sums for the bias
 * gradients are reduce::sum over axis 0 (reduce.cpp:39-62).
 * Shapes: x [b, d0], w1 [d0, d1], w2 [d1, d2], w3 [d2, d3]. */
void orc_mlp_step(const float *x, const int32_t *labels, float *w1, float *b1, float *w2,
                  float *b2, float *w3, float *b3, size_t b, size_t d0, size_t d1, size_t d2,
                  size_t d3, float lr, float *loss_out) {
    float *z1 = (float *)malloc(b * d1 * sizeof(float));
    float *h1 = (float *)malloc(b * d1 * sizeof(float));
    float *z2 = (float *)malloc(b * d2 * sizeof(float));
    float *h2 = (float *)malloc(b * d2 * sizeof(float));
    float *lg = (float *)malloc(b * d3 * sizeof(float));
    float *dl = (float *)malloc(b * d3 * sizeof(float));
    float *dh2 = (float *)malloc(b * d2 * sizeof(float));
    float *dh1 = (float *)malloc(b * d1 * sizeof(float));
    float *gw1 = (float *)malloc(d0 * d1 * sizeof(float));
    float *gw2 = (float *)malloc(d1 * d2 * sizeof(float));
    float *gw3 = (float *)malloc(d2 * d3 * sizeof(float));
    float *gb1 = (float *)malloc(d1 * sizeof(float));
    float *gb2 = (float *)malloc(d2 * sizeof(float));
    float *gb3 = (float *)malloc(d3 * sizeof(float));

    orc_matmul(x, w1, z1, b, d0, d1);
    orc_bcast_row(z1, b1, z1, b, d1, ORC_ADD);
    orc_unary(z1, h1, b * d1, ORC_ACT_RELU);
    orc_matmul(h1, w2, z2, b, d1, d2);
    orc_bcast_row(z2, b2, z2, b, d2, ORC_ADD);
    orc_unary(z2, h2, b * d2, ORC_ACT_RELU);
    orc_matmul(h2, w3, lg, b, d2, d3);
    orc_bcast_row(lg, b3, lg, b, d3, ORC_ADD);

    orc_softmax_xent(lg, labels, loss_out, dl, b, d3);

    /* layer 3 */
    orc_gemm(h2, dl, gw3, d2, b, d3, 1, 0);
    orc_reduce_sum(dl, gb3, 1, b, d3);
    orc_gemm(dl, w3, dh2, b, d3, d2, 0, 1);
    for (size_t i = 0; i < b * d2; ++i) dh2[i] = dh2[i] * act_grad(ORC_ACT_RELU, h2[i]);
    /* layer 2 */
    orc_gemm(h1, dh2, gw2, d1, b, d2, 1, 0);
    orc_reduce_sum(dh2, gb2, 1, b, d2);
    orc_gemm(dh2, w2, dh1, b, d2, d1, 0, 1);
    for (size_t i = 0; i < b * d1; ++i) dh1[i] = dh1[i] * act_grad(ORC_ACT_RELU, h1[i]);
    /* layer 1 */
    orc_gemm(x, dh1, gw1, d0, b, d1, 1, 0);
    orc_reduce_sum(dh1, gb1, 1, b, d1);

    orc_sgd(w1, gw1, lr, d0 * d1);
    orc_sgd(b1, gb1, lr, d1);
    orc_sgd(w2, gw2, lr, d1 * d2);
    orc_sgd(b2, gb2, lr, d2);
    orc_sgd(w3, gw3, lr, d2 * d3);
    orc_sgd(b3, gb3, lr, d3);

    free(z1); free(h1); free(z2); free(h2); free(lg); free(dl); free(dh2); free(dh1);
    free(gw1); free(gw2); free(gw3); free(gb1); free(gb2); free(gb3);
}
